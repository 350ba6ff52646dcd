// Library set-up, status words, trellis dequantisation, the router's top-8 and the shared expert's SwiGLU.
#include <hip/hip_runtime.h>

#include <mutex>
#include <vector>

#include "ea_device.hpp"
#include "ea_gemm.hpp"
#include "ea_host.hpp"

namespace ea {

namespace {
std::mutex g_mu;
std::vector<DevCtx> g_ctx;
}  // namespace

DevCtx* ctx() {
    int dev = -1;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0) return nullptr;
    std::lock_guard<std::mutex> lk(g_mu);
    if ((size_t)dev >= g_ctx.size()) return nullptr;
    return &g_ctx[dev];
}

// ---- dequantisation -------------------------------------------------------------------------------------------
// A wave a tile, through the same lane decoder the GEMM kernels feed to MFMA (TileLane): lane l decodes the four
// values of column l & 15 at rows 2g, 2g + 1, 2g + 8, 2g + 9 (g = l >> 4), so the bit-exact dequant tests pin
// exactly the values the matrix products consume.
template <int CB, int K2>
__device__ __forceinline__ void unpack_tile(const uint32_t* __restrict__ tile, uint16_t* __restrict__ W, int N, int kt,
                                            int nt, int lane) {
    const TileLane<K2, CB> tl(lane);
    const u2v v = tl.decode_at(tile);
    const int n = nt * 16 + (lane & 15), g = (lane >> 4) & 3;
    uint16_t* w = W + (size_t)(kt * 16 + 2 * g) * N + n;
    w[0] = (uint16_t)(v.x & 0xffffu);
    w[N] = (uint16_t)(v.x >> 16);
    w[8 * (size_t)N] = (uint16_t)(v.y & 0xffffu);
    w[9 * (size_t)N] = (uint16_t)(v.y >> 16);
}

template <int CB>
__global__ void __launch_bounds__(256) unpack_kernel(const uint32_t* __restrict__ T, uint16_t* __restrict__ W, int N,
                                                     int k2, int64_t stride_k, int64_t stride_nb) {
    const int nt = blockIdx.x * 4 + (threadIdx.x >> 6), kt = blockIdx.y, lane = threadIdx.x & 63;
    if (nt * 16 >= N) return;
    const uint32_t* tile = T + kt * stride_k + (nt >> 3) * stride_nb + (nt & 7) * 4 * k2;
    const bool ok = EA_K2_SWITCH(k2, 2, 16, (unpack_tile<CB, K2V>(tile, W, N, kt, nt, lane)));
    (void)ok;
}

// ---- router top-8 ----------------------------------------------------------------------------------------------
// One block a row, a thread an expert (E = 256). Eight rounds of a block arg-max over the ranking key of choice =
// sigmoid + bias (order_key: NaN below every number), the lower id winning ties; the winner's key becomes 0, below
// every choice (native_ops.cu:1015-1068).
__global__ void __launch_bounds__(256) topk8_kernel(const float* __restrict__ logits, const float* __restrict__ bias,
                                                    int32_t* __restrict__ pick, float* __restrict__ wts, float scale,
                                                    uint8_t* __restrict__ log) {
    __shared__ uint32_t s_key[4];
    __shared__ int s_idx[4];
    __shared__ float s_wts[8];
    __shared__ int s_pick[8];
    const int r = blockIdx.x, t = threadIdx.x, lane = t & 63, wave = t >> 6;
    const float score = 1.0f / (expf_path(0.0f - logits[(size_t)r * 256 + t]) + 1.0f);
    uint32_t key = order_key(score + bias[t]);
    for (int k = 0; k < 8; ++k) {
        uint32_t v = key;
        int i = t;
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) {
            const uint32_t ov = (uint32_t)__shfl_xor((int)v, o, 64);
            const int oi = __shfl_xor(i, o, 64);
            if (ov > v || (ov == v && oi < i)) {
                v = ov;
                i = oi;
            }
        }
        if (lane == 0) {
            s_key[wave] = v;
            s_idx[wave] = i;
        }
        __syncthreads();
        uint32_t bv = s_key[0];
        int bi = s_idx[0];
#pragma unroll
        for (int w = 1; w < 4; ++w)
            if (s_key[w] > bv || (s_key[w] == bv && s_idx[w] < bi)) {
                bv = s_key[w];
                bi = s_idx[w];
            }
        __syncthreads();  // every thread has read the winners before the next round writes them
        if (t == bi) {
            s_pick[k] = bi;
            s_wts[k] = score;
            key = 0u;
        }
    }
    __syncthreads();
    if (t < 8) {
        float total = 0.0f;
        for (int k = 0; k < 8; ++k) total = total + s_wts[k];
        pick[(size_t)r * 8 + t] = s_pick[t];
        wts[(size_t)r * 8 + t] = s_wts[t] / (total + 1e-20f) * scale;
        if (log) log[(size_t)r * 8 + t] = (uint8_t)s_pick[t];
    }
}

// ---- SwiGLU of the shared expert ------------------------------------------------------------------------------
__global__ void __launch_bounds__(256) swiglu2_kernel(const uint16_t* __restrict__ g, const uint16_t* __restrict__ u,
                                                      uint16_t* __restrict__ out, size_t n) {
    for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (size_t)gridDim.x * 256) {
        const float gv = bf2f(g[i]);
        const float s = bf16r(gv / (expf_path(0.0f - gv) + 1.0f));
        out[i] = f2bf(s * bf2f(u[i]));
    }
}

__global__ void __launch_bounds__(256) add_f32_kernel(float* __restrict__ a, const float* __restrict__ b, size_t n) {
    for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (size_t)gridDim.x * 256) a[i] = a[i] + b[i];
}

}  // namespace ea

using namespace ea;

extern "C" {

const char* ea_strerror(int s) {
    switch (s) {
        case EA_OK: return "ok";
        case EA_BAD_ROT_IN: return "BadRotIn: rot_in needs 1 to 3 jobs and K a multiple of 128";
        case EA_UNPORTED_LINEAR_WALK: return "UnportedLinearWalk: only loads with bits 1 and 2 set are built";
        case EA_UNEVEN_K_SPLIT: return "UnevenKSplit: K / 16 must split evenly over SK * WK";
        case EA_UNPORTED_LINEAR_VARIANT: return "UnportedLinearVariant: no linear kernel for this width / codebook / warps";
        case EA_TOO_MANY_EXPERTS: return "TooManyExperts: at most 4096 experts";
        case EA_TOO_MANY_SLOTS: return "TooManySlots: at most 32 slots a row";
        case EA_GROUP_SHARED_MEMORY: return "GroupSharedMemory: the picks do not fit in shared memory";
        case EA_UNEVEN_SPLIT: return "UnevenSplit: K and N must split evenly over the tile setting";
        case EA_BAD_ROW_STRIDE: return "BadRowStride: the trellis row stride is below N / 16";
        case EA_UNPORTED_GROUPED_VARIANT: return "UnportedGroupedVariant: no grouped kernel for this tile setting";
        case EA_BAD_WIDTH: return "BadWidth: the width must be a multiple of 128";
        case EA_SCRATCH_TOO_SMALL: return "ScratchTooSmall: more rows than the scratch holds";
        case EA_INVALID: return "Invalid: conflicting options";
        case EA_NOT_GROUPABLE: return "NotGroupable: 1 to 3 layers of one K, width, codebook and warps, 1 to 128 rows";
        case EA_HIP_FAILED: return "HIP call failed";
        case EA_OUT_OF_DEVICE_MEMORY: return "out of device memory";
        case EA_NOT_INITIALIZED: return "ea_init was not called on this device";
        case EA_BAD_ARGUMENT: return "bad argument";
        case EA_UNSUPPORTED_WIDTH: return "an expert width (K2) or codebook this build has no decoder for";
        case EA_SYNC_TIMEOUT: return "a kernel's bounded wait on its block's LDS counters gave up";
        case EA_BANK_IO: return "a bank or checkpoint file could not be opened or mapped";
        case EA_BAD_SAFETENSORS: return "BadSafetensors: a safetensors header breaks the format";
        case EA_BAD_INDEX: return "BadIndex: model.safetensors.index.json has no weight_map of file names";
        case EA_MISSING_TENSOR: return "MissingTensor: the checkpoint does not hold this tensor (or a stored rank of it)";
        case EA_NO_SPLIT_RULE: return "NoSplitRule: no tensor-parallel split rule for this tensor name";
        case EA_STRADDLES_HADAMARD: return "StraddlesHadamard: a rank's share would cut a 128-value Hadamard block";
        case EA_STORED_WORLD_NOT_MULTIPLE: return "StoredWorldNotMultiple: stored ranks must be a multiple of the ranks";
        case EA_TOO_MANY_STORED_RANKS: return "TooManyStoredRanks: at most 16 stored ranks joined into one share";
        case EA_STORED_SHARES_DIFFER: return "StoredSharesDiffer: the stored ranks of one tensor differ in dtype or shape";
        case EA_BAD_TRELLIS: return "BadTrellis: a trellis must be i16 [K/16, N/16, 8 K2] of the layer's shape";
        case EA_PACKED_SCALES: return "PackedScalesUnsupported: suh / svh must be fp16 of the layer's shape";
        case EA_MIXED_CODEBOOKS: return "MixedCodebooks: an expert's codebook differs from expert 0's";
        case EA_SWAP_CODEBOOK_DIFFERS: return "SwapCodebookDiffers: the bank's codebook differs from the layer's";
        case EA_SWAP_BAD_TRELLIS: return "SwapBadTrellis: the bank's trellis is not of the layer's shape and width";
        case EA_SWAP_BAD_SCALES: return "SwapBadScales: the bank's scales are not of the layer's shape";
        case EA_SWAP_WIDTH_UNSUPPORTED: return "SwapWidthUnsupported: the kernels take widths of 2 to 5 bits";
        case EA_SWAP_NO_BANK: return "SwapNoBank: no bank for a width the change asks for";
        case EA_OUT_OF_HOST_MEMORY: return "a host allocation of the bank reader failed";
        default: return "unknown status";
    }
}

int ea_init(int device) {
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess || device < 0 || device >= n) return EA_BAD_ARGUMENT;
    int r = hip_status(hipSetDevice(device));
    if (r) return r;
    std::lock_guard<std::mutex> lk(g_mu);
    if ((size_t)device >= g_ctx.size()) g_ctx.resize(device + 1);
    DevCtx& c = g_ctx[device];
    if (c.ready) return EA_OK;
    hipDeviceProp_t p;
    r = hip_status(hipGetDeviceProperties(&p, device));
    if (r) return r;
    c.device = device;
    c.cus = p.multiProcessorCount;
    c.lds_optin = p.sharedMemPerBlock;
    r = hip_status(hipMalloc(&c.status, 256));
    if (r) return r;
    r = hip_status(hipMemset(c.status, 0, 256));
    if (r) return r;
    r = hip_status(hipStreamCreateWithFlags(&c.side, hipStreamNonBlocking));
    if (r) return r;
    r = hip_status(hipEventCreateWithFlags(&c.fork, hipEventDisableTiming));
    if (r) return r;
    r = hip_status(hipEventCreateWithFlags(&c.join, hipEventDisableTiming));
    if (r) return r;
    r = dl_static_setup(c);
    if (r) return r;
    r = hip_status(hipDeviceSynchronize());
    if (r) return r;
    c.ready = true;
    return EA_OK;
}

int ea_fini(void) {
    std::lock_guard<std::mutex> lk(g_mu);
    for (auto& c : g_ctx)
        if (c.ready) {
            (void)hipSetDevice(c.device);
            (void)hipFree(c.status);
            c.status = nullptr;
            if (c.side) (void)hipStreamDestroy(c.side);
            if (c.fork) (void)hipEventDestroy(c.fork);
            if (c.join) (void)hipEventDestroy(c.join);
            c.side = nullptr;
            c.fork = c.join = nullptr;
            c.static_scratch = nullptr;  // the array itself lives until the process ends
            c.ready = false;
        }
    return EA_OK;
}

}  // extern "C"

namespace ea {
static std::mutex g_fork_mu;
int fork_join(hipStream_t s, const std::function<int(hipStream_t)>& side_work,
              const std::function<int(hipStream_t)>& main_work) {
    DevCtx* c = ctx();
    if (!c || !c->ready) return EA_NOT_INITIALIZED;
    std::lock_guard<std::mutex> lk(g_fork_mu);
    int r = hip_status(hipEventRecord(c->fork, s));
    if (r) return r;
    r = hip_status(hipStreamWaitEvent(c->side, c->fork, 0));
    if (r) return r;
    r = side_work(c->side);
    const int r2 = main_work(s);  // always issued, so s never waits on a join that is not recorded
    const int r3 = hip_status(hipEventRecord(c->join, c->side));
    const int r4 = r3 ? r3 : hip_status(hipStreamWaitEvent(s, c->join, 0));
    return r ? r : r2 ? r2 : r4;
}
}  // namespace ea

extern "C" {

int ea_device_status(int* code) {
    EA_REQUIRE_CTX(c);
    if (!code) return EA_BAD_ARGUMENT;
    int r = hip_status(hipMemcpy(code, c->status, sizeof(int), hipMemcpyDeviceToHost));
    if (r) return r;
    return hip_status(hipMemset(c->status, 0, sizeof(int)));
}

int ea_device_status_address(void** addr) {
    EA_REQUIRE_CTX(c);
    if (!addr) return EA_BAD_ARGUMENT;
    *addr = c->status;
    return EA_OK;
}

static int unpack_launch(ea_stream_t stream, const void* t, void* w, uint32_t kdim, uint32_t n, uint32_t k2,
                         uint32_t cb, int64_t stride_k, int64_t stride_nb) {
    EA_REQUIRE_CTX(c);
    if (!t || !w || kdim % 16 || n % 16 || kdim == 0 || n == 0) return EA_BAD_ARGUMENT;
    if (k2 < 2 || k2 > 16 || cb > 2) return EA_UNSUPPORTED_WIDTH;
    dim3 grid((n / 16 + 3) / 4, kdim / 16);
    auto T = static_cast<const uint32_t*>(t);
    auto W = static_cast<uint16_t*>(w);
    hipStream_t s = as_stream(stream);
    if (cb == 0) unpack_kernel<0><<<grid, 256, 0, s>>>(T, W, (int)n, (int)k2, stride_k, stride_nb);
    else if (cb == 1) unpack_kernel<1><<<grid, 256, 0, s>>>(T, W, (int)n, (int)k2, stride_k, stride_nb);
    else unpack_kernel<2><<<grid, 256, 0, s>>>(T, W, (int)n, (int)k2, stride_k, stride_nb);
    return launched();
}

// The expert layout is the strided one with stride_k = (N / 16) * TW and stride_nb = 8 * TW.
int ea_dequant(ea_stream_t stream, const void* trellis, void* w, uint32_t K, uint32_t N, uint32_t k2, uint32_t cb) {
    const int64_t tw = 4 * (int64_t)k2;
    return unpack_launch(stream, trellis, w, K, N, k2, cb, (int64_t)(N / 16) * tw, 8 * tw);
}

int ea_exl3_unpack(ea_stream_t stream, const void* t, void* w, uint32_t kdim, uint32_t n, uint32_t k2, uint32_t cb,
                   int64_t stride_k, int64_t stride_nb) {
    // every K2 in 2..16 and every codebook (the reference builds four of these pairs, exl3.zig:40)
    if (k2 < 2 || k2 > 16 || cb > 2) return EA_UNPORTED_LINEAR_VARIANT;
    return unpack_launch(stream, t, w, kdim, n, k2, cb, stride_k, stride_nb);
}

int ea_topk8(ea_stream_t stream, const float* logits, const float* bias, int32_t* pick, float* wts, uint32_t rows,
             float scale, uint8_t* log) {
    EA_REQUIRE_CTX(c);
    if (!logits || !bias || !pick || !wts) return EA_BAD_ARGUMENT;
    if (rows == 0) return EA_OK;
    topk8_kernel<<<rows, 256, 0, as_stream(stream)>>>(logits, bias, pick, wts, scale, log);
    return launched();
}

int ea_swiglu2(ea_stream_t stream, const void* g, const void* u, void* out, uint32_t rows, uint32_t width) {
    EA_REQUIRE_CTX(c);
    if (!g || !u || !out) return EA_BAD_ARGUMENT;
    const size_t n = (size_t)rows * width;
    if (n == 0) return EA_OK;
    size_t blocks = (n + 255) / 256;
    if (blocks > (size_t)c->cus * 16) blocks = (size_t)c->cus * 16;
    swiglu2_kernel<<<(unsigned)blocks, 256, 0, as_stream(stream)>>>(static_cast<const uint16_t*>(g),
                                                                   static_cast<const uint16_t*>(u),
                                                                   static_cast<uint16_t*>(out), n);
    return launched();
}

int ea_add_f32(ea_stream_t stream, float* a, const float* b, size_t n) {
    EA_REQUIRE_CTX(c);
    if (!a || !b) return EA_BAD_ARGUMENT;
    if (n == 0) return EA_OK;
    size_t blocks = (n + 255) / 256;
    if (blocks > (size_t)c->cus * 8) blocks = (size_t)c->cus * 8;
    add_f32_kernel<<<(unsigned)blocks, 256, 0, as_stream(stream)>>>(a, b, n);
    return launched();
}

}  // extern "C"
