// EXL3 linear for 1 to 128 rows (the shared expert and any strips-layout linear): input rotation for 1..3 jobs
// of one input, and one launch over 1..3 jobs with per-job K splits finished by the last-arriving block
// (exl3_linear.cu:69-484, exl3.zig, linear.zig). Rows are independent; sums run in a fixed order: waves of a
// block in order, then splits in order.
#include <hip/hip_runtime.h>

#include "ea_device.hpp"
#include "ea_gemm.hpp"
#include "ea_host.hpp"

namespace ea {

// xh_j [M, K] = fp16((x * suh_j) @ H * HAD_SCALE); block (group of four 128-blocks, row, job), a wave a block.
__global__ void __launch_bounds__(256) lin_rot_in_kernel(const void* __restrict__ x, int x_dtype, ea_rot_jobs jobs,
                                                         int K) {
    const int blk = blockIdx.x * 4 + (threadIdx.x >> 6), row = blockIdx.y, lane = threadIdx.x & 63;
    if (blk * 128 >= K) return;
    const uint16_t* suh = dptr<const uint16_t>(jobs.suh[blockIdx.z]);
    uint16_t* xh = dptr<uint16_t>(jobs.xh[blockIdx.z]);
    const int k = blk * 128 + 2 * lane;
    float v0 = load_act(x, x_dtype, (size_t)row * K + k) * h2f(suh[k]);
    float v1 = load_act(x, x_dtype, (size_t)row * K + k + 1) * h2f(suh[k + 1]);
    fwht128_w64(v0, v1, lane);
    *reinterpret_cast<uint32_t*>(xh + (size_t)row * K + k) =
        (uint32_t)f2h(v0 * HAD_SCALE) | ((uint32_t)f2h(v1 * HAD_SCALE) << 16);
}

// One row's 128 outputs of a column block from their fp32 sums (two a lane): FWHT, * HAD_SCALE * svh (+ bias),
// stored as y_dtype (exl3_linear.cu:69-81).
__device__ __forceinline__ void finish_store(float v0, float v1, int lane, const uint16_t* svh, const uint16_t* bias,
                                             void* y, int y_dtype, size_t at, int col) {
    fwht128_w64(v0, v1, lane);
    v0 = v0 * HAD_SCALE * h2f(svh[col]);
    v1 = v1 * HAD_SCALE * h2f(svh[col + 1]);
    if (bias) {
        v0 += h2f(bias[col]);
        v1 += h2f(bias[col + 1]);
    }
    store_act(y, y_dtype, at, v0);
    store_act(y, y_dtype, at + 1, v1);
}

__device__ __forceinline__ float load_coherent(const float* p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Block (job, column block nb of 128, split): WK waves each take per_warp consecutive k tiles of the split; rows in
// passes of 16. SK == 1: the block finishes its columns. SK > 1: partial sums to Z[split], and the block that
// arrives last on the (pass, nb) counter sums the splits in order, finishes, and resets the counter to zero.
template <int CB, int K2, int WK>
__global__ void __launch_bounds__(WK * 64) linear_kernel(ea_jobs jobs, int M, int K) {
    int ji = 0;
#pragma unroll
    for (int q = 1; q < EA_MAX_JOBS; ++q)
        if (q < jobs.n && (int)blockIdx.x >= jobs.j[q].start) ji = q;
    const ea_job& J = jobs.j[ji];
    const uint16_t* __restrict__ xh = dptr<const uint16_t>(J.xh);
    const uint32_t* __restrict__ T = dptr<const uint32_t>(J.T);
    const uint16_t* svh = dptr<const uint16_t>(J.svh);
    const uint16_t* bias = dptr<const uint16_t>(J.bias);
    void* y = dptr<void>(J.y);
    float* Z = dptr<float>(J.Z);
    int* counters = dptr<int>(J.counters);
    const int N = J.N, SK = J.SK, NB = N >> 7;
    const int local = (int)blockIdx.x - J.start, nb = local % NB, split = local / NB;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int per_warp = (K >> 4) / SK / WK;
    const int kt0 = split * (per_warp * WK) + wave * per_warp;
    const uint32_t* base = T + nb * J.stride_nb + (int64_t)kt0 * J.stride_k;
    const int col0 = nb * 128;

    __shared__ float red[WK][16][128];
    __shared__ int last;
    for (int m0 = 0, pass = 0; m0 < M; m0 += 16, ++pass) {
        const int R = min(16, M - m0);
        const int r = m0 + (lane & 15);
        const uint16_t* const xrow[1] = {r < M ? xh + (size_t)r * K : nullptr};
        f4v acc[1][8];
#pragma unroll
        for (int j = 0; j < 8; ++j) acc[0][j] = f4v{0.f, 0.f, 0.f, 0.f};
        wave_tiles<CB, K2, 8, 1>(base, (size_t)J.stride_k, per_warp, kt0 * 16, xrow, lane, acc);
        __syncthreads();  // red is free (the previous pass has read it)
#pragma unroll
        for (int j = 0; j < 8; ++j)
#pragma unroll
            for (int i = 0; i < 4; ++i) red[wave][4 * (lane >> 4) + i][j * 16 + (lane & 15)] = acc[0][j][i];
        __syncthreads();
        if (SK == 1) {
            for (int rr = wave; rr < R; rr += WK) {
                float v0 = red[0][rr][2 * lane], v1 = red[0][rr][2 * lane + 1];
#pragma unroll
                for (int w = 1; w < WK; ++w) {
                    v0 += red[w][rr][2 * lane];
                    v1 += red[w][rr][2 * lane + 1];
                }
                finish_store(v0, v1, lane, svh, bias, y, J.y_dtype, (size_t)(m0 + rr) * N + col0 + 2 * lane,
                             col0 + 2 * lane);
            }
        } else {
            for (int idx = threadIdx.x; idx < R * 128; idx += WK * 64) {
                const int rr = idx >> 7, c = idx & 127;
                float s = red[0][rr][c];
#pragma unroll
                for (int w = 1; w < WK; ++w) s += red[w][rr][c];
                Z[((size_t)split * M + m0 + rr) * N + col0 + c] = s;
            }
            __threadfence();
            __syncthreads();
            if (threadIdx.x == 0) last = atomicAdd(counters + pass * NB + nb, 1) == SK - 1;
            __syncthreads();
            if (last) {
                __threadfence();
                for (int rr = wave; rr < R; rr += WK) {
                    const size_t at = ((size_t)m0 + rr) * N + col0 + 2 * lane;
                    float v0 = load_coherent(Z + at), v1 = load_coherent(Z + at + 1);
                    for (int q = 1; q < SK; ++q) {
                        v0 += load_coherent(Z + (size_t)q * M * N + at);
                        v1 += load_coherent(Z + (size_t)q * M * N + at + 1);
                    }
                    finish_store(v0, v1, lane, svh, bias, y, J.y_dtype, at, col0 + 2 * lane);
                }
                if (threadIdx.x == 0) counters[pass * NB + nb] = 0;  // every split of the column block arrived
            }
        }
    }
}

// the (K2, codebook) pairs this build instantiates: the reference's four (exl3.zig:40) and 3 / 4 bits mcg
template <int CB, int K2>
static void launch_wk(const ea_jobs& jobs, int blocks, hipStream_t s, int M, int K, int wk) {
    if (wk == 2) linear_kernel<CB, K2, 2><<<blocks, 2 * 64, 0, s>>>(jobs, M, K);
    else if (wk == 4) linear_kernel<CB, K2, 4><<<blocks, 4 * 64, 0, s>>>(jobs, M, K);
    else linear_kernel<CB, K2, 8><<<blocks, 8 * 64, 0, s>>>(jobs, M, K);
}

static bool launch_variant(const ea_jobs& jobs, int blocks, hipStream_t s, int M, int K, uint32_t k2, uint32_t cb,
                           int wk) {
#define EA_LV(K2_, CB_)                                            \
    if (k2 == K2_ && cb == CB_) {                                  \
        launch_wk<CB_, K2_>(jobs, blocks, s, M, K, wk);            \
        return true;                                               \
    }
    EA_LV(10, 2) EA_LV(12, 2) EA_LV(8, 1) EA_LV(8, 2) EA_LV(6, 1) EA_LV(4, 1)
#undef EA_LV
    return false;
}

static bool variant_built(uint32_t k2, uint32_t cb, uint32_t wk) {
    if (wk != 2 && wk != 4 && wk != 8) return false;
    return (cb == 2 && (k2 == 10 || k2 == 12 || k2 == 8)) || (cb == 1 && (k2 == 8 || k2 == 6 || k2 == 4));
}

int launch_lin_rot_in(hipStream_t s, const void* x, int x_dtype, const ea_rot_jobs* jobs, uint32_t njobs, uint32_t m,
                      uint32_t kdim) {
    EA_REQUIRE_CTX(c);
    if (njobs == 0 || njobs > EA_MAX_JOBS || kdim % 128 != 0 || !jobs) return EA_BAD_ROT_IN;
    if (!x || x_dtype < 0 || x_dtype > 2) return EA_BAD_ARGUMENT;
    if (m == 0) return EA_OK;
    dim3 grid((kdim / 128 + 3) / 4, m, njobs);
    lin_rot_in_kernel<<<grid, 256, 0, s>>>(x, x_dtype, *jobs, (int)kdim);
    return launched();
}

int launch_linear(hipStream_t s, const ea_jobs* jobs_in, uint32_t m, uint32_t kdim, uint32_t k2, uint32_t cb,
                  uint32_t wk, uint32_t loads) {
    EA_REQUIRE_CTX(c);
    if (!jobs_in || jobs_in->n < 1 || jobs_in->n > EA_MAX_JOBS) return EA_BAD_ARGUMENT;
    // only the load walk with bits 1 and 2 set is built (exl3.zig:96-98)
    if (!(loads & 1) || !(loads & 2)) return EA_UNPORTED_LINEAR_WALK;
    ea_jobs jobs = *jobs_in;
    int blocks = 0;
    for (int i = 0; i < jobs.n; ++i) {
        ea_job& j = jobs.j[i];
        if (j.SK < 1 || wk == 0 || (kdim / 16) % (j.SK * wk) != 0) return EA_UNEVEN_K_SPLIT;
        if (j.N % 128 != 0) return EA_BAD_WIDTH;
        if (j.SK > 1 && (!j.Z || !j.counters)) return EA_BAD_ARGUMENT;
        j.start = blocks;
        blocks += (j.N / 128) * j.SK;
    }
    if (!variant_built(k2, cb, wk)) return EA_UNPORTED_LINEAR_VARIANT;
    if (m == 0 || blocks == 0) return EA_OK;
    if (m > 128) return EA_NOT_GROUPABLE;
    launch_variant(jobs, blocks, s, (int)m, (int)kdim, k2, cb, (int)wk);
    return launched();
}

}  // namespace ea

using namespace ea;

extern "C" {

int ea_exl3_rot_in(ea_stream_t stream, const void* x, int x_dtype, const ea_rot_jobs* jobs, uint32_t njobs,
                   uint32_t m, uint32_t kdim) {
    return launch_lin_rot_in(as_stream(stream), x, x_dtype, jobs, njobs, m, kdim);
}

int ea_exl3_linear(ea_stream_t stream, const ea_jobs* jobs, uint32_t m, uint32_t kdim, uint32_t k2, uint32_t cb,
                   uint32_t wk, uint32_t loads) {
    return launch_linear(as_stream(stream), jobs, m, kdim, k2, cb, wk, loads);
}

// linear.zig:198-214
void ea_linear_plan(uint32_t k, uint32_t n, uint32_t* sk_out, uint32_t* wk_out) {
    const uint32_t kt = k / 16, nb = n / 128;
    uint32_t sk = 1, wk = nb >= 64 ? 8 : 4;
    if (nb < 64)
        while (nb * sk < 192 && sk < 64) sk *= 2;
    while ((wk > 4 || sk > 1) && (kt % (sk * wk) != 0 || kt / (sk * wk) < 8)) {
        if (wk > 4) wk = 4;
        else if (sk > 1) sk /= 2;
        else break;
    }
    if (sk_out) *sk_out = sk;
    if (wk_out) *wk_out = wk;
}

// linear.zig:270-275
static bool groupable(const ea_linear* const* ls, uint32_t n) {
    if (!ls || n == 0 || n > EA_MAX_JOBS) return false;
    const ea_linear* a = ls[0];
    if (!a) return false;
    for (uint32_t i = 0; i < n; ++i)
        if (!ls[i] || ls[i]->k != a->k || ls[i]->k2 != a->k2 || ls[i]->cb != a->cb || ls[i]->wk != a->wk) return false;
    return true;
}

// the kernels' load options the engine uses: bits 1 and 2 (linear.zig:293-295; PDL has no counterpart here)
static const uint32_t LOADS = 3;

int ea_linear_call_rotated(ea_stream_t stream, const ea_linear_scratch* s, const ea_linear* const* ls, uint32_t nls,
                           uint32_t m, const uint64_t* outs, const int* out_dtypes) {
    if (!groupable(ls, nls) || m < 1 || m > 128) return EA_NOT_GROUPABLE;
    if (!s || !outs || !out_dtypes) return EA_BAD_ARGUMENT;
    ea_jobs jobs{};
    jobs.n = (int32_t)nls;
    for (uint32_t i = 0; i < nls; ++i) {
        const ea_linear* l = ls[i];
        const int64_t tw = 4 * (int64_t)l->k2;
        ea_job& j = jobs.j[i];
        j.xh = s->xh[i];
        j.T = l->words;
        j.stride_k = 8 * tw;
        j.stride_nb = (int64_t)(l->k / 16) * 8 * tw;
        j.svh = l->svh;
        j.bias = 0;
        j.y = outs[i];
        j.Z = l->sk > 1 ? s->z[i] : 0;
        j.counters = l->counters;
        j.y_dtype = out_dtypes[i];
        j.N = (int32_t)l->n;
        j.SK = (int32_t)l->sk;
    }
    return launch_linear(as_stream(stream), &jobs, m, ls[0]->k, ls[0]->k2, ls[0]->cb, ls[0]->wk, LOADS);
}

int ea_linear_call(ea_stream_t stream, const ea_linear_scratch* s, const ea_linear* const* ls, uint32_t nls,
                   const void* x, int x_dtype, uint32_t m, const uint64_t* outs, const int* out_dtypes) {
    if (!groupable(ls, nls) || m < 1 || m > 128) return EA_NOT_GROUPABLE;
    if (!s) return EA_BAD_ARGUMENT;
    ea_rot_jobs rj{};
    for (uint32_t i = 0; i < nls; ++i) {
        rj.suh[i] = ls[i]->suh;
        rj.xh[i] = s->xh[i];
    }
    int r = launch_lin_rot_in(as_stream(stream), x, x_dtype, &rj, nls, m, ls[0]->k);
    if (r) return r;
    return ea_linear_call_rotated(stream, s, ls, nls, m, outs, out_dtypes);
}

}  // extern "C"
