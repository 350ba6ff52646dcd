// EXL3 linear for 1 to 128 rows (the shared expert and any strips-layout linear): input rotation for 1..3 jobs
// of one input, and one launch over 1..3 jobs with per-job K splits finished by the last-arriving block
// (exl3_linear.cu:69-484, exl3.zig, linear.zig). Rows are independent; sums run in a fixed order: waves of a
// block in order, then splits in order.
#include <hip/hip_runtime.h>

#include "ea_device.hpp"
#include "ea_gemm.hpp"
#include "ea_host.hpp"
#include "ea_stamps.hpp"

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

// The same with svh and bias already loaded: sw, bw hold this lane's two columns (two fp16 each; bias optional).
__device__ __forceinline__ void finish_store_pre(float v0, float v1, int lane, uint32_t sw, bool has_bias, uint32_t bw,
                                                 void* y, int y_dtype, size_t at) {
    fwht128_w64(v0, v1, lane);
    v0 = v0 * HAD_SCALE * h2f((uint16_t)(sw & 0xffffu));
    v1 = v1 * HAD_SCALE * h2f((uint16_t)(sw >> 16));
    if (has_bias) {
        v0 += h2f((uint16_t)(bw & 0xffffu));
        v1 += h2f((uint16_t)(bw >> 16));
    }
    store_act(y, y_dtype, at, v0);
    store_act(y, y_dtype, at + 1, v1);
}

__device__ __forceinline__ float load_coherent(const float* p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Block (job, column block nb of 128, split; pass of 16 rows = blockIdx.y): WK waves each take per_warp consecutive k
// tiles of the split for the pass's rows. Every pass is its own block (the passes decode the same tiles side by side,
// not one after another: 128 rows of a 6144 x 256 linear are 256 blocks, not 32 blocks of eight passes). SK == 1: the
// block finishes its columns. SK > 1: partial sums to Z[split], and the block that arrives last on the (pass, nb)
// counter sums the splits in order, finishes, and resets the counter to zero.
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
    {
        const int pass = (int)blockIdx.y, m0 = 16 * pass;
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
                // the wave's rows wave, wave + WK, ..: QB splits of all of them loaded at once (64 values a lane),
                // then added in split order (one round trip a batch of splits instead of one a split and row)
                constexpr int RW = 16 / WK, QB = 32 / RW;
                float v[RW][2];
                for (int q0 = 0; q0 < SK; q0 += QB) {
                    float z[QB][RW][2];
#pragma unroll
                    for (int q = 0; q < QB; ++q)
#pragma unroll
                        for (int i = 0; i < RW; ++i) {
                            const int rr = wave + WK * i < R ? wave + WK * i : wave;  // rows past R re-read a row
                            const size_t at = (size_t)(q0 + q < SK ? q0 + q : q0) * M * N +
                                              ((size_t)m0 + rr) * N + col0 + 2 * lane;
                            z[q][i][0] = load_coherent(Z + at);
                            z[q][i][1] = load_coherent(Z + at + 1);
                        }
#pragma unroll
                    for (int q = 0; q < QB; ++q)
                        if (q0 + q < SK) {  // uniform
#pragma unroll
                            for (int i = 0; i < RW; ++i) {
                                v[i][0] = q0 + q == 0 ? z[q][i][0] : v[i][0] + z[q][i][0];
                                v[i][1] = q0 + q == 0 ? z[q][i][1] : v[i][1] + z[q][i][1];
                            }
                        }
                }
#pragma unroll
                for (int i = 0; i < RW; ++i) {
                    const int rr = wave + WK * i;
                    if (rr >= R) break;  // uniform
                    const size_t at = ((size_t)m0 + rr) * N + col0 + 2 * lane;
                    finish_store(v[i][0], v[i][1], lane, svh, bias, y, J.y_dtype, at, col0 + 2 * lane);
                }
                if (threadIdx.x == 0) counters[pass * NB + nb] = 0;  // every split of the column block arrived
            }
        }
    }
}

// ---- the small-row linear: up to 16 rows, K split, every CU busy ----------------------------------------------------
// Block (job, group g of 32 columns, split s) with WK waves: wave w multiplies k tiles [s KS + w NKT, + NKT) of the
// group's two column tiles (KS = WK NKT, the split's tiles), the trellis staged in LDS by 16-byte loads; the waves'
// sums are added in order into Z[s] (agent-scope stores), and the last of the 4 SK blocks of a 128-column block to
// count in adds the splits in order and finishes it (FWHT, svh, bias). That is the reference's order of sums (waves,
// then splits, exl3_linear.cu:231-484) over four times as many blocks as its (column block, split) grid. With ROT
// the block rotates the activations of its split itself (the Hadamard blocks its k range touches) and the column
// group 0 blocks also store them to xh, as the separate rotation would.
//
// Tagged form (TAG; the split count even, at most 2 LS_MAXTS, and the block's LDS within bounds): the caller's Z
// (fp32 [SK, M, N]) holds SK / 2 splits of 8-byte slots instead, each block twice the k range on twice the waves, and
// a block stores each sum with the tag LS_TAG in the slot's high half in one 8-byte agent-scope store; the
// finisher polls the slots themselves until every tag is LS_TAG, adds the splits in order, and stores zero into every
// slot it read. So a writer never waits for its stores, and the finisher needs one round trip once the data has
// landed, where the flag form needs the writer's store acknowledgement, the flag's round trip and then a second
// round trip for the data. The tag is a signalling-NaN bit pattern: no fp32 result has it (arithmetic quiets NaNs),
// so partial sums the flag form left in the same buffer are never taken for tagged slots, and Z needs no clearing
// between the two forms. A Z buffer must not hold the tag when first used (zero, as the counters start, is fine).
constexpr int LS_MAXR = 16;
constexpr int LS_MAXNKT = 16;
constexpr int LS_FLAGS = 32;  // flag bytes a 128-column block has in the counters (int32 [8 N / 128], zero between calls)
constexpr int LS_MAXTS = 8;   // tagged splits the finisher polls at once (two slots a lane each)
constexpr int LS_PASS = 8;    // rows a pass of the tagged form (passes side by side up to 128 rows)
constexpr uint32_t LS_TAG = 0x7FB5EA1Du;
constexpr int LS_POLLS = 1 << 20;  // polls before the finisher gives up (tens of milliseconds)

// A small-row block's sum of (row m, column c) over its WK (at most 16) waves' sums in red, added in wave order, with
// every LDS read issued before the first add (a loop over the run-time wave count waited for its reads in turn).
__device__ __forceinline__ float ls_wave_sum(const float* red, int WK, int m, int c) {
    float v[16];
#pragma unroll
    for (int w = 0; w < 16; ++w) v[w] = red[(min(w, WK - 1) * 16 + m) * 32 + c];
    float sum = v[0];
#pragma unroll
    for (int w = 1; w < 16; ++w) sum = w < WK ? sum + v[w] : sum;
    return sum;
}

// The tagged form's finisher (the highest-index block of a 128-column block's blocks): a wave a row of its pass, two
// columns a lane. Its own split's slots of its own 32 columns (lanes 48..63) come from red, the others are polled;
// every read slot is set back to zero. TS >= SK splits are loaded each poll, every one before any is checked (loads
// under a lane condition, or under the split count, made the compiler wait for each split's loads in turn): splits
// past SK read the last split's slots again, and a lane's own split (never written) is read but not checked.
template <int TS>
__device__ __forceinline__ void ls_finish_rows(const ea_job& J, uint64_t* Zt, const float* red, int M_all, int m0,
                                               int M, int N, int col, int SK, int wave, int WK, int lane, uint32_t svw,
                                               uint32_t bw, int* status) {
    const bool own = lane >= 48;
    for (int m = wave; m < M; m += WK) {
        uint64_t p[TS][2];
        bool timed_out = false;
        for (int n = 0;; ++n) {
#pragma unroll
            for (int q = 0; q < TS; ++q) {
                const uint64_t* at = Zt + ((size_t)min(q, SK - 1) * M_all + m0 + m) * N + col;
                p[q][0] = __hip_atomic_load(at, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                p[q][1] = __hip_atomic_load(at + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
            bool ok = true;
#pragma unroll
            for (int q = 0; q < TS; ++q)
                ok &= q >= SK || (own && q == SK - 1) ||
                      ((uint32_t)(p[q][0] >> 32) == LS_TAG && (uint32_t)(p[q][1] >> 32) == LS_TAG);
            if (__builtin_amdgcn_ballot_w64(!ok) == 0) break;
            if (n >= LS_POLLS) {
                timed_out = true;
                if (lane == 0) record_error(status, DEV_SYNC_TIMEOUT);
                break;
            }
            __builtin_amdgcn_s_sleep(1);
        }
        EA_STAMP(7, threadIdx.x == 0);  // wave 0's polls done
        // the lane's own split (lanes 48..63, the last split) from red: every lane reads red, in bounds
        const int c = own ? 2 * lane - 96 : 0;
        const float r0 = red[m * 32 + c], r1 = red[m * 32 + c + 1];
        const bool own0 = own && SK == 1;
        float2 acc2 = float2{own0 ? r0 : __uint_as_float((uint32_t)p[0][0]),
                             own0 ? r1 : __uint_as_float((uint32_t)p[0][1])};
#pragma unroll
        for (int q = 1; q < TS; ++q)
            if (q < SK) {
                const bool mine = own && q == SK - 1;
                acc2.x += mine ? r0 : __uint_as_float((uint32_t)p[q][0]);
                acc2.y += mine ? r1 : __uint_as_float((uint32_t)p[q][1]);
            }
        // the slots read go back to zero for the next call. After a give-up they are left as they are: a writer that
        // arrives late would tag a slot just cleared, and the next call's finisher would take that stale sum for its
        // own; the status word says EA_SYNC_TIMEOUT instead, and z must be zeroed again before reuse
        if (!timed_out)
            for (int q = 0; q < SK; ++q)
                if (!(own && q == SK - 1)) {
                    uint64_t* at = Zt + ((size_t)q * M_all + m0 + m) * N + col;
                    __hip_atomic_store(at, (uint64_t)0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                    __hip_atomic_store(at + 1, (uint64_t)0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                }
        if (timed_out) acc2 = float2{__builtin_nanf(""), __builtin_nanf("")};  // a writer never arrived
        finish_store_pre(acc2.x, acc2.y, lane, svw, J.bias != 0, bw, dptr<void>(J.y), J.y_dtype,
                         (size_t)(m0 + m) * N + col);
    }
}

template <int CB, int K2, int NKT, bool ROT, int XL, bool TAG>
__global__ void __launch_bounds__(1024) lin_small_kernel(ea_jobs jobs, ea_rot_jobs rj, int M_all, int K,
                                                        const void* x, int x_bf16, int* status) {
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    constexpr int TW = 4 * K2;
    EA_STAMP(0, threadIdx.x == 0);  // the block's start
    // the tagged form takes the call's rows in passes of LS_PASS side by side (blockIdx.y): rows m0 .. m0 + M - 1 of
    // M_all; the flag form all of them (at most LS_MAXR) in one
    const int m0 = TAG ? (int)blockIdx.y * LS_PASS : 0;
    const int M = TAG ? min(LS_PASS, M_all - m0) : M_all;
    int ji = 0;
#pragma unroll
    for (int q = 1; q < EA_MAX_JOBS; ++q)
        if (q < jobs.n && (int)blockIdx.x >= jobs.j[q].start) ji = q;
    const ea_job& J = jobs.j[ji];
    const int WK = blockDim.x >> 6, NT = WK * 64;
    const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6)), lane = threadIdx.x & 63;
    const int N = J.N, SK = J.SK, G = N >> 5;
    const int local = (int)blockIdx.x - J.start, g = local % G, split = local / G;
    const int kh = NKT * WK * 16, lo = split * kh;
    // the block's activations: rows of the Hadamard blocks [hb0, hb0 + span / 128) that its k range touches (ROT), or
    // its k range (rotated already)
    const int hb0 = ROT ? lo >> 7 : 0, span = ROT ? (((lo + kh + 127) >> 7) - hb0) * 128 : kh;
    const int k_first = ROT ? hb0 * 128 : lo, xoff = lo - k_first, XS = span + 8;  // XS: rows in different banks
    uint16_t* xs = reinterpret_cast<uint16_t*>(lds);
    uint16_t* suh_s = xs + M * XS;
    uint32_t* stage = reinterpret_cast<uint32_t*>(lds + (((size_t)(M + 1) * XS * 2 + 15) & ~(size_t)15));
    float* red = reinterpret_cast<float*>(stage);  // after the products: [WK][16][32]
    uint32_t* st = stage + wave * NKT * 2 * TW;

    // the wave's trellis first: NKT rows of its two adjacent column tiles (strips layout). The tiles decode into
    // registers as soon as they land, while the activations (loaded next) are still in flight: the decode needs only
    // the trellis, and the MFMAs wait for the rotated activations.
    const int nt0 = 2 * g;
    TileSpan sp;
    const int64_t tiles_end = (int64_t)((N >> 7) - 1) * J.stride_nb + (int64_t)(K >> 4) * J.stride_k;
    sp.r = buffer_rsrc(dptr<const uint32_t>(J.T), (uint32_t)(tiles_end * 4));
    sp.off = (int)((((int64_t)(lo >> 4) + wave * NKT) * J.stride_k + (nt0 >> 3) * J.stride_nb + (nt0 & 7) * TW) * 4);
    sp.kstride = (int)(J.stride_k * 4);
    u4v v[stage_loads_k<NKT, K2>()];
    stage_issue_k<NKT, K2>(sp, lane, v);

    // then the activation rows (and suh), 16 bytes a load, every load issued (a thread past the end reads the last
    // chunk again). XL = 0 (rotating, and no more (row, Hadamard block) items than waves): wave w loads item w's two
    // values a lane and their suh itself, rotates them in registers while the other waves decode, and only the barrier
    // before the products is left (the block-level form stages the rows, waits, rotates, waits again)
    constexpr bool PWR = ROT && XL == 0;
    const uint16_t* xsrc = ROT ? static_cast<const uint16_t*>(x) : dptr<const uint16_t>(J.xh);
    const int cpr = span >> 3, chunks = M * cpr;  // 16-byte chunks a row, in all
    const int nhb = span >> 7;
    u4v xv[XL > 0 ? XL : 1];
    u4v sv = u4v{0u, 0u, 0u, 0u};
    uint32_t rxw = 0u, rsw = 0u;
    if constexpr (PWR) {
        const int it = wave < M * nhb ? wave : 0, m = it / nhb, hb = it - m * nhb;  // past the items: item 0 again
        rxw = *reinterpret_cast<const uint32_t*>(xsrc + (size_t)(m0 + m) * K + k_first + hb * 128 + 2 * lane);
        rsw = *reinterpret_cast<const uint32_t*>(dptr<const uint16_t>(rj.suh[ji]) + k_first + hb * 128 + 2 * lane);
    } else {
#pragma unroll
        for (int i = 0; i < XL; ++i) {
            const int c = min(i * NT + (int)threadIdx.x, chunks - 1), m = c / cpr, cc = c - m * cpr;
            xv[i] = *reinterpret_cast<const u4v*>(xsrc + (size_t)(m0 + m) * K + k_first + 8 * cc);
        }
        if constexpr (ROT)
            sv = *reinterpret_cast<const u4v*>(dptr<const uint16_t>(rj.suh[ji]) + k_first +
                                               8 * min((int)threadIdx.x, cpr - 1));
    }
    // the svh and bias of the lane's two columns of the 128-column block, for whichever block finishes it (loaded by
    // every block, unconditionally: a load in a branch would make the compiler wait for all loads before the first use)
    const bool finisher = (g & 3) == 3 && split == SK - 1;  // the highest-index block of the 4 SK
    // descriptor: 1 a block that hands its sums on, 2 the finisher; column group, split
    EA_STAMP_VALUE(STAMP_POINTS - 1, (uint64_t)(finisher ? 2 : 1) | (uint64_t)g << 8 | (uint64_t)split << 20,
                   threadIdx.x == 0);
    const int col = (g >> 2) * 128 + 2 * lane;
    const uint16_t* svh = dptr<const uint16_t>(J.svh);
    const uint16_t* bias = dptr<const uint16_t>(J.bias);
    const uint32_t svw = *reinterpret_cast<const uint32_t*>(svh + col);
    const uint32_t bw = *reinterpret_cast<const uint32_t*>((bias ? bias : svh) + col);
    issued();
#pragma unroll
    for (int i = 0; i < XL; ++i) hold(xv[i]);
    hold(sv);
    hold(rxw);
    hold(rsw);
    if constexpr (PWR) {
        // this wave's item, rotated into the staged rows (exl3_linear.cu:152-173 per (row, Hadamard block))
        if (wave < M * nhb) {
            const int m = wave / nhb, hb = wave - m * nhb;
            const uint16_t x0 = (uint16_t)(rxw & 0xffffu), x1 = (uint16_t)(rxw >> 16);
            float v0 = (x_bf16 ? bf2f(x0) : h2f(x0)) * h2f((uint16_t)(rsw & 0xffffu));
            float v1 = (x_bf16 ? bf2f(x1) : h2f(x1)) * h2f((uint16_t)(rsw >> 16));
            fwht128_w64(v0, v1, lane);
            const uint32_t h = (uint32_t)f2h(v0 * HAD_SCALE) | ((uint32_t)f2h(v1 * HAD_SCALE) << 16);
            *reinterpret_cast<uint32_t*>(xs + m * XS + hb * 128 + 2 * lane) = h;
            uint16_t* xh = dptr<uint16_t>(rj.xh[ji]);
            if (g == 0 && xh)
                *reinterpret_cast<uint32_t*>(xh + (size_t)(m0 + m) * K + (hb0 + hb) * 128 + 2 * lane) = h;
        }
    }
    // the trellis into the wave's LDS region (it waits only for the trellis loads), then every tile decoded into its
    // MFMA operand
    stage_store_k<NKT, K2>(st, lane, v);
    EA_STAMP(1, threadIdx.x == 0);  // wave 0's trellis landed
    const LaneQuad lq = lane_quad_k<K2>(lane);
    u4v bq[NKT / 2][2];
    {
        const uint32_t* wa = st + lq.w0;
        const uint32_t* wb = st + lq.w1;
#pragma unroll
        for (int t = 0; t < NKT; t += 2)
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                const int t0 = (2 * t + j) * TW, t1 = (2 * (t + 1) + j) * TW;
                const u2v b0 = decode_quad<K2, CB>(wa[t0], wb[t0], lq.sh);
                const u2v b1 = decode_quad<K2, CB>(wa[t1], wb[t1], lq.sh);
                bq[t >> 1][j] = u4v{b0.x, b0.y, b1.x, b1.y};
            }
    }
#pragma unroll
    for (int t = 0; t < NKT / 2; ++t)
#pragma unroll
        for (int j = 0; j < 2; ++j) hold(bq[t][j]);  // decoded before the activations are waited for
    EA_STAMP(2, threadIdx.x == 0);  // wave 0's tiles decoded
#pragma unroll
    for (int i = 0; i < XL; ++i) {
        const int c = i * NT + (int)threadIdx.x;
        if (c < chunks) {
            const int m = c / cpr, cc = c - m * cpr;
            *reinterpret_cast<u4v*>(xs + m * XS + 8 * cc) = xv[i];
        }
    }
    if (ROT && !PWR && (int)threadIdx.x < cpr) *reinterpret_cast<u4v*>(suh_s + 8 * threadIdx.x) = sv;
    __syncthreads();
    EA_STAMP(3, threadIdx.x == 0);  // the activations in LDS (rotated with PWR), every wave's tiles decoded
    if constexpr (ROT && !PWR) {
        // rotate in place: a wave a (row, Hadamard block), two values a lane (exl3_linear.cu:152-173)
        uint16_t* xh = dptr<uint16_t>(rj.xh[ji]);
        for (int item = wave; item < M * nhb; item += WK) {
            const int m = item / nhb, hb = item - m * nhb;
            uint32_t* p = reinterpret_cast<uint32_t*>(xs + m * XS + hb * 128 + 2 * lane);
            const uint32_t xw = *p, sw = *reinterpret_cast<const uint32_t*>(suh_s + hb * 128 + 2 * lane);
            const uint16_t x0 = (uint16_t)(xw & 0xffffu), x1 = (uint16_t)(xw >> 16);
            float v0 = (x_bf16 ? bf2f(x0) : h2f(x0)) * h2f((uint16_t)(sw & 0xffffu));
            float v1 = (x_bf16 ? bf2f(x1) : h2f(x1)) * h2f((uint16_t)(sw >> 16));
            fwht128_w64(v0, v1, lane);
            const uint32_t h = (uint32_t)f2h(v0 * HAD_SCALE) | ((uint32_t)f2h(v1 * HAD_SCALE) << 16);
            *p = h;
            if (g == 0 && xh)
                *reinterpret_cast<uint32_t*>(xh + (size_t)(m0 + m) * K + (hb0 + hb) * 128 + 2 * lane) = h;
        }
        __syncthreads();
        EA_STAMP(4, threadIdx.x == 0);  // rotated
    }

    // the product: A rows are the activation rows (zero past M), B the decoded tiles. The lanes of the call's rows
    // read every k step's operand in one branch before the first product (one LDS round trip, not one a step);
    // the other lanes' operands stay zero.
    const int row = lane & 15;
    h8v a[NKT / 2];
#pragma unroll
    for (int t = 0; t < NKT / 2; ++t) a[t] = h8v{0, 0, 0, 0, 0, 0, 0, 0};
    if (row < M) {
        const uint16_t* xr = xs + row * XS + xoff + wave * NKT * 16;
#pragma unroll
        for (int t = 0; t < NKT / 2; ++t) a[t] = load_a8(xr, 2 * t * 16, lane);
    }
    f4v acc[2] = {f4v{0.f, 0.f, 0.f, 0.f}, f4v{0.f, 0.f, 0.f, 0.f}};
#pragma unroll
    for (int t = 0; t < NKT; t += 2) {
#pragma unroll
        for (int j = 0; j < 2; ++j)
            acc[j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[t >> 1], __builtin_bit_cast(h8v, bq[t >> 1][j]), acc[j],
                                                            0, 0, 0);
    }
    // the wave sums take the staged trellis' place in LDS with no barrier first: each wave read only its own staged
    // tiles, and every wave had decoded them before the barrier above
    EA_STAMP(5, threadIdx.x == 0);  // this wave's MFMAs done
    // the rows the call has (lane group lane >> 4 holds rows 4 (lane >> 4) .. + 3); the others are never read
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int i = 0; i < 4; ++i)
            if (4 * (lane >> 4) + i < M) red[(wave * 16 + 4 * (lane >> 4) + i) * 32 + j * 16 + row] = acc[j][i];
    __syncthreads();
    if constexpr (TAG) {
        // the block's sums into its tagged slots; the finisher keeps its own in red's first rows (its slots are
        // never written, so nothing it does not read carries the tag)
        uint64_t* Zt = dptr<uint64_t>(J.Z);
        for (int idx = threadIdx.x; idx < M * 32; idx += WK * 64) {
            const int m = idx >> 5, c = idx & 31;
            const float sum = ls_wave_sum(red, WK, m, c);
            red[m * 32 + c] = sum;
            if (!finisher)
                __hip_atomic_store(Zt + ((size_t)split * M_all + m0 + m) * N + g * 32 + c,
                                   ((uint64_t)LS_TAG << 32) | __float_as_uint(sum), __ATOMIC_RELAXED,
                                   __HIP_MEMORY_SCOPE_AGENT);
        }
        EA_STAMP(6, threadIdx.x == 0);  // thread 0's sums stored (the finisher: kept)
        if (!finisher) return;
        __syncthreads();
        // the finisher: a wave a row, two columns a lane (ls_finish_rows), its poll built for the split count rounded
        // up to a power of two
        if (SK <= 1)
            ls_finish_rows<1>(J, Zt, red, M_all, m0, M, N, col, SK, wave, WK, lane, svw, bw, status);
        else if (SK <= 2)
            ls_finish_rows<2>(J, Zt, red, M_all, m0, M, N, col, SK, wave, WK, lane, svw, bw, status);
        else if (SK <= 4)
            ls_finish_rows<4>(J, Zt, red, M_all, m0, M, N, col, SK, wave, WK, lane, svw, bw, status);
        else
            ls_finish_rows<LS_MAXTS>(J, Zt, red, M_all, m0, M, N, col, SK, wave, WK, lane, svw, bw, status);
        EA_STAMP(8, threadIdx.x == 0);  // wave 0's rows finished
        return;
    }
    float* Z = dptr<float>(J.Z);
    for (int idx = threadIdx.x; idx < M * 32; idx += WK * 64) {
        const int m = idx >> 5, c = idx & 31;
        const float sum = ls_wave_sum(red, WK, m, c);
        st_coh(Z + ((size_t)split * M + m) * N + g * 32 + c, sum);
    }
    stores_done();
    __syncthreads();
    __shared__ int last;
    if (4 * SK <= LS_FLAGS) {
        // flags: each of the 4 SK blocks of the 128-column block sets its byte in the column block's eight counter
        // words (zero between calls); the block of highest index among them (the last dispatched) waits for all of
        // them, then finishes and clears them. Nothing contends for one address.
        uint8_t* flags = reinterpret_cast<uint8_t*>(dptr<int>(J.counters) + (g >> 2) * (LS_FLAGS / 4));
        if (threadIdx.x == 0) __hip_atomic_store(flags + (g & 3) + 4 * split, (uint8_t)1, __ATOMIC_RELAXED,
                                                 __HIP_MEMORY_SCOPE_AGENT);
        if (!finisher) return;
        if (threadIdx.x < 64) {
            const int* fw = reinterpret_cast<const int*>(flags);
            const int words = SK;  // 4 SK flag bytes
            int n = 0;
            bool ready = false;
            while (!ready) {
                const int v = lane < words ? ld_coh(fw + lane) : 0x01010101;
                ready = __builtin_amdgcn_ballot_w64(v != 0x01010101) == 0;
                if (!ready && ++n > (1 << 20)) break;
                if (!ready) __builtin_amdgcn_s_sleep(1);
            }
            if (lane < words) reset_count(const_cast<int*>(fw) + lane);
            if (lane == 0) {
                last = ready ? 1 : 2;
                if (!ready) record_error(status, DEV_SYNC_TIMEOUT);
            }
        }
        __syncthreads();
    } else {
        int* counter = dptr<int>(J.counters) + (g >> 2);
        if (threadIdx.x == 0) {
            last = count_in(counter) == 4 * SK - 1;
            if (last) reset_count(counter);
        }
        __syncthreads();
        if (!last) return;
    }
    // the last block of the 128-column block: the splits in order (eight loaded at once), then finish
    for (int m = wave; m < M; m += WK) {
        float2 acc2;
        for (int q0 = 0; q0 < SK; q0 += 8) {
            float2 z[8];
#pragma unroll
            for (int q = 0; q < 8; ++q) z[q] = ld_coh2(Z + ((size_t)(q0 + q < SK ? q0 + q : q0) * M + m) * N + col);
#pragma unroll
            for (int q = 0; q < 8; ++q)
                if (q0 + q < SK) {
                    acc2.x = q0 + q == 0 ? z[q].x : acc2.x + z[q].x;
                    acc2.y = q0 + q == 0 ? z[q].y : acc2.y + z[q].y;
                }
        }
        if (last == 2) acc2 = float2{__builtin_nanf(""), __builtin_nanf("")};  // a writer never arrived
        finish_store_pre(acc2.x, acc2.y, lane, svw, bias != nullptr, bw, dptr<void>(J.y), J.y_dtype,
                         (size_t)m * N + col);
    }
}

// LDS of a small-row block: the activation rows and suh, and the staged trellis (then the wave sums).
static size_t lin_small_lds(int M, int K2, int NKT, int WK, bool rot) {
    const int kh = NKT * WK * 16, span = rot ? kh + 256 : kh;
    const size_t xs = (((size_t)(M + 1) * (span + 8) * 2) + 15) & ~(size_t)15;
    const size_t stage = (size_t)WK * NKT * 2 * 4 * K2 * 4, red = (size_t)WK * 16 * 32 * 4;
    return xs + (stage > red ? stage : red);
}

template <int CB, int K2, bool ROT, int XL, bool TAG>
static void launch_small_xl(const ea_jobs& jobs, const ea_rot_jobs& rj, int blocks, hipStream_t s, int M, int K, int wk,
                            int nkt, const void* x, int x_bf16, size_t lds, int* status) {
    const dim3 grid((unsigned)blocks, TAG ? (unsigned)((M + LS_PASS - 1) / LS_PASS) : 1u);  // the tagged form's passes
#define EA_LS(NKT_)                                                                                                 \
    if (nkt == NKT_) {                                                                                              \
        lin_small_kernel<CB, K2, NKT_, ROT, XL, TAG><<<grid, wk * 64, lds, s>>>(jobs, rj, M, K, x, x_bf16, status); \
        return;                                                                                                     \
    }
    EA_LS(2) EA_LS(4) EA_LS(6) EA_LS(8) EA_LS(10) EA_LS(12) EA_LS(14) EA_LS(16)
#undef EA_LS
}

template <int CB, int K2, bool ROT, bool TAG>
static bool launch_small_k2(const ea_jobs& jobs, const ea_rot_jobs& rj, int blocks, hipStream_t s, int M, int K,
                            int wk, int nkt, const void* x, int x_bf16, int* status) {
    const int mp = TAG && M > LS_PASS ? LS_PASS : M;  // the rows a block takes
    const size_t lds = lin_small_lds(mp, K2, nkt, wk, ROT);
    if (lds > 64 * 1024) return false;
    // 16-byte activation loads a thread: the rows' span over the block's threads
    const int kh = nkt * wk * 16, span_max = ROT ? kh + 256 : kh;
    const int xl = (mp * (span_max / 8) + wk * 64 - 1) / (wk * 64);
    // rotating with at most one (row, Hadamard block) a wave (the blocks' k ranges then start on Hadamard blocks)
    if constexpr (ROT) {
        if (kh % 128 == 0 && mp * (kh / 128) <= wk) {
            launch_small_xl<CB, K2, ROT, 0, TAG>(jobs, rj, blocks, s, M, K, wk, nkt, x, x_bf16, lds, status);
            return true;
        }
    }
    if (xl <= 1) launch_small_xl<CB, K2, ROT, 1, TAG>(jobs, rj, blocks, s, M, K, wk, nkt, x, x_bf16, lds, status);
    else if (xl <= 2) launch_small_xl<CB, K2, ROT, 2, TAG>(jobs, rj, blocks, s, M, K, wk, nkt, x, x_bf16, lds, status);
    else if (xl <= 4) launch_small_xl<CB, K2, ROT, 4, TAG>(jobs, rj, blocks, s, M, K, wk, nkt, x, x_bf16, lds, status);
    else if (xl <= 8) launch_small_xl<CB, K2, ROT, 8, TAG>(jobs, rj, blocks, s, M, K, wk, nkt, x, x_bf16, lds, status);
    else return false;
    return true;
}

// The small-row grid of a job set: 32-column groups x splits of every job, each job's first block in `start`.
static int small_grid(ea_jobs& sj) {
    int nb = 0;
    for (int i = 0; i < sj.n; ++i) {
        sj.j[i].start = nb;
        nb += (sj.j[i].N >> 5) * sj.j[i].SK;
    }
    return nb;
}

// The small-row kernel when it applies (m <= 16, every job split (SK > 1) with the same even per-wave tile count up to
// 16, a width the staged decode takes, 16-bit activations when rotating); false otherwise, and nothing is launched.
static bool launch_small(const ea_jobs& jobs, const ea_rot_jobs* rj, hipStream_t s, int M, int K, uint32_t k2,
                         uint32_t cb, int wk, const void* x, int x_dtype, int* status) {
    if (M > 128 || k2 > (uint32_t)STAGE_MAXK2) return false;
    if (rj && x_dtype != F16 && x_dtype != BF16) return false;
    const uintptr_t align = rj ? reinterpret_cast<uintptr_t>(x) | (uintptr_t)K * 2 : (uintptr_t)K * 2;
    if (align & 15) return false;  // 16-byte activation loads
    const int nkt = (K >> 4) / jobs.j[0].SK / wk;
    for (int i = 0; i < jobs.n; ++i) {
        const ea_job& j = jobs.j[i];
        if (j.SK < 2 || (K >> 4) % (j.SK * wk) != 0 || (K >> 4) / j.SK / wk != nkt) return false;
        if (!rj && (!j.xh || (j.xh & 15))) return false;
        if (rj && ((rj->suh[i] & 15) || (rj->xh[i] & 3))) return false;
    }
    if (nkt < 2 || nkt > LS_MAXNKT || (nkt & 1)) return false;
    const ea_rot_jobs r = rj ? *rj : ea_rot_jobs{};
    const int bf = x_dtype == BF16;
    // the tagged form when every job's split count is even and at most 2 LS_MAXTS (half the splits, twice the
    // waves, 8-byte slots in the same Z); the flag form otherwise, or when the tagged block's LDS does not fit
    bool tag = 2 * wk <= 8;
    for (int i = 0; i < jobs.n; ++i) tag = tag && jobs.j[i].SK % 2 == 0 && jobs.j[i].SK <= 2 * LS_MAXTS;
    ea_jobs tj = jobs;
    for (int i = 0; i < tj.n; ++i) tj.j[i].SK /= 2;
    ea_jobs sj = jobs;
    const int tb = small_grid(tj), nb = small_grid(sj);
    // the tagged form on sixteen waves a block (four a SIMD) when its waves' k tiles halve evenly once more: the
    // same decode over twice the waves (config 1: 8.64 -> 8.55 us)
    int tw = 2 * wk, tn = nkt;
    if (tn % 4 == 0 && 2 * tw <= 16) {
        tw *= 2;
        tn /= 2;
    }
    // the tagged form on sixteen waves; above LS_MAXR rows, when its block's LDS is too large for a pass's rows, on
    // eight; the flag form up to LS_MAXR rows; otherwise not this kernel
#define EA_SV(K2_, CB_)                                                                                            \
    if (k2 == K2_ && cb == CB_) {                                                                                  \
        if (tag && (rj ? launch_small_k2<CB_, K2_, true, true>(tj, r, tb, s, M, K, tw, tn, x, bf, status)          \
                       : launch_small_k2<CB_, K2_, false, true>(tj, r, tb, s, M, K, tw, tn, x, bf, status)))       \
            return true;                                                                                           \
        if (tag && M > LS_MAXR && tw != 2 * wk &&                                                                  \
            (rj ? launch_small_k2<CB_, K2_, true, true>(tj, r, tb, s, M, K, 2 * wk, nkt, x, bf, status)            \
                : launch_small_k2<CB_, K2_, false, true>(tj, r, tb, s, M, K, 2 * wk, nkt, x, bf, status)))         \
            return true;                                                                                           \
        if (M > LS_MAXR) return false;                                                                             \
        return rj ? launch_small_k2<CB_, K2_, true, false>(sj, r, nb, s, M, K, wk, nkt, x, bf, status)             \
                  : launch_small_k2<CB_, K2_, false, false>(sj, r, nb, s, M, K, wk, nkt, x, bf, status);           \
    }
    EA_SV(10, 2) EA_SV(8, 1) EA_SV(8, 2) EA_SV(6, 1) EA_SV(4, 1)
#undef EA_SV
    return false;
}

// the (K2, codebook) pairs this build instantiates: the reference's four (exl3.zig:40) and 3 / 4 bits mcg
template <int CB, int K2>
static void launch_wk(const ea_jobs& jobs, int blocks, hipStream_t s, int M, int K, int wk) {
    const dim3 grid((unsigned)blocks, (unsigned)((M + 15) / 16));  // passes of 16 rows side by side
    if (wk == 2) linear_kernel<CB, K2, 2><<<grid, 2 * 64, 0, s>>>(jobs, M, K);
    else if (wk == 4) linear_kernel<CB, K2, 4><<<grid, 4 * 64, 0, s>>>(jobs, M, K);
    else linear_kernel<CB, K2, 8><<<grid, 8 * 64, 0, s>>>(jobs, M, K);
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

// One linear launch over 1..3 jobs. rot: the jobs' rotation (suh, xh) when x is the unrotated input; then the
// small-row kernel rotates in-kernel, and otherwise a rotation launch runs first.
int launch_linear(hipStream_t s, const ea_jobs* jobs_in, uint32_t m, uint32_t kdim, uint32_t k2, uint32_t cb,
                  uint32_t wk, uint32_t loads, const ea_rot_jobs* rot = nullptr, const void* x = nullptr,
                  int x_dtype = 0) {
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
    if (launch_small(jobs, rot, s, (int)m, (int)kdim, k2, cb, (int)wk, x, x_dtype, c->status)) return launched();
    if (rot) {
        const int r = launch_lin_rot_in(s, x, x_dtype, rot, (uint32_t)jobs.n, m, kdim);
        if (r) return r;
    }
    launch_variant(jobs, blocks, s, (int)m, (int)kdim, k2, cb, (int)wk);
    return launched();
}

}  // namespace ea

using namespace ea;

extern "C" {

#ifdef EA_STAMPS
// The timeline build only: the stamp region of the linear kernels (ea_stamps.hpp).
int ea_stamps_attach_linear(void* region) { return stamp_attach(region); }
#endif

int ea_exl3_rot_in(ea_stream_t stream, const void* x, int x_dtype, const ea_rot_jobs* jobs, uint32_t njobs,
                   uint32_t m, uint32_t kdim) {
    return launch_lin_rot_in(as_stream(stream), x, x_dtype, jobs, njobs, m, kdim);
}

int ea_exl3_linear(ea_stream_t stream, const ea_jobs* jobs, uint32_t m, uint32_t kdim, uint32_t k2, uint32_t cb,
                   uint32_t wk, uint32_t loads) {
    return launch_linear(as_stream(stream), jobs, m, kdim, k2, cb, wk, loads);
}

// linear.zig:61-79 plan
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

// linear.zig:133-138 groupable
static bool groupable(const ea_linear* const* ls, uint32_t n) {
    if (!ls || n == 0 || n > EA_MAX_JOBS) return false;
    const ea_linear* a = ls[0];
    if (!a) return false;
    for (uint32_t i = 0; i < n; ++i)
        if (!ls[i] || ls[i]->k != a->k || ls[i]->k2 != a->k2 || ls[i]->cb != a->cb || ls[i]->wk != a->wk) return false;
    return true;
}

// the kernels' load options the engine uses: bits 1 and 2 (linear.zig:156-158; PDL has no counterpart here)
static const uint32_t LOADS = 3;

// linear.call / callRotated: jobs over the layers; rot and x given for call (the rotation then happens in the
// launch or just before it).
static int linear_call_jobs(hipStream_t stream, const ea_linear_scratch* s, const ea_linear* const* ls, uint32_t nls,
                            uint32_t m, const uint64_t* outs, const int* out_dtypes, const ea_rot_jobs* rot,
                            const void* x, int x_dtype) {
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
    return launch_linear(stream, &jobs, m, ls[0]->k, ls[0]->k2, ls[0]->cb, ls[0]->wk, LOADS, rot, x, x_dtype);
}

int ea_linear_call_rotated(ea_stream_t stream, const ea_linear_scratch* s, const ea_linear* const* ls, uint32_t nls,
                           uint32_t m, const uint64_t* outs, const int* out_dtypes) {
    return linear_call_jobs(as_stream(stream), s, ls, nls, m, outs, out_dtypes, nullptr, nullptr, 0);
}

int ea_linear_call(ea_stream_t stream, const ea_linear_scratch* s, const ea_linear* const* ls, uint32_t nls,
                   const void* x, int x_dtype, uint32_t m, const uint64_t* outs, const int* out_dtypes) {
    if (!groupable(ls, nls) || m < 1 || m > 128) return EA_NOT_GROUPABLE;
    if (!s) return EA_BAD_ARGUMENT;
    if (ls[0]->k % 128 != 0) return EA_BAD_ROT_IN;
    if (!x || x_dtype < 0 || x_dtype > 2) return EA_BAD_ARGUMENT;
    ea_rot_jobs rj{};
    for (uint32_t i = 0; i < nls; ++i) {
        rj.suh[i] = ls[i]->suh;
        rj.xh[i] = s->xh[i];
    }
    return linear_call_jobs(as_stream(stream), s, ls, nls, m, outs, out_dtypes, &rj, x, x_dtype);
}

}  // extern "C"
