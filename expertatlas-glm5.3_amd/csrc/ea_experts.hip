// Routed experts, decode path: grouping, per-pair input rotation, the grouped EXL3 GEMV on MFMA, the gate/up
// epilogue (FWHT, svh, SwiGLU, suh_d, FWHT) and the down epilogue with the slot-ordered combine.
//
// Semantics follow exl3_experts.cu / experts_grouped.cuh of the reference; the work decomposition is this
// build's own: wave64 lanes decode trellis values straight into v_mfma_f32_16x16x32_f16 B operands (see
// ea_device.hpp: mfma_lane_p0), and the wavefronts of a block split the K range and are summed in wave order.
#include <hip/hip_runtime.h>

#include "ea_device.hpp"
#include "ea_experts.hpp"
#include "ea_gemm.hpp"
#include "ea_host.hpp"

namespace ea {

// ---- grouping ---------------------------------------------------------------------------------------------------
constexpr int GROUP_THREADS = 1024;
constexpr int GROUP_MAXE = 4096;  // experts the presence bitmap holds (experts.zig:99)

// The number of lanes below this one: the lane's place among the set bits of a ballot.
__device__ __forceinline__ int lanes_below(uint64_t mask) {
    return (int)__builtin_amdgcn_mbcnt_hi((uint32_t)(mask >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)mask, 0u));
}

// Exclusive prefix sum over the wave of a value below 2^bits, one ballot a bit: a lane's sum is, for every bit, the
// count of lower lanes with that bit set, times the bit's weight. Every lane gets its own prefix; `total` the sum.
template <int BITS>
__device__ __forceinline__ int wave_prefix(int v, int& total) {
    int below = 0, all = 0;
#pragma unroll
    for (int b = 0; b < BITS; ++b) {
        const uint64_t m = __builtin_amdgcn_ballot_w64((v >> b) & 1);
        below += lanes_below(m) << b;
        all += __builtin_popcountll(m) << b;
    }
    total = all;
    return below;
}

// The distinct picked experts (< E) in id order, and each one's first maxm picks in pick order as row * 32 + slot,
// -1 after its last (the grouping of exl3_experts.cu:36-90, a different decomposition):
//   1. every pick sets its expert's bit in an LDS presence bitmap (E <= 4096: 128 words);
//   2. wave 0 numbers the units: lane l owns bitmap words 2l, 2l + 1; its first unit is the count of set bits in the
//      lower lanes' words (a bit-sliced ballot prefix), and it lists its experts in bit order;
//   3. a wave a unit streams the picks 64 at a time: a ballot of the picks naming the unit's expert gives each
//      match its place (the matches before it in this batch plus all earlier batches), until maxm are placed.
__global__ void __launch_bounds__(GROUP_THREADS) group_kernel(const int* __restrict__ pick, int* __restrict__ uids,
                                                              int* __restrict__ ucount, int* __restrict__ members,
                                                              int R, int slots, int E, int maxm) {
    extern __shared__ int s_pick[];
    __shared__ uint32_t s_present[GROUP_MAXE / 32];
    __shared__ int16_t s_expert[GROUP_MAXE];  // unit -> expert
    __shared__ int s_units;
    const int n = R * slots, t = threadIdx.x, lane = t & 63, wave = t >> 6;
    for (int w = t; w < GROUP_MAXE / 32; w += GROUP_THREADS) s_present[w] = 0u;
    __syncthreads();
    for (int i = t; i < n; i += GROUP_THREADS) {
        const int e = pick[i];
        s_pick[i] = e;
        if (e >= 0 && e < E) atomicOr(&s_present[e >> 5], 1u << (e & 31));
    }
    __syncthreads();
    if (wave == 0) {
        const uint32_t w0 = s_present[2 * lane], w1 = s_present[2 * lane + 1];
        int total = 0;
        int u = wave_prefix<7>(__builtin_popcount(w0) + __builtin_popcount(w1), total);  // <= 64 a lane
        const uint64_t bits = (uint64_t)w0 | ((uint64_t)w1 << 32);
        for (uint64_t b = bits; b; b &= b - 1) {
            const int e = 64 * lane + (int)__builtin_ctzll(b);
            s_expert[u] = (int16_t)e;
            uids[u++] = e;
        }
        if (lane == 0) {
            s_units = total;
            ucount[0] = total;
        }
    }
    __syncthreads();
    const int units = s_units;
    for (int u = wave; u < units; u += GROUP_THREADS / 64) {
        const int e = s_expert[u];
        int* mem = members + (size_t)u * maxm;
        int placed = 0;
        for (int c = 0; c < n && placed < maxm; c += 64) {
            const int i = c + lane;
            const bool hit = i < n && s_pick[i] == e;
            const uint64_t m = __builtin_amdgcn_ballot_w64(hit);
            const int at = placed + lanes_below(m);
            if (hit && at < maxm) mem[at] = (i / slots) * 32 + (i % slots);
            placed += __builtin_popcountll(m);
        }
        for (int j = (placed < maxm ? placed : maxm) + lane; j < maxm; j += 64) mem[j] = -1;
    }
}

// ---- per-pair input rotation ------------------------------------------------------------------------------------
// Block (row, matrix, 2048 columns of K): 16 lanes a 128-block, lane l holding its values 8 h8_group(l) .. +7; the
// row's activations are read once and rotated for each of its slots in turn. out[p] = fp16((x[row] * suh[e]) @ H *
// HAD_SCALE) for each pair p of the row with an expert (exl3_experts.cu:116-134). The butterflies run over value-index
// bits 0..6 in that order (three inside a lane, four across lanes: fwht128_x8), as in a one-lane-pair-a-value layout,
// so each output is the same fp32 sum rounded the same way. With `zero`, the matrix-0 blocks also clear the row's values
// k .. k + 7 of zero [rows, K] (fp32, or fp16 with zero_half): the output that a prefill pass without a pair plane
// adds its slots into.
__global__ void __launch_bounds__(256) rot_in_kernel(const void* __restrict__ x, int x_dtype, int x_stride,
                                                     const int* __restrict__ pick, const uint16_t* __restrict__ suh0,
                                                     const uint16_t* __restrict__ suh1, uint16_t* __restrict__ out0,
                                                     uint16_t* __restrict__ out1, int K, int slots, int E, int vec,
                                                     void* __restrict__ zero, int zero_half) {
    const int row = blockIdx.x, mat = blockIdx.y, lane = threadIdx.x & 63;
    const int k = blockIdx.z * 2048 + 128 * ((int)threadIdx.x >> 4) + 8 * h8_group(lane);
    if (k >= K) return;  // whole 16-lane groups (K % 128 == 0)
    if (zero && mat == 0) {
        const bool al = (reinterpret_cast<uintptr_t>(zero) & 15) == 0;  // uniform; K % 128 == 0 keeps rows aligned
        if (zero_half) {
            uint16_t* z = static_cast<uint16_t*>(zero) + (size_t)row * K + k;
            if (al)
                *reinterpret_cast<u4v*>(z) = u4v{0u, 0u, 0u, 0u};
            else
#pragma unroll
                for (int j = 0; j < 8; ++j) z[j] = 0;
        } else {
            float* z = static_cast<float*>(zero) + (size_t)row * K + k;
            if (al) {
                *reinterpret_cast<f4v*>(z) = f4v{0.f, 0.f, 0.f, 0.f};
                *reinterpret_cast<f4v*>(z + 4) = f4v{0.f, 0.f, 0.f, 0.f};
            } else {
#pragma unroll
                for (int j = 0; j < 8; ++j) z[j] = 0.f;
            }
        }
    }
    const uint16_t* suh = mat ? suh1 : suh0;
    uint16_t* out = mat ? out1 : out0;
    const size_t xr = (size_t)row * x_stride;
    float xv[8];
    if (vec) {  // 16-byte aligned rows
        if (x_dtype == F32) {
            const f4v a = *reinterpret_cast<const f4v*>(static_cast<const float*>(x) + xr + k);
            const f4v b = *reinterpret_cast<const f4v*>(static_cast<const float*>(x) + xr + k + 4);
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                xv[j] = a[j];
                xv[4 + j] = b[j];
            }
        } else {
            const u4v w = *reinterpret_cast<const u4v*>(static_cast<const uint16_t*>(x) + xr + k);
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const uint16_t h = (uint16_t)(w[j >> 1] >> (16 * (j & 1)));
                xv[j] = x_dtype == BF16 ? bf2f(h) : h2f(h);
            }
        }
    } else {
#pragma unroll
        for (int j = 0; j < 8; ++j) xv[j] = load_act(x, x_dtype, xr + k + j);
    }
    // eight slots at a time: their picks, then all their suh loads in flight before the first rotation (a slot
    // without an expert loads expert 0's and is skipped)
    constexpr int QB = 8;
    for (int q0 = 0; q0 < slots; q0 += QB) {
        int ev[QB];
        u4v sw[QB];
#pragma unroll
        for (int j = 0; j < QB; ++j) {
            const int q = q0 + j < slots ? q0 + j : q0;
            const int e = pick[row * slots + q];
            ev[j] = q0 + j < slots && e >= 0 && e < E ? e : -1;
        }
#pragma unroll
        for (int j = 0; j < QB; ++j)
            sw[j] = *reinterpret_cast<const u4v*>(suh + (size_t)(ev[j] >= 0 ? ev[j] : 0) * K + k);
        issued();
#pragma unroll
        for (int j = 0; j < QB; ++j) {
            if (ev[j] < 0) continue;  // uniform over the block
            float v[8];
#pragma unroll
            for (int i = 0; i < 8; ++i) v[i] = xv[i] * h2f((uint16_t)(sw[j][i >> 1] >> (16 * (i & 1))));
            const float sc = fwht128_x8(v, lane) * HAD_SCALE;  // the values' sign folded into the scale (exact)
            u4v w;
#pragma unroll
            for (int i = 0; i < 4; ++i)
                w[i] = f2h2(__builtin_fmaf(v[2 * i], sc, 0.f), __builtin_fmaf(v[2 * i + 1], sc, 0.f));
            *reinterpret_cast<u4v*>(out + (size_t)(row * slots + q0 + j) * K + k) = w;
        }
    }
}

// Block (expert u, n block of NTW tiles, (matrix, split, member tile)): NW waves split the split's k tiles in
// equal consecutive ranges, their partial sums added in wave order into Z[mat][split][pair][n]
// (experts_grouped.cuh:214-313). K2 comes from the expert's table entry at run time.
template <int CB, int LO, int HI, int NTW, int NW>
__global__ void __launch_bounds__(NW * 64) grouped_kernel(
    const uint16_t* __restrict__ X0, const uint16_t* __restrict__ X1, const int64_t* __restrict__ TP0,
    const int64_t* __restrict__ TP1, const int* __restrict__ K2_0, const int* __restrict__ K2_1,
    const int* __restrict__ uids, const int* __restrict__ ucount, const int* __restrict__ members,
    float* __restrict__ Z, int K, int N, int P, int SK, int maxm, int slots, int NS, int* __restrict__ status) {
    const int u = blockIdx.x;
    if (u >= ucount[0]) return;
    const int MT = (maxm + 15) / 16;
    const int mtile = blockIdx.z % MT;
    const int split = (blockIdx.z / MT) % SK;
    const int mat = blockIdx.z / MT / SK;
    const uint16_t* X = mat ? X1 : X0;
    const int e = uids[u];
    const uint32_t* T = reinterpret_cast<const uint32_t*>(mat ? TP1[e] : TP0[e]);
    const int k2 = mat ? K2_1[e] : K2_0[e];
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int KT = K >> 4, ns = NS > 0 ? NS : (N >> 4);

    __shared__ int rows_sh[16];
    if (threadIdx.x < 16) {
        const int m = mtile * 16 + threadIdx.x;
        const int code = m < maxm ? members[u * maxm + m] : -1;
        rows_sh[threadIdx.x] = code >= 0 ? (code >> 5) * slots + (code & 31) : -1;
    }
    __syncthreads();
    if (rows_sh[0] < 0) return;  // members are packed first: this member tile is empty
    const int r = rows_sh[lane & 15];
    const uint16_t* const xrow[1] = {r >= 0 ? X + (size_t)r * K : nullptr};

    const int per_split = KT / SK, per_wave = per_split / NW;
    const int kt0 = split * per_split + wave * per_wave;
    const int nt0 = blockIdx.y * NTW;

    f4v acc[1][NTW];
#pragma unroll
    for (int j = 0; j < NTW; ++j) acc[0][j] = f4v{0.f, 0.f, 0.f, 0.f};

    const uint32_t* base = T + ((size_t)kt0 * ns + nt0) * 4 * k2;
    const bool ok = EA_K2_SWITCH(k2, LO, HI,
                                 (wave_tiles<CB, K2V, NTW, 1>(base, (size_t)ns * 4 * K2V, per_wave, kt0 * 16, xrow,
                                                              lane, acc)));
    if (!ok) {
        if (threadIdx.x == 0) record_error(status, DEV_UNSUPPORTED_WIDTH);
#pragma unroll
        for (int j = 0; j < NTW; ++j) acc[0][j] = nan4();
    }

    // wave partials through LDS, added in wave order; lane l holds D[4 (l >> 4) + i][l & 15] of each tile
    __shared__ float red[NW][16][NTW * 16];
#pragma unroll
    for (int j = 0; j < NTW; ++j)
#pragma unroll
        for (int i = 0; i < 4; ++i) red[wave][4 * (lane >> 4) + i][j * 16 + (lane & 15)] = acc[0][j][i];
    __syncthreads();
    for (int idx = threadIdx.x; idx < 16 * NTW * 16; idx += NW * 64) {
        const int row = idx / (NTW * 16), col = idx % (NTW * 16);
        const int rr = rows_sh[row];
        if (rr < 0) continue;
        float s = red[0][row][col];
#pragma unroll
        for (int w = 1; w < NW; ++w) s += red[w][row][col];
        Z[(((size_t)mat * SK + split) * P + rr) * N + nt0 * 16 + col] = s;
    }
}

// ---- gate/up epilogue -----------------------------------------------------------------------------------------
// Wave (pair p, 128-block): splits summed in order, FWHT, * HAD_SCALE * svh, SwiGLU (act_mode 0: bf16 roundings,
// 1: fp32; limit clamps), * suh_d, FWHT, xd = fp16(* HAD_SCALE) (exl3_experts.cu:142-184). A pair marked in pclass
// takes its splits from Z's split 0 and Zp's planes ([SKP - 1][2][P][N]), in split order. With only >= 0 a pair
// whose class (pclass[p] != 0) is not `only` is left alone.
constexpr int EPI_SPLITS = 4;  // K splits whose loads the gate / up epilogue issues together (more: in turn)
__global__ void __launch_bounds__(64) gateup_epilogue_kernel(const float* __restrict__ Z, const int* __restrict__ pick,
                                                             const uint16_t* __restrict__ svh_g,
                                                             const uint16_t* __restrict__ svh_u,
                                                             const uint16_t* __restrict__ suh_d,
                                                             uint16_t* __restrict__ xd, int P, int N, int SK, int E,
                                                             float limit, int act_mode, const int* __restrict__ pclass,
                                                             const float* __restrict__ Zp, int SKP, int only) {
    const int p = blockIdx.x, blk = blockIdx.y, lane = threadIdx.x;
    const int e = pick[p];
    if (e < 0 || e >= E) return;
    const int n = blk * 128 + 2 * lane;
    const bool part = pclass && pclass[p];
    if (only >= 0 && (int)part != only) return;
    const int ns = part ? SKP : SK;
    const size_t mstride = part ? (size_t)P * N : (size_t)SK * P * N;
    auto split = [&](int s) __attribute__((always_inline)) {
        return (part ? (s ? Zp + (size_t)(s - 1) * 2 * P * N : Z) : Z + (size_t)s * P * N) + (size_t)p * N + n;
    };
    // the scales and every split's gate and up values (8-byte loads: a lane's two columns) are all in flight before
    // the first is used; a loop that loaded a split after adding the previous one waited for each in turn
    const size_t at = (size_t)e * N + n;
    const uint32_t sg2 = *reinterpret_cast<const uint32_t*>(svh_g + at);
    const uint32_t su2 = *reinterpret_cast<const uint32_t*>(svh_u + at);
    const uint32_t sd2 = *reinterpret_cast<const uint32_t*>(suh_d + at);
    float g[2] = {0.f, 0.f}, u[2] = {0.f, 0.f};
    if (ns <= EPI_SPLITS) {
        float2 zg[EPI_SPLITS], zu[EPI_SPLITS];
#pragma unroll
        for (int s = 0; s < EPI_SPLITS; ++s)
            if (s < ns) {
                zg[s] = *reinterpret_cast<const float2*>(split(s));
                zu[s] = *reinterpret_cast<const float2*>(split(s) + mstride);
            }
#pragma unroll
        for (int s = 0; s < EPI_SPLITS; ++s)
            if (s < ns) {  // the splits in order from zero
                g[0] += zg[s].x;
                g[1] += zg[s].y;
                u[0] += zu[s].x;
                u[1] += zu[s].y;
            }
    } else {
        for (int s = 0; s < ns; ++s) {
            const float2 zg = *reinterpret_cast<const float2*>(split(s));
            const float2 zu = *reinterpret_cast<const float2*>(split(s) + mstride);
            g[0] += zg.x;
            g[1] += zg.y;
            u[0] += zu.x;
            u[1] += zu.y;
        }
    }
    fwht128_w64(g[0], g[1], lane);
    fwht128_w64(u[0], u[1], lane);
    float v[2];
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        const float svg = h2f((uint16_t)(sg2 >> (16 * j))), svu = h2f((uint16_t)(su2 >> (16 * j)));
        float act;
        if (act_mode == 0) {
            const float gg = fminf(bf16r(g[j] * HAD_SCALE * svg), limit);
            const float uu = fminf(fmaxf(bf16r(u[j] * HAD_SCALE * svu), -limit), limit);
            act = bf16r(bf16r(gg / (1.f + expf_path(-gg))) * uu);
        } else {
            const float gg = fminf(g[j] * HAD_SCALE * svg, limit);
            const float uu = fminf(fmaxf(u[j] * HAD_SCALE * svu, -limit), limit);
            act = gg / (1.f + expf_path(-gg)) * uu;
        }
        v[j] = act * h2f((uint16_t)(sd2 >> (16 * j)));
    }
    fwht128_w64(v[0], v[1], lane);
    *reinterpret_cast<uint32_t*>(xd + (size_t)p * N + n) =
        (uint32_t)f2h(v[0] * HAD_SCALE) | ((uint32_t)f2h(v[1] * HAD_SCALE) << 16);
}

// ---- down epilogue + combine ----------------------------------------------------------------------------------
// Block (row r, 128-block): wave w does slots w, w + NWV, ..: y[p] = FWHT(sum of splits) * HAD_SCALE * svh_d (a slot
// whose pick is not an expert reads y as it is); then out[r] = fma chain over the slots in order from 0
// (exl3_experts.cu:223-268).
constexpr int DC_WAVES = 8;
__global__ void __launch_bounds__(DC_WAVES * 64) down_combine_kernel(
    const float* __restrict__ Z, const int* __restrict__ pick, const uint16_t* __restrict__ svh_d, float* __restrict__ y,
    const float* __restrict__ wts, float* __restrict__ out, int P, int D, int SK, int E, int slots, int skip_invalid) {
    __shared__ float part[32][128];
    const int r = blockIdx.x, blk = blockIdx.y;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int n = blk * 128 + 2 * lane;
    for (int k = wave; k < slots; k += DC_WAVES) {
        const int p = r * slots + k;
        const int e = pick[p];
        float o[2];
        if (e >= 0 && e < E) {
            float v[2];
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                float s = 0.f;
                for (int q = 0; q < SK; ++q) s += Z[((size_t)q * P + p) * D + n + j];
                v[j] = s;
            }
            fwht128_w64(v[0], v[1], lane);
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                o[j] = v[j] * HAD_SCALE * h2f(svh_d[(size_t)e * D + n + j]);
                y[(size_t)p * D + n + j] = o[j];
            }
        } else if (skip_invalid) {
            o[0] = o[1] = 0.f;
        } else {
#pragma unroll
            for (int j = 0; j < 2; ++j) o[j] = y[(size_t)p * D + n + j];
        }
        part[k][2 * lane] = o[0];
        part[k][2 * lane + 1] = o[1];
    }
    __syncthreads();
    if (wave != 0) return;
    float a0 = 0.f, a1 = 0.f;
    for (int q = 0; q < slots; ++q) {
        const float w = wts[r * slots + q];
        a0 = __builtin_fmaf(w, part[q][2 * lane], a0);
        a1 = __builtin_fmaf(w, part[q][2 * lane + 1], a1);
    }
    out[(size_t)r * D + n] = a0;
    out[(size_t)r * D + n + 1] = a1;
}

// ---- launchers --------------------------------------------------------------------------------------------------

int launch_group(hipStream_t s, const int* pick, int* uids, int* ucount, int* members, uint32_t rows, uint32_t slots,
                 uint32_t experts, uint32_t maxm) {
    EA_REQUIRE_CTX(c);
    if (experts > GROUP_MAXE) return EA_TOO_MANY_EXPERTS;
    if (slots > 32) return EA_TOO_MANY_SLOTS;
    const size_t smem = (size_t)rows * slots * 4;
    // the picks, the presence bitmap, the unit -> expert table and the unit count in LDS
    if (smem + GROUP_MAXE / 8 + GROUP_MAXE * 2 + 4 > c->lds_optin) return EA_GROUP_SHARED_MEMORY;
    if (!pick || !uids || !ucount || !members) return EA_BAD_ARGUMENT;
    group_kernel<<<1, GROUP_THREADS, smem, s>>>(pick, uids, ucount, members, (int)rows, (int)slots, (int)experts,
                                                (int)maxm);
    return launched();
}

int launch_rot_in(hipStream_t s, const void* x, int x_dtype, uint32_t x_stride, const int* pick, const uint16_t* suh0,
                  const uint16_t* suh1, uint16_t* out0, uint16_t* out1, uint32_t rows, uint32_t kdim, uint32_t slots,
                  uint32_t experts, void* zero, int zero_half) {
    EA_REQUIRE_CTX(c);
    if (kdim % 128 != 0) return EA_BAD_ROT_IN;
    if (x_dtype < 0 || x_dtype > 2 || !x || !pick) return EA_BAD_ARGUMENT;
    if (rows * slots == 0) return EA_OK;
    const size_t eb = x_dtype == F32 ? 4 : 2;
    const int vec = (reinterpret_cast<uintptr_t>(x) & 15) == 0 && ((size_t)x_stride * eb) % 16 == 0;
    dim3 grid(rows, 2, (kdim + 2047) / 2048);
    rot_in_kernel<<<grid, 256, 0, s>>>(x, x_dtype, (int)x_stride, pick, suh0, suh1, out0, out1, (int)kdim,
                                       (int)slots, (int)experts, vec, zero, zero_half);
    return launched();
}

template <int CB, int LO, int HI>
static void grouped_dispatch(const ea_grouped_args& a, hipStream_t s, int nw, int ntw, int* status) {
    const int MT = (a.maxm + 15) / 16;
    dim3 grid(a.nexp_max, a.N / (16 * ntw), a.mats * a.SK * MT);
    auto X0 = dptr<const uint16_t>(a.x0);
    auto X1 = dptr<const uint16_t>(a.x1);
    auto TP0 = dptr<const int64_t>(a.tp0);
    auto TP1 = dptr<const int64_t>(a.tp1);
    auto B0 = dptr<const int>(a.k2_0);
    auto B1 = dptr<const int>(a.k2_1);
    auto U = dptr<const int>(a.uids);
    auto UC = dptr<const int>(a.ucount);
    auto M = dptr<const int>(a.members);
    auto Zp = dptr<float>(a.z);
#define EA_GL(NTW_, NW_)                                                                                          \
    grouped_kernel<CB, LO, HI, NTW_, NW_><<<grid, NW_ * 64, 0, s>>>(X0, X1, TP0, TP1, B0, B1, U, UC, M, Zp,      \
                                                                   (int)a.K, (int)a.N, (int)a.P, (int)a.SK,      \
                                                                   (int)a.maxm, (int)a.slots, (int)a.ns, status)
#define EA_GL_NW(NTW_)                 \
    if (nw == 8) EA_GL(NTW_, 8);       \
    else if (nw == 4) EA_GL(NTW_, 4);  \
    else if (nw == 2) EA_GL(NTW_, 2);  \
    else EA_GL(NTW_, 1);
    if (ntw == 4) {
        EA_GL_NW(4)
    } else if (ntw == 2) {
        EA_GL_NW(2)
    } else {
        EA_GL_NW(1)
    }
#undef EA_GL_NW
#undef EA_GL
}

int launch_grouped(hipStream_t s, const ea_grouped_args& a) {
    EA_REQUIRE_CTX(c);
    // the reference's launch checks (experts.zig:141-148)
    if (a.warps == 0 || a.nt == 0 || a.SK == 0 || a.K % (16 * a.SK * a.warps) != 0 || a.N % (16 * a.nt) != 0)
        return EA_UNEVEN_SPLIT;
    if (a.ns != 0 && a.ns < a.N / 16) return EA_BAD_ROW_STRIDE;
    if (a.cb > 2 || a.mats < 1 || a.mats > 2) return EA_UNPORTED_GROUPED_VARIANT;
    // the K2 ranges: [8, 8], else [2, 10], else [2, 16] (experts.zig:143-145)
    const bool only8 = a.lo == 8 && a.hi == 8;
    const bool to10 = a.lo >= 2 && a.hi <= 10;
    if (a.lo < 2 || a.hi > 16) return EA_UNPORTED_GROUPED_VARIANT;
    if (!a.x0 || !a.x1 || !a.tp0 || !a.tp1 || !a.k2_0 || !a.k2_1 || !a.uids || !a.ucount || !a.members || !a.z)
        return EA_BAD_ARGUMENT;
    if (a.nexp_max == 0 || a.maxm == 0) return EA_OK;
    // this build's tiling: NTW n tiles a wave, NW waves a block splitting the split's k tiles into equal ranges
    const uint32_t nt16 = a.N / 16, per_split = a.K / 16 / a.SK;
    const int ntw = nt16 % 4 == 0 ? 4 : (nt16 % 2 == 0 ? 2 : 1);
    int nw = 1;
    for (int cand : {8, 4, 2})
        if (per_split % cand == 0 && per_split / cand >= 2) {
            nw = cand;
            break;
        }
    if (a.cb == 1) {
        if (only8) grouped_dispatch<1, 8, 8>(a, s, nw, ntw, c->status);
        else if (to10) grouped_dispatch<1, 2, 10>(a, s, nw, ntw, c->status);
        else grouped_dispatch<1, 2, 16>(a, s, nw, ntw, c->status);
    } else if (a.cb == 2) {
        grouped_dispatch<2, 2, 16>(a, s, nw, ntw, c->status);
    } else {
        grouped_dispatch<0, 2, 16>(a, s, nw, ntw, c->status);
    }
    return launched();
}

int launch_gateup_epilogue(hipStream_t s, const float* z, const int* pick, const uint16_t* svh_g,
                           const uint16_t* svh_u, const uint16_t* suh_d, uint16_t* xd, uint32_t rows, uint32_t p,
                           uint32_t n, uint32_t sk, uint32_t slots, uint32_t experts, float limit, uint32_t act_mode,
                           const int* pclass, const float* zp, uint32_t skp, int only) {
    EA_REQUIRE_CTX(c);
    if (n % 128 != 0) return EA_BAD_WIDTH;
    if (!z || !pick || !svh_g || !svh_u || !suh_d || !xd) return EA_BAD_ARGUMENT;
    if (rows * slots == 0 || n == 0) return EA_OK;
    dim3 grid(rows * slots, n / 128);
    gateup_epilogue_kernel<<<grid, 64, 0, s>>>(z, pick, svh_g, svh_u, suh_d, xd, (int)p, (int)n, (int)sk,
                                               (int)experts, limit, (int)act_mode, pclass, zp, (int)skp, only);
    return launched();
}

int launch_down_combine(hipStream_t s, const float* z, const int* pick, const uint16_t* svh_d, float* y,
                        const float* wts, float* out, uint32_t rows, uint32_t p, uint32_t d, uint32_t sk,
                        uint32_t slots, uint32_t experts, bool skip_invalid) {
    EA_REQUIRE_CTX(c);
    if (slots > 32) return EA_TOO_MANY_SLOTS;
    if (d % 128 != 0) return EA_BAD_WIDTH;
    if (!z || !pick || !svh_d || !y || !wts || !out) return EA_BAD_ARGUMENT;
    if (rows == 0 || d == 0) return EA_OK;
    dim3 grid(rows, d / 128);
    down_combine_kernel<<<grid, DC_WAVES * 64, 0, s>>>(z, pick, svh_d, y, wts, out, (int)p, (int)d, (int)sk,
                                                       (int)experts, (int)slots, skip_invalid ? 1 : 0);
    return launched();
}

}  // namespace ea

using namespace ea;

extern "C" {

int ea_experts_group(ea_stream_t stream, const int32_t* pick, int32_t* uids, int32_t* ucount, int32_t* members,
                     uint32_t rows, uint32_t slots, uint32_t experts, uint32_t maxm) {
    return launch_group(as_stream(stream), pick, uids, ucount, members, rows, slots, experts, maxm);
}

int ea_experts_rot_in(ea_stream_t stream, const void* x, int x_dtype, uint32_t x_stride, const int32_t* pick,
                      const void* suh0, const void* suh1, void* out0, void* out1, uint32_t rows, uint32_t kdim,
                      uint32_t slots, uint32_t experts) {
    return launch_rot_in(as_stream(stream), x, x_dtype, x_stride, pick, static_cast<const uint16_t*>(suh0),
                         static_cast<const uint16_t*>(suh1), static_cast<uint16_t*>(out0),
                         static_cast<uint16_t*>(out1), rows, kdim, slots, experts);
}

int ea_experts_grouped(ea_stream_t stream, const ea_grouped_args* a) {
    if (!a) return EA_BAD_ARGUMENT;
    return launch_grouped(as_stream(stream), *a);
}

int ea_experts_gateup_epilogue(ea_stream_t stream, const float* z, const int32_t* pick, const void* svh_g,
                               const void* svh_u, const void* suh_d, void* xd, uint32_t rows, uint32_t p, uint32_t n,
                               uint32_t sk, uint32_t slots, uint32_t experts, float limit, uint32_t act_mode) {
    return launch_gateup_epilogue(as_stream(stream), z, pick, static_cast<const uint16_t*>(svh_g),
                                  static_cast<const uint16_t*>(svh_u), static_cast<const uint16_t*>(suh_d),
                                  static_cast<uint16_t*>(xd), rows, p, n, sk, slots, experts, limit, act_mode);
}

int ea_experts_down_combine(ea_stream_t stream, const float* z, const int32_t* pick, const void* svh_d, float* y,
                            const float* wts, float* out, uint32_t rows, uint32_t p, uint32_t d, uint32_t sk,
                            uint32_t slots, uint32_t experts) {
    return launch_down_combine(as_stream(stream), z, pick, static_cast<const uint16_t*>(svh_d), y, wts, out, rows, p,
                               d, sk, slots, experts);
}

}  // extern "C"
