// One decode window's MoE FFN (R <= 16 rows, top-8) in a few launches, each boundary carrying one dependency and no
// block ever waiting on, or counting with, another:
//   route (more than one row): one block computes the router top-8 of every row and the grouping, and publishes
//     them; with one row every gate|up block routes the row itself (in LDS) instead, which costs less than a launch.
//   gate|up: every block works through its share of the (unit, column block, matrix, k chunk) items, a unit being a
//     distinct routed expert or the shared expert. An item issues all of its trellis loads before it rotates its
//     activations, multiplies on MFMA and stores its partial sums.
//   epilogue (more than one row): a block per (unit, column block, group of members) sums the chunks in order and
//     runs FWHT, SwiGLU and FWHT into the members' down inputs; with one row the down launch does this itself.
//   down: a block per (unit, column blocks of 128 outputs): the pair's (or the shared expert's) output rows.
//   combine: out = the slots in order from 0 (+ the shared expert).
// In-launch hand-offs between blocks were measured slower: a release fence writes back the XCD's whole L2, and
// polling blocks saturate the memory channel of the flag they poll.
//
// Reference semantics: moe.routed (moe.zig:279-293; exl3_experts.cu:36-268), the shared expert's mlp
// (forward.zig:2328-2341: EXL3 linears with bf16 outputs, swiglu2, the down linear), the router top-8
// (native_ops.cu:1015-1068) and ffnMain's add (forward.zig:2401-2403). Partial sums are added in chunk order and the
// slots in slot order, so the output bits do not depend on timing.
#include <hip/hip_runtime.h>

#include "ea_device.hpp"
#include "ea_experts.hpp"
#include "ea_gemm.hpp"
#include "ea_host.hpp"

namespace ea {

constexpr int DL_THREADS = 256;
constexpr int DL_WAVES = DL_THREADS / 64;
constexpr int DL_MAXR = 16;                  // rows of a window (one MFMA row tile)
constexpr int DL_SLOTS = 8;                  // picks a row
constexpr int DL_MAXP = DL_MAXR * DL_SLOTS;  // pairs
constexpr int DL_MAXE = 1024;                // experts the LDS grouping holds
constexpr int DL_KT = 16;                    // k tiles of a gate|up item: 256 k, two Hadamard blocks
constexpr int DL_MAXI = 256;                 // widest rank-local intermediate (I) the LDS layout holds
constexpr int DL_RS = 264;                   // LDS row stride of the staged activations, halves
constexpr int DL_MAXKC = 24;                 // k chunks of 256 (D up to 6144)
constexpr int DL_MAXK2 = STAGE_MAXK2;        // widest trellis (K2) the decode layer runs
constexpr int DL_STAGE_WORDS = DL_KT * 2 * 4 * DL_MAXK2;  // a wave's staged trellis words: 16 rows of 2 tiles
constexpr int L1_LINE = 32;                  // ints between two of the one-row launch's counters (a 128-byte line)
constexpr size_t L1_SYNC_BYTES = 16384;      // the one-row launch's counters

// Scratch of the layer's launches, carved on the host for the scratch's row capacity (any R up to it runs).
struct DLLayout {
    int* sync;          // the one-row launch's counters (first in the region; zero between launches)
    float* zp;          // [Q, NH, 2, KC, 128] gate|up partial sums, Q = pairs + rows (the shared expert's rows last)
    uint16_t* xd;       // [Q, I] down inputs
    float* sy;          // [rows, D] the shared expert's output
    int* uids;          // [DL_MAXP] routed unit -> expert
    int* ucount;        // [1] routed units
    int* members;       // [DL_MAXP, DL_MAXR] pair ids of a routed unit, ascending
    int* mcount;        // [DL_MAXP]
    uint64_t* tptr;     // [DL_MAXP, 3] a routed unit's gate, up and down trellis addresses
    int* tk2;           // [DL_MAXP, 3] and widths
};

struct DLArgs {
    const float* logits;  // [R, 256] or null: pick / wts are then inputs
    const void* router_w; // bf16 [256, D] or null: when given, a router launch first writes the logits (host side only)
    const float* bias;
    float scale;
    int32_t* pick;
    float* wts;
    const void* x;
    int x_dtype, x_stride;
    const int64_t* ptr[3];
    const int32_t* k2t[3];
    const uint16_t *suh_g, *suh_u, *svh_g, *svh_u, *suh_d, *svh_d;
    int E;
    int hs, sh_k2;            // hs: 1 with a shared expert (unit 0)
    const uint32_t* sh_w[3];  // shared gate, up, down words (strips layout)
    const uint16_t* sh_suh[3];
    const uint16_t* sh_svh[3];
    float* out;
    float* yroute;  // [P, D] routed per-pair down outputs (read as they are for slots without an expert)
    DLLayout lay;
    int R, D, I, U;  // U: units the launch grids cover (hs + min(P, E))
    int* status;
};

// ---- the router and the grouping, per block ------------------------------------------------------------------------

// The largest (MAX) or smallest key over the wavefront, in every lane: DPP within rows of 16 (quad swaps, rotations
// by 4 and 8), then row broadcasts 15 and 31 leave the result in lane 63. Integer compares fold into the DPP moves.
template <int CTRL, int ROW_MASK, bool MAX>
__device__ __forceinline__ uint32_t dpp_step(uint32_t x) {
    // lanes of a masked row read the identity, so the compare folds into one DPP instruction
    constexpr int ID = MAX ? 0 : -1;
    const uint32_t y = (uint32_t)__builtin_amdgcn_update_dpp(ID, (int)x, CTRL, ROW_MASK, 0xf, false);
    return MAX ? (x > y ? x : y) : (x < y ? x : y);
}
template <bool MAX>
__device__ __forceinline__ uint32_t wave_reduce(uint32_t v) {
    v = dpp_step<0xB1, 0xf, MAX>(v);   // quad_perm (1, 0, 3, 2)
    v = dpp_step<0x4E, 0xf, MAX>(v);   // quad_perm (2, 3, 0, 1)
    v = dpp_step<0x124, 0xf, MAX>(v);  // row_ror:4
    v = dpp_step<0x128, 0xf, MAX>(v);  // row_ror:8
    v = dpp_step<0x142, 0xa, MAX>(v);  // row_bcast:15 into rows 1, 3
    v = dpp_step<0x143, 0xc, MAX>(v);  // row_bcast:31 into rows 2, 3
    return (uint32_t)__builtin_amdgcn_readlane((int)v, 63);
}

// The routing's working set, dead once the routing is published: the block's trellis staging reuses it.
struct RouteScratch {
    int pick[DL_MAXP];
    float wts[DL_MAXP];
    int unit[DL_MAXE];  // count of an expert's picks (mask of the rows that pick it, from logits)
    int uidx[256];      // an expert's unit, from logits
    int wsum[16];       // a wave's count of picked experts (up to 16 waves)
    uint64_t tptr[3][256];  // one row's path: every expert's addresses and widths, loaded with the logits
    int tk2[3][256];
};

struct RouteSh {
    int uids[DL_MAXP];
    int16_t members[DL_MAXP][DL_MAXR];
    int mcount[DL_MAXP];
    int ucount;
    uint64_t uptr[DL_MAXP][3];  // a routed unit's gate, up and down trellis addresses and widths
    int uk2[DL_MAXP][3];
    union {
        RouteScratch r;
        __attribute__((aligned(16))) uint32_t stage[DL_WAVES][DL_STAGE_WORDS];
    };
};

// One row's top-8 on one wave (E = 256: expert q * 64 + lane in choice[q]): choice = sigmoid + bias, the larger
// first, the lower id on a tie; wts = sigmoid / (sum of the picks' sigmoids in pick order + 1e-20) * scale
// (native_ops.cu:1015-1068). A round: the wave maximum of the choices' keys (one broadcast), then the lowest id holding
// it from four ballots, one a key register: the first non-empty ballot names q and its lowest set bit the lane, in
// scalar registers. The routing is the serial head of every routed item and its wave shares a SIMD with other blocks'
// decoding waves, so it runs at the highest wave priority. `rounds` < 8 stops after the first picks (wts are then
// not written: they need all eight).
__device__ __forceinline__ void topk8_wave(const float* logits, const float* bias, float scale, int* pick, float* wts,
                                           int lane, int rounds = DL_SLOTS) {
    __builtin_amdgcn_s_setprio(3);
    // all eight loads in flight before any is used
    float lg[4], bs[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        lg[q] = logits[q * 64 + lane];
        bs[q] = bias[q * 64 + lane];
    }
    asm volatile("" : "+v"(lg[0]), "+v"(lg[1]), "+v"(lg[2]), "+v"(lg[3]), "+v"(bs[0]), "+v"(bs[1]), "+v"(bs[2]),
                 "+v"(bs[3]));
    float score[4];
    uint32_t key[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        score[q] = 1.0f / (expf_path(0.0f - lg[q]) + 1.0f);
        key[q] = order_key(score[q] + bs[q]);
    }
    float total = 0.0f, my_w = 0.0f;
    int my_p = 0;
    for (int k = 0; k < rounds; ++k) {
        const uint32_t km = key[0] > key[1] ? key[0] : key[1], kn = key[2] > key[3] ? key[2] : key[3];
        const uint32_t m = wave_reduce<true>(km > kn ? km : kn);
        // some key equals the maximum, so one ballot is non-empty
        const uint64_t b0 = __builtin_amdgcn_ballot_w64(key[0] == m), b1 = __builtin_amdgcn_ballot_w64(key[1] == m);
        const uint64_t b2 = __builtin_amdgcn_ballot_w64(key[2] == m), b3 = __builtin_amdgcn_ballot_w64(key[3] == m);
        const int q = b0 ? 0 : (b1 ? 1 : (b2 ? 2 : 3));
        const uint64_t bq = b0 ? b0 : (b1 ? b1 : (b2 ? b2 : b3));
        const int src = (int)__builtin_ctzll(bq), e = q * 64 + src;
        const float sq = q == 0 ? score[0] : (q == 1 ? score[1] : (q == 2 ? score[2] : score[3]));
        const float sw = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, sq), src));
        total = total + sw;
        my_w = lane == k ? sw : my_w;
        my_p = lane == k ? e : my_p;
        const bool mine = lane == src;
        key[0] = (mine && q == 0) ? 0u : key[0];
        key[1] = (mine && q == 1) ? 0u : key[1];
        key[2] = (mine && q == 2) ? 0u : key[2];
        key[3] = (mine && q == 3) ? 0u : key[3];
    }
    if (lane < rounds) pick[lane] = my_p;
    if (rounds == DL_SLOTS && lane < DL_SLOTS) wts[lane] = my_w / (total + 1e-20f) * scale;
    __builtin_amdgcn_s_setprio(0);
}

// The trellis addresses and widths of every routed unit, into LDS (one round trip for the block, instead of one an
// item): gate and up, and down for the block that publishes them. Routed from logits, every expert's tables are in
// LDS already (loaded with the logits) and no round trip is left.
__device__ __forceinline__ void route_tables(const DLArgs& a, RouteSh& sh, int mats) {
    for (int u = threadIdx.x; u < sh.ucount; u += DL_THREADS) {
        const int e = sh.uids[u];
#pragma unroll
        for (int m = 0; m < 3; ++m)
            if (m < mats) {
                sh.uptr[u][m] = a.logits ? sh.r.tptr[m][e] : (uint64_t)a.ptr[m][e];
                sh.uk2[u][m] = a.logits ? sh.r.tk2[m][e] : a.k2t[m][e];
            }
    }
    __syncthreads();
}

// The grouping of the picks in sh.r.pick (route_block, route_kernel), by a block of DL_THREADS or more threads: the
// distinct picked experts in id order, each one's members, the units' tables.
__device__ __forceinline__ void route_group(const DLArgs& a, RouteSh& sh, int mats) {
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
    const int n = a.R * DL_SLOTS;
    // unit[e]: the count of expert e's picks, or (routed from logits, where a row's picks are distinct) the mask of the
    // rows that pick it
    for (int e = t; e < a.E; e += DL_THREADS) sh.r.unit[e] = 0;
    __syncthreads();
    for (int i = t; i < n; i += DL_THREADS) {
        const int e = sh.r.pick[i];
        if (e >= 0 && e < a.E) {
            if (a.logits)
                atomicOr(&sh.r.unit[e], 1 << (i / DL_SLOTS));
            else
                atomicAdd(&sh.r.unit[e], 1);
        }
    }
    __syncthreads();
    // units in expert order: an exclusive scan of "picked" over experts 4t .. 4t + 3
    int used = 0;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const int e = 4 * t + q;
        used += (e < a.E && sh.r.unit[e] > 0) ? 1 : 0;
    }
    int inc = used;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const int v = __shfl_up(inc, o, 64);
        if (lane >= o) inc += v;
    }
    if (lane == 63) sh.r.wsum[wave] = inc;
    __syncthreads();
    int place = inc - used;
    for (int w = 0; w < wave; ++w) place += sh.r.wsum[w];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const int e = 4 * t + q;
        if (e < a.E && sh.r.unit[e] > 0) {
            if (a.logits) sh.r.uidx[e] = place;
            sh.uids[place++] = e;
        }
    }
    if (t == DL_THREADS - 1) sh.ucount = place;
    __syncthreads();
    // a unit's members: its first R pairs in pair order (exl3_experts.cu:83-86 with maxm = R, moe.zig:288); a pair
    // past them keeps its y as it is, as a slot without an expert does. From logits a unit has one pair a row that
    // picks it, so a pair's place is the count of the earlier rows in its expert's mask (a thread a pair).
    if (a.logits) {
        for (int i = t; i < n; i += DL_THREADS) {
            const int e = sh.r.pick[i], r = i / DL_SLOTS, u = sh.r.uidx[e];
            const uint32_t mask = (uint32_t)sh.r.unit[e];
            sh.members[u][__builtin_popcount(mask & ((1u << r) - 1u))] = (int16_t)i;
            if ((mask >> r) == 1u) sh.mcount[u] = __builtin_popcount(mask);  // the unit's last row
        }
    } else {
        for (int u = t; u < sh.ucount; u += DL_THREADS) {
            const int e = sh.uids[u];
            int c = 0;
            for (int i = 0; i < n && c < a.R; ++i)
                if (sh.r.pick[i] == e) sh.members[u][c++] = (int16_t)i;
            sh.mcount[u] = c;
        }
    }
    __syncthreads();
    route_tables(a, sh, mats);
}

// The window's routing in LDS: picks (top-8 of the logits, or the given picks), the distinct picked experts in id
// order and each one's first R pairs in ascending order (exl3_experts.cu:36-90), and the units' trellis tables
// (`mats` matrices of each). One row from logits: the units are the picks in order, and a block that runs only units
// below `need` stops the top-8 there (its loads then start sooner; the tables of units from `need` on are not set).
__device__ __forceinline__ void route_block(const DLArgs& a, RouteSh& sh, int mats, int need = DL_SLOTS) {
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
    const int n = a.R * DL_SLOTS;
    if (a.logits && a.R == 1) {
        // one row: the tables of all 256 experts are loaded with the logits (a thread an expert), so the picks' need
        // no round trip after the top-8; each pick names a different expert and is a unit of its own
        uint64_t tp[3];
        int tk[3];
#pragma unroll
        for (int m = 0; m < 3; ++m) {
            tp[m] = (uint64_t)a.ptr[m][t];
            tk[m] = a.k2t[m][t];
        }
        // the routing wave by block, so that the routing waves of a CU's blocks are not all on one SIMD
        if (wave == (int)(blockIdx.x % DL_WAVES)) topk8_wave(a.logits, a.bias, a.scale, sh.r.pick, sh.r.wts, lane, need);
#pragma unroll
        for (int m = 0; m < 3; ++m) {
            sh.r.tptr[m][t] = tp[m];
            sh.r.tk2[m][t] = tk[m];
        }
        __syncthreads();
        if (t < need) {
            const int e = sh.r.pick[t];
            sh.uids[t] = e;
            sh.mcount[t] = 1;
            sh.members[t][0] = t;
#pragma unroll
            for (int m = 0; m < 3; ++m) {
                sh.uptr[t][m] = sh.r.tptr[m][e];
                sh.uk2[t][m] = sh.r.tk2[m][e];
            }
        }
        if (t == 0) sh.ucount = DL_SLOTS;
        __syncthreads();
        return;
    }
    // given picks (with more than one row route_kernel routes the window)
    for (int i = t; i < n; i += DL_THREADS) {
        sh.r.pick[i] = a.pick[i];
        sh.r.wts[i] = a.wts[i];
    }
    route_group(a, sh, mats);
}

// One block hands the routing to the caller (pick, wts) and the grouping to the later launches.
__device__ __forceinline__ void route_publish(const DLArgs& a, const RouteSh& sh) {
    const int t = threadIdx.x;
    const int n = a.R * DL_SLOTS;
    const DLLayout& l = a.lay;
    if (a.logits)
        for (int i = t; i < n; i += DL_THREADS) {
            a.pick[i] = sh.r.pick[i];
            a.wts[i] = sh.r.wts[i];
        }
    for (int u = t; u < sh.ucount; u += DL_THREADS) {
        l.uids[u] = sh.uids[u];
        l.mcount[u] = sh.mcount[u];
#pragma unroll
        for (int m = 0; m < 3; ++m) {
            l.tptr[u * 3 + m] = sh.uptr[u][m];
            l.tk2[u * 3 + m] = sh.uk2[u][m];
        }
        for (int i = 0; i < sh.mcount[u]; ++i) l.members[u * DL_MAXR + i] = sh.members[u][i];
    }
    if (t == 0) *l.ucount = sh.ucount;
}

// More than one row: one block routes the window (route_kernel) and publishes it, and every gate|up block reads the
// grouping and the units' gate and up tables back into LDS in one round trip, instead of routing every row itself.
// Every entry is read (entries past the counts are not used), so all the loads are in flight at once.
constexpr int DL_MEMW = DL_MAXP * DL_MAXR / DL_THREADS;  // member entries a thread
__device__ __forceinline__ void route_read(const DLArgs& a, RouteSh& sh) {
    const int t = threadIdx.x;  // the first DL_THREADS threads of the block read
    if (t < DL_THREADS) {
        const DLLayout& l = a.lay;
        const int tu = t < DL_MAXP ? t : DL_MAXP - 1;
        const int ucount = *l.ucount, uid = l.uids[tu], mc = l.mcount[tu];
        const uint64_t p0 = l.tptr[tu * 3], p1 = l.tptr[tu * 3 + 1];
        const int k0 = l.tk2[tu * 3], k1 = l.tk2[tu * 3 + 1];
        int mem[DL_MEMW];
#pragma unroll
        for (int j = 0; j < DL_MEMW; ++j) mem[j] = l.members[t + j * DL_THREADS];
        if (t < DL_MAXP) {
            sh.uids[t] = uid;
            sh.mcount[t] = mc;
            sh.uptr[t][0] = p0;
            sh.uptr[t][1] = p1;
            sh.uk2[t][0] = k0;
            sh.uk2[t][1] = k1;
        }
#pragma unroll
        for (int j = 0; j < DL_MEMW; ++j) {
            const int idx = t + j * DL_THREADS;
            sh.members[idx / DL_MAXR][idx % DL_MAXR] = (int16_t)mem[j];
        }
        if (t == 0) sh.ucount = ucount;
    }
    __syncthreads();
}

// The window's routing and grouping, once, for the gate|up blocks and the later launches (more than one row): a wave
// a row's top-8 (DL_MAXR waves), every expert's tables loaded with the logits by the first DL_THREADS threads.
constexpr int DL_ROUTE_THREADS = 64 * DL_MAXR;
__global__ void __launch_bounds__(DL_ROUTE_THREADS) route_kernel(DLArgs a) {
    static_assert(DL_ROUTE_THREADS <= 1024 && DL_ROUTE_THREADS / 64 <= 16, "a wave a row; wsum holds 16 waves");
    __shared__ RouteSh sh;
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
    if (a.logits) {
        const int te = t < 256 ? t : 255;  // E = 256
        uint64_t tp[3];
        int tk[3];
#pragma unroll
        for (int m = 0; m < 3; ++m) {
            tp[m] = (uint64_t)a.ptr[m][te];
            tk[m] = a.k2t[m][te];
        }
        if (wave < a.R)
            topk8_wave(a.logits + (size_t)wave * 256, a.bias, a.scale, sh.r.pick + wave * DL_SLOTS,
                       sh.r.wts + wave * DL_SLOTS, lane);
        if (t < 256)
#pragma unroll
            for (int m = 0; m < 3; ++m) {
                sh.r.tptr[m][t] = tp[m];
                sh.r.tk2[m][t] = tk[m];
            }
    } else {
        for (int i = t; i < a.R * DL_SLOTS; i += DL_ROUTE_THREADS) {
            sh.r.pick[i] = a.pick[i];
            sh.r.wts[i] = a.wts[i];
        }
    }
    route_group(a, sh, 3);  // its first barrier orders the picks and tables before their readers
    route_publish(a, sh);
}

// ---- the MFMA core of an item ------------------------------------------------------------------------------------

// The wave's two column tiles times the activation rows in xs over NKT k tiles: acc[j] += A (rows of xs, the MFMA's
// 16 rows; rows past the unit's members hold zeros) x B (tile pair (t, t + 1) of column tile j). The tiles' words are
// staged in LDS (st: tile (t, j) at word (2 t + j) * 4 K2); each lane reads the two words its four values come from
// and decodes the pair right before its MFMA.
template <int CB, int K2, int NKT>
__device__ __forceinline__ void mfma_tiles(const uint32_t* st, const LaneQuad& lq, const uint16_t* xs, int nm,
                                           int lane, f4v (&acc)[2]) {
    constexpr int TW = 4 * K2;
    const uint32_t* wa = st + lq.w0;
    const uint32_t* wb = st + lq.w1;
    const int m = lane & 15, g = (lane >> 4) & 3;
    const uint16_t* xr = xs + m * DL_RS + 2 * g;
#pragma unroll
    for (int t = 0; t < NKT; t += 2) {
        const uint16_t* xk = xr + t * 16;
        const u4v au = {*reinterpret_cast<const uint32_t*>(xk), *reinterpret_cast<const uint32_t*>(xk + 8),
                        *reinterpret_cast<const uint32_t*>(xk + 16), *reinterpret_cast<const uint32_t*>(xk + 24)};
        const h8v a = __builtin_bit_cast(h8v, au);
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const int t0 = (2 * t + j) * TW, t1 = (2 * (t + 1) + j) * TW;
            const u2v b0 = decode_quad<K2, CB>(wa[t0], wb[t0], lq.sh);
            const u2v b1 = decode_quad<K2, CB>(wa[t1], wb[t1], lq.sh);
            const h8v bb = __builtin_bit_cast(h8v, (u4v{b0.x, b0.y, b1.x, b1.y}));
            acc[j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, bb, acc[j], 0, 0, 0);
        }
    }
}

// The same product for a run-time width in 2..10 (false for any other): only this loop is specialised per width.
template <int CB, int NKT>
__device__ __forceinline__ bool mfma_tiles_k2(int k2, const uint32_t* st, const LaneQuad& lq, const uint16_t* xs,
                                              int nm, int lane, f4v (&acc)[2]) {
    return EA_K2_SWITCH(k2, 2, 10, (mfma_tiles<CB, K2V, NKT>(st, lq, xs, nm, lane, acc)));
}

// Wave-uniform values the compiler cannot prove uniform (a wave's index, what a block read from LDS or memory) moved
// to scalar registers: trellis addresses then live in SGPRs and the VGPRs hold the prefetched words.
__device__ __forceinline__ int uniform(int v) { return __builtin_amdgcn_readfirstlane(v); }
template <typename T>
__device__ __forceinline__ T* uniform(T* p) {
    const uint64_t v = reinterpret_cast<uint64_t>(p);
    const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)v);
    const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(v >> 32));
    return reinterpret_cast<T*>(((uint64_t)hi << 32) | lo);
}

// An opaque copy of the lane id: keeps the compiler from hoisting every width's lane constants out of the item loop
// (they would stay live across it and spill).
__device__ __forceinline__ int opaque_lane(int lane) {
    asm volatile("" : "+v"(lane));
    return lane;
}

// Rows [from, to) of a staged-activation array (DL_RS halves a row) set to zero by the block of NT threads.
template <int NT = DL_THREADS>
__device__ __forceinline__ void zero_rows(uint16_t* xs, int from, int to) {
    uint32_t* w = reinterpret_cast<uint32_t*>(xs + from * DL_RS);
    const int n = (to - from) * DL_RS / 2;
    for (int i = threadIdx.x; i < n; i += NT) w[i] = 0u;
}

// ---- gate | up ----------------------------------------------------------------------------------------------------

struct UnitView {
    bool shared;
    int nm;          // members (rows) of the unit
    int e;           // routed expert, -1 for the shared expert
    const int16_t* mem;  // routed members (pair ids)
};

__device__ __forceinline__ int member_q(const DLArgs& a, const UnitView& uv, int m) {
    return uv.shared ? a.R * DL_SLOTS + m : uv.mem[m];
}
__device__ __forceinline__ int member_row(const UnitView& uv, int m) { return uv.shared ? m : uv.mem[m] / DL_SLOTS; }

// The item's product for one width: prefetch every trellis word, rotate the activations of the k chunk into xs
// (xs[m][k] = fp16(((x * suh) @ H) * HAD_SCALE), a wave a (row, 128-block)), then the MFMAs.
template <int CB, int NW>
__device__ __forceinline__ bool gateup_product(const DLArgs& a, const UnitView& uv, const TileSpan& sp, int k2,
                                               const uint16_t* suh, int c, uint16_t* xs, uint32_t* st,
                                               f4v (&acc)[2]) {
    const int lane = opaque_lane(threadIdx.x & 63), wave = uniform((int)threadIdx.x >> 6);
    const LaneQuad lq = lane_quad(k2, lane);
    // activations and suh of this wave's (row, block) tasks, then the trellis: loads complete in order, so the
    // rotation waits only for the first two while the trellis is in flight. The trellis goes to the wave's LDS region
    // after the block barrier, so the barrier never waits for it.
    constexpr int MT = 2 * DL_MAXR / NW;
    uint32_t xv[MT], sv[MT];
    const int ntask = 2 * uv.nm;
#pragma unroll
    for (int i = 0; i < MT; ++i) {
        const int task = min(wave + NW * i, ntask - 1);  // unconditional (see stage_issue); extra lanes repeat
        const int m = task >> 1, blk = task & 1;
        const int k = c * 256 + blk * 128 + 2 * lane;
        const uint16_t* xr = static_cast<const uint16_t*>(a.x) + (size_t)member_row(uv, m) * a.x_stride;
        xv[i] = *reinterpret_cast<const uint32_t*>(xr + k);
        sv[i] = *reinterpret_cast<const uint32_t*>(suh + k);
    }
    u4v v[stage_loads<DL_KT>()];
    stage_issue<DL_KT>(sp, k2, lane, v);
    issued();
#pragma unroll
    for (int i = 0; i < MT; ++i) {
        hold(xv[i]);
        hold(sv[i]);
    }
    const bool bf = a.x_dtype == BF16;
#pragma unroll
    for (int i = 0; i < MT; ++i) {
        const int task = wave + NW * i;
        if (task < ntask) {
            const int m = task >> 1, blk = task & 1;
            const uint16_t xl = (uint16_t)(xv[i] & 0xffffu), xh = (uint16_t)(xv[i] >> 16);
            const float x0 = bf ? bf2f(xl) : h2f(xl);
            const float x1 = bf ? bf2f(xh) : h2f(xh);
            float v0 = x0 * h2f((uint16_t)(sv[i] & 0xffffu));
            float v1 = x1 * h2f((uint16_t)(sv[i] >> 16));
            fwht128_w64(v0, v1, lane);
            *reinterpret_cast<uint32_t*>(xs + m * DL_RS + blk * 128 + 2 * lane) =
                (uint32_t)f2h(v0 * HAD_SCALE) | ((uint32_t)f2h(v1 * HAD_SCALE) << 16);
        }
    }
    __syncthreads();
    stage_store<DL_KT>(st, k2, lane, v);
    return mfma_tiles_k2<CB, DL_KT>(k2, st, lq, xs, uv.nm, lane, acc);
}

// The unit of block u as the later launches see it, from the grouping the gate|up launch published. Every field loads
// at once (a unit's members past its count are read and not used), and with them the unit's down trellis address and
// width, so one round trip precedes the trellis.
struct UnitDown {
    const uint32_t* ptr;
    int k2;
};
__device__ __forceinline__ bool unit_from_layout(const DLArgs& a, int u, UnitView& uv, int16_t* s_mem,
                                                 UnitDown* down = nullptr) {
    const DLLayout& l = a.lay;
    const int ur = u > a.hs ? u - a.hs : 0;
    const int ucount = *l.ucount;
    const int nm = l.mcount[ur], e = l.uids[ur], dk2 = l.tk2[ur * 3 + 2];
    const uint64_t dptr = l.tptr[ur * 3 + 2];
    if (threadIdx.x < DL_MAXR) s_mem[threadIdx.x] = l.members[ur * DL_MAXR + threadIdx.x];
    if (u >= a.hs + ucount) return false;
    uv.shared = a.hs && u == 0;
    uv.nm = uniform(uv.shared ? a.R : nm);
    uv.e = uniform(uv.shared ? -1 : e);
    uv.mem = s_mem;
    if (down) {
        down->ptr = uniform(reinterpret_cast<const uint32_t*>(dptr));
        down->k2 = uniform(dk2);
    }
    return true;
}

// ---- the SwiGLU epilogue --------------------------------------------------------------------------------------------

// The gate|up partials of member q, column block nh, matrix mat (two columns a lane): every chunk's pair in flight at
// once.
__device__ __forceinline__ void zp_load(const DLArgs& a, int q, int nh, int mat, int lane, float2 (&v)[DL_MAXKC]) {
    const int NH = a.I / 128, KC = a.D / 256;
    const float* z = a.lay.zp + ((size_t)(q * NH + nh) * 2 + mat) * KC * 128 + 2 * lane;
#pragma unroll
    for (int cc = 0; cc < DL_MAXKC; ++cc) {
        const int ci = cc < KC ? cc : KC - 1;
        v[cc] = *reinterpret_cast<const float2*>(z + ci * 128);
    }
}

// Their sum in chunk order.
__device__ __forceinline__ float2 zp_sum(const DLArgs& a, const float2 (&v)[DL_MAXKC]) {
    const int KC = a.D / 256;
    float s0 = 0.f, s1 = 0.f;
#pragma unroll
    for (int cc = 0; cc < DL_MAXKC; ++cc)
        if (cc < KC) {
            s0 += v[cc].x;
            s1 += v[cc].y;
        }
    return float2{s0, s1};
}

// The two fp16 scales of columns n, n + 1 of a column block (packed, as loaded): the gate or up output scale svh,
// and the down input scale suh_d. Callers load them with the partial sums, ahead of any trellis load, since a load
// issued after the trellis completes only after it.
__device__ __forceinline__ uint32_t svh_pair(const DLArgs& a, const UnitView& uv, int nh, int mat, int lane) {
    const uint16_t* svh =
        uv.shared ? (mat ? a.sh_svh[1] : a.sh_svh[0]) : (mat ? a.svh_u : a.svh_g) + (size_t)uv.e * a.I;
    return *reinterpret_cast<const uint32_t*>(svh + nh * 128 + 2 * lane);
}
__device__ __forceinline__ uint32_t suhd_pair(const DLArgs& a, const UnitView& uv, int nh, int lane) {
    const uint16_t* suh = uv.shared ? a.sh_suh[2] : a.suh_d + (size_t)uv.e * a.I;
    return *reinterpret_cast<const uint32_t*>(suh + nh * 128 + 2 * lane);
}

// A matrix's outputs of a column block: FWHT of the sums, HAD_SCALE, the output scale svh (the pair sv). The shared
// expert's gate and up linears write bf16 (forward.zig:2330); the routed experts keep fp32 (exl3_experts.cu:142-184).
__device__ __forceinline__ float2 gu_out(const UnitView& uv, float2 v, uint32_t sv, int lane) {
    fwht128_w64(v.x, v.y, lane);
    float o0 = v.x * HAD_SCALE * h2f((uint16_t)(sv & 0xffffu));
    float o1 = v.y * HAD_SCALE * h2f((uint16_t)(sv >> 16));
    if (uv.shared) {
        o0 = bf16r(o0);
        o1 = bf16r(o1);
    }
    return float2{o0, o1};
}

// SwiGLU of a column block, the down input scale suh (the pair sd), FWHT, HAD_SCALE: the packed fp16 down inputs of
// columns n, n + 1. Routed experts: act_mode 1 with no limit (moe.zig:290; exl3_experts.cu:142-184). The shared
// expert: swiglu2 in bf16 (native_ops.cu:429-441), read by the down linear's rot_in (exl3_linear.cu:152-173).
__device__ __forceinline__ uint32_t act_pair(const UnitView& uv, float2 g, float2 u, uint32_t sd, int lane) {
    const float gs[2] = {g.x, g.y}, us[2] = {u.x, u.y};
    const float ss[2] = {h2f((uint16_t)(sd & 0xffffu)), h2f((uint16_t)(sd >> 16))};
    float v[2];
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        if (uv.shared) {
            const float sg = bf16r(gs[j] / (expf_path(0.0f - gs[j]) + 1.0f));
            v[j] = bf16r(sg * us[j]) * ss[j];
        } else {
            v[j] = gs[j] / (1.f + expf_path(-gs[j])) * us[j] * ss[j];
        }
    }
    fwht128_w64(v[0], v[1], lane);
    return (uint32_t)f2h(v[0] * HAD_SCALE) | ((uint32_t)f2h(v[1] * HAD_SCALE) << 16);
}

// Block (unit, column block nh of 128, group g of DL_WAVES members): the down inputs of the group's members, a wave a
// member, so that every member's partial sums are in flight at once.
__global__ void __launch_bounds__(DL_THREADS) epilogue_kernel(DLArgs a) {
    __shared__ int16_t s_mem[DL_MAXR];
    const int NH = a.I / 128, MG = (a.R + DL_WAVES - 1) / DL_WAVES;
    const int unit = blockIdx.x / (NH * MG), nh = (blockIdx.x / MG) % NH, grp = blockIdx.x % MG;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    UnitView uv;
    if (!unit_from_layout(a, unit, uv, s_mem)) return;
    __syncthreads();
    const int m = grp * DL_WAVES + wave;
    if (m < uv.nm) {
        const uint32_t svg = svh_pair(a, uv, nh, 0, lane), svu = svh_pair(a, uv, nh, 1, lane);
        const uint32_t sd = suhd_pair(a, uv, nh, lane);
        const int q = member_q(a, uv, m);
        float2 zg[DL_MAXKC], zu[DL_MAXKC];
        zp_load(a, q, nh, 0, lane, zg);
        zp_load(a, q, nh, 1, lane, zu);
        const float2 g = gu_out(uv, zp_sum(a, zg), svg, lane);
        const float2 u = gu_out(uv, zp_sum(a, zu), svu, lane);
        *reinterpret_cast<uint32_t*>(a.lay.xd + (size_t)q * a.I + nh * 128 + 2 * lane) = act_pair(uv, g, u, sd, lane);
    }
}

// Item (unit u, column block nh, matrix mat, k chunk c) of the shared expert (SHARED, codebook CB) or of a routed
// unit.
// NW = 2 * DL_WAVES (more than one row, I = 256): the block covers both column blocks of the unit, waves from
// DL_WAVES on the second (nh is then the wave's), and rotates the members' activations once for both; st is the
// wave's trellis staging.
template <int CB, bool SHARED, int NW = DL_WAVES>
__device__ __forceinline__ void gateup_item(const DLArgs& a, RouteSh& sh, int u, int nh, int mat, int c,
                                            uint16_t* xs, uint32_t* st) {
    static_assert(NW == DL_WAVES || NW == 2 * DL_WAVES, "one or both column blocks of 128");
    const int lane = threadIdx.x & 63, wave = uniform((int)threadIdx.x >> 6);
    const int KC = a.D / 256, NH = a.I / 128;
    const int wl = wave & (DL_WAVES - 1);  // the wave within its column block
    if (NW != DL_WAVES) nh = wave / DL_WAVES;
    UnitView uv;
    uv.shared = SHARED;
    const int ur = u - a.hs;
    uv.nm = SHARED ? a.R : uniform(sh.mcount[ur]);
    uv.e = SHARED ? -1 : uniform(sh.uids[ur]);
    uv.mem = SHARED ? nullptr : sh.members[ur];
    // wave w: n tiles nh * 8 + 2w, + 1 over the 16 k tiles of chunk c
    const int nt0 = nh * 8 + 2 * wl, kt0 = c * DL_KT;
    f4v acc[2] = {f4v{0.f, 0.f, 0.f, 0.f}, f4v{0.f, 0.f, 0.f, 0.f}};
    // matrix D x I: routed in the expert layout (tile (kt, nt) at (kt * I / 16 + nt) * TW words), the shared expert
    // in strips ([I / 128][D / 16][8][TW])
    const int ns = a.I / 16;
    TileSpan sp;
    int k2;
    const uint16_t* suh;
    if constexpr (SHARED) {
        k2 = a.sh_k2;
        const int TWB = 16 * k2;  // bytes a tile
        sp.r = buffer_rsrc(mat ? a.sh_w[1] : a.sh_w[0], (uint32_t)((a.D / 16) * ns * TWB));
        sp.off = ((nt0 >> 3) * (a.D / 16) * 8 + kt0 * 8 + (nt0 & 7)) * TWB;
        sp.kstride = 8 * TWB;
        suh = mat ? a.sh_suh[1] : a.sh_suh[0];
    } else {
        k2 = uniform(sh.uk2[ur][mat]);
        const uint32_t* T = uniform(reinterpret_cast<const uint32_t*>(sh.uptr[ur][mat]));
        const int TWB = 16 * k2;
        sp.r = buffer_rsrc(T, (uint32_t)((a.D / 16) * ns * TWB));
        sp.off = (kt0 * ns + nt0) * TWB;
        sp.kstride = ns * TWB;
        suh = (mat ? a.suh_u : a.suh_g) + (size_t)uv.e * a.D;
    }
    const bool ok = gateup_product<CB, NW>(a, uv, sp, k2, suh, c, xs, st, acc);
    if (!ok) {
        if (lane == 0) record_error(a.status, DEV_UNSUPPORTED_WIDTH);
        acc[0] = acc[1] = nan4();
    }
    // partial sums of this chunk: zp[q][nh][mat][c][128]
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int m = 4 * (lane >> 4) + i;
            if (m < uv.nm) {
                const int col = (2 * wl + j) * 16 + (lane & 15);
                a.lay.zp[((((size_t)member_q(a, uv, m) * NH + nh) * 2 + mat) * KC + c) * 128 + col] = acc[j][i];
            }
        }
}

template <int CB, int SCB>
__global__ void __launch_bounds__(DL_THREADS) __attribute__((amdgpu_waves_per_eu(4)))
gateup_kernel(DLArgs a) {
    static_assert(DL_THREADS == 256, "the one-row routing loads an expert a thread");
    __shared__ RouteSh sh;
    __shared__ __attribute__((aligned(16))) uint16_t xs[DL_MAXR * DL_RS];
    const int NH = a.I / 128, KC = a.D / 256;
    const int per_unit = NH * 2 * KC;
    const int items = a.U * per_unit;
    // the shared expert's items (unit 0, the first per_unit items) need no routing: they run first, their trellis loads
    // starting with the launch; a block routes before its first routed item, and the block that runs the first
    // routed item publishes the routing
    const int first_routed = a.hs * per_unit;
    // the MFMAs read all 16 rows and an item writes its members' rows: rows from R on stay zero, rows below R are
    // zeroed before an item with fewer members (every write is ordered before the reads by the item's rotation
    // barrier, and no item writes the rows being zeroed)
    zero_rows(xs, a.R, DL_MAXR);
    int dirty = a.R;  // rows that may hold an earlier item's activations
    int it = blockIdx.x;
    for (; it < items && it < first_routed; it += gridDim.x) {
        gateup_item<SCB, true>(a, sh, 0, it / (2 * KC), (it / KC) & 1, it % KC, xs, sh.stage[uniform((int)threadIdx.x >> 6)]);
        __syncthreads();
    }
    if (it >= items) return;
    if (a.R > 1) {
        route_read(a, sh);
    } else {
        const bool publisher = it == first_routed;
        int need = DL_SLOTS;  // from logits: the picks up to the block's last unit (the publisher needs them all)
        if (a.logits && !publisher) {
            const int last = it + (items - 1 - it) / (int)gridDim.x * (int)gridDim.x;
            need = min(DL_SLOTS, last / per_unit - a.hs + 1);
        }
        route_block(a, sh, publisher ? 3 : 2, need);
        if (publisher) route_publish(a, sh);
    }
    // the routed items, in unit order (issuing the next item's loads before the current item's product measured no
    // faster: with more than one row the items are decode-bound, and the larger kernel slowed the one-row layer)
    const int units = a.hs + sh.ucount;
    for (; it < items; it += gridDim.x) {
        const int u = it / per_unit, rem = it % per_unit;
        if (u >= units) break;
        const int nm = sh.mcount[u - a.hs];
        if (nm < dirty) zero_rows(xs, nm, dirty);
        gateup_item<CB, false>(a, sh, u, rem / (2 * KC), (rem / KC) & 1, rem % KC, xs,
                               sh.stage[uniform((int)threadIdx.x >> 6)]);
        dirty = nm;
        __syncthreads();
    }
}

// More than one row with I = 256: items (unit, matrix, k chunk) over both column blocks, blocks of 2 * DL_WAVES
// waves, the routing read from route_kernel's output. Each item rotates its members' activations once for both column
// blocks (a block of DL_WAVES waves per column block rotates them twice).
template <int CB, int SCB>
__global__ void __launch_bounds__(2 * DL_THREADS) __attribute__((amdgpu_waves_per_eu(2)))
gateup_wide_kernel(DLArgs a) {
    constexpr int NW = 2 * DL_WAVES, NT = 64 * NW;
    __shared__ RouteSh sh;
    __shared__ __attribute__((aligned(16))) uint32_t stage_hi[DL_WAVES][DL_STAGE_WORDS];  // waves DL_WAVES.. 2 DL_WAVES
    __shared__ __attribute__((aligned(16))) uint16_t xs[DL_MAXR * DL_RS];
    const int KC = a.D / 256;
    const int per_unit = 2 * KC;
    const int items = a.U * per_unit;
    const int first_routed = a.hs * per_unit;
    const int wave = uniform((int)threadIdx.x >> 6);
    uint32_t* st = wave < DL_WAVES ? sh.stage[wave] : stage_hi[wave - DL_WAVES];
    zero_rows<NT>(xs, a.R, DL_MAXR);
    int dirty = a.R;
    int it = blockIdx.x;
    for (; it < items && it < first_routed; it += gridDim.x) {
        gateup_item<SCB, true, NW>(a, sh, 0, 0, it / KC, it % KC, xs, st);
        __syncthreads();
    }
    if (it >= items) return;
    route_read(a, sh);
    const int units = a.hs + sh.ucount;
    for (; it < items; it += gridDim.x) {
        const int u = it / per_unit, rem = it % per_unit;
        if (u >= units) break;
        const int nm = sh.mcount[u - a.hs];
        if (nm < dirty) zero_rows<NT>(xs, nm, dirty);
        gateup_item<CB, false, NW>(a, sh, u, 0, rem / KC, rem % KC, xs, st);
        dirty = nm;
        __syncthreads();
    }
}

// ---- down ---------------------------------------------------------------------------------------------------------

// The unit's down inputs into xs, then the product, for a block of NW waves. FOLD (one row: a unit has at most 8
// members): the block computes the inputs itself from the gate|up partials, a wave a (member, column block, matrix)
// task, instead of the epilogue launch; a wave's first task's partials load ahead of its trellis, and a wave without a
// task loads only its trellis. Otherwise they are the epilogue's, loaded ahead of the trellis. Loads complete in
// order, so the inputs never wait for the trellis.
template <int CB, int SCB, int NKT, bool FOLD, int NW>
__device__ __forceinline__ bool down_product(const DLArgs& a, const UnitView& uv, const TileSpan& sp, int k2,
                                             uint16_t* xs, float* gus, uint32_t* st, f4v (&acc)[2]) {
    constexpr int NT = 64 * NW;
    const int lane = opaque_lane(threadIdx.x & 63), wave = uniform((int)threadIdx.x >> 6);
    const LaneQuad lq = lane_quad(k2, lane);
    u4v v[stage_loads<NKT>()];
    if constexpr (FOLD) {
        const int NH = a.I / 128, tasks = uv.nm * NH * 2;
        // the scales of the wave's first epilogue task ((member, column block, matrix), then (member, column block)
        // of the activation), loaded with its partial sums and ahead of the trellis; a wave past the last task
        // reads the last one's
        const int t0 = min(wave, tasks - 1), a0 = min(wave, uv.nm * NH - 1);
        uint32_t sv0 = svh_pair(a, uv, (t0 >> 1) % NH, t0 & 1, lane), sd0 = suhd_pair(a, uv, a0 % NH, lane);
        if (wave < tasks) {
            float2 zv[DL_MAXKC];
            zp_load(a, member_q(a, uv, wave / (2 * NH)), (wave >> 1) % NH, wave & 1, lane, zv);
            stage_issue<NKT>(sp, k2, lane, v);
            issued();
            hold(sv0);
            hold(sd0);
#pragma unroll
            for (int cc = 0; cc < DL_MAXKC; ++cc) hold(zv[cc]);
            for (int task = wave; task < tasks; task += NW) {
                const int m = task / (2 * NH), nh = (task >> 1) % NH, mat = task & 1;
                uint32_t sv = sv0;
                if (task != wave) {
                    zp_load(a, member_q(a, uv, m), nh, mat, lane, zv);
                    sv = svh_pair(a, uv, nh, mat, lane);
                }
                const float2 o = gu_out(uv, zp_sum(a, zv), sv, lane);
                *reinterpret_cast<float2*>(gus + (m * 2 + mat) * DL_MAXI + nh * 128 + 2 * lane) = o;
            }
        } else {
            stage_issue<NKT>(sp, k2, lane, v);
            issued();
            hold(sd0);
        }
        zero_rows<NT>(xs, uv.nm, DL_MAXR);  // the MFMAs read all 16 rows
        __syncthreads();
        for (int task = wave; task < uv.nm * NH; task += NW) {
            const int m = task / NH, nh = task % NH;
            const float2 g = *reinterpret_cast<const float2*>(gus + (m * 2) * DL_MAXI + nh * 128 + 2 * lane);
            const float2 u = *reinterpret_cast<const float2*>(gus + (m * 2 + 1) * DL_MAXI + nh * 128 + 2 * lane);
            const uint32_t sd = task == wave ? sd0 : suhd_pair(a, uv, nh, lane);
            *reinterpret_cast<uint32_t*>(xs + m * DL_RS + nh * 128 + 2 * lane) = act_pair(uv, g, u, sd, lane);
        }
    } else {
        constexpr int WPR = NKT * 16 / 2;  // words a row
        constexpr int MW = DL_MAXR * WPR / NT;
        uint32_t xv[MW];
#pragma unroll
        for (int i = 0; i < MW; ++i) {
            const int idx = threadIdx.x + NT * i;
            const int m = min(idx / WPR, uv.nm - 1), k = 2 * (idx % WPR);  // unconditional (see stage_issue)
            xv[i] = *reinterpret_cast<const uint32_t*>(a.lay.xd + (size_t)member_q(a, uv, m) * a.I + k);
        }
        stage_issue<NKT>(sp, k2, lane, v);
        issued();
        zero_rows<NT>(xs, uv.nm, DL_MAXR);  // the MFMAs read all 16 rows
#pragma unroll
        for (int i = 0; i < MW; ++i) hold(xv[i]);
#pragma unroll
        for (int i = 0; i < MW; ++i) {
            const int idx = threadIdx.x + NT * i;
            const int m = idx / WPR, k = 2 * (idx % WPR);
            if (m < uv.nm) *reinterpret_cast<uint32_t*>(xs + m * DL_RS + k) = xv[i];
        }
    }
    __syncthreads();
    stage_store<NKT>(st, k2, lane, v);
    return uv.shared ? mfma_tiles_k2<SCB, NKT>(k2, st, lq, xs, uv.nm, lane, acc)
                     : mfma_tiles_k2<CB, NKT>(k2, st, lq, xs, uv.nm, lane, acc);
}

// The down launches' LDS besides the staged activations, for a block of NW waves (NW / 4 column blocks of 128): the
// folded epilogue's gate and up values, the trellis staging and the product's column sums are live one after
// another, so they share one region.
template <int NW>
union DownSh {
    float gus[DL_SLOTS * 2 * DL_MAXI];
    __attribute__((aligned(16))) uint32_t stage[NW][DL_STAGE_WORDS];
    float ys[DL_MAXR * 128 * (NW / 4)];
};

// Block (unit, NW / 4 adjacent column blocks of 128 outputs), four waves a column block: the members' down products,
// FWHT, svh -> the pair's y (or the shared expert's sy). The unit's down inputs are formed once for all of the
// block's column blocks.
template <int CB, int SCB, bool FOLD, int NW>
__device__ __forceinline__ void down_block(const DLArgs& a, uint16_t* xs, DownSh<NW>& ds, int16_t* s_mem) {
    constexpr int CBB = NW / 4;
    const int GB = a.D / 128 / CBB;
    const int u = blockIdx.x / GB, cg = blockIdx.x % GB;
    const int lane = threadIdx.x & 63, wave = uniform((int)threadIdx.x >> 6);
    UnitView uv;
    UnitDown dn;
    if (!unit_from_layout(a, u, uv, s_mem, &dn)) return;
    __syncthreads();
    const int cbl = wave >> 2, nt0 = (cg * CBB + cbl) * 8 + 2 * (wave & 3), KT = a.I / 16;
    // the output scales of the wave's column block in the FWHT tasks below (every task of a wave has the same one),
    // loaded ahead of the trellis
    const uint16_t* svh = uv.shared ? a.sh_svh[2] : a.svh_d + (size_t)uv.e * a.D;
    uint32_t sd = *reinterpret_cast<const uint32_t*>(svh + (cg * CBB + wave % CBB) * 128 + 2 * lane);
    f4v acc[2] = {f4v{0.f, 0.f, 0.f, 0.f}, f4v{0.f, 0.f, 0.f, 0.f}};
    // matrix I x D: routed in the expert layout, the shared expert in strips ([D / 128][I / 16][8][TW])
    const int ns = a.D / 16;
    const int k2 = uv.shared ? a.sh_k2 : dn.k2, TWB = 16 * k2;
    TileSpan sp;
    if (uv.shared) {
        sp.r = buffer_rsrc(a.sh_w[2], (uint32_t)(KT * ns * TWB));
        sp.off = ((nt0 >> 3) * KT * 8 + (nt0 & 7)) * TWB;
        sp.kstride = 8 * TWB;
    } else {
        sp.r = buffer_rsrc(dn.ptr, (uint32_t)(KT * ns * TWB));
        sp.off = nt0 * TWB;
        sp.kstride = ns * TWB;
    }
    const bool ok = a.I == 256
                        ? down_product<CB, SCB, 16, FOLD, NW>(a, uv, sp, k2, xs, ds.gus, ds.stage[wave], acc)
                        : down_product<CB, SCB, 8, FOLD, NW>(a, uv, sp, k2, xs, ds.gus, ds.stage[wave], acc);
    if (!ok) {
        if (lane == 0) record_error(a.status, DEV_UNSUPPORTED_WIDTH);
        acc[0] = acc[1] = nan4();
    }
    __syncthreads();  // the column sums overwrite the other waves' staging
    constexpr int YS = 128 * CBB;  // ys row stride
    float* ys = ds.ys;
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int i = 0; i < 4; ++i)
            ys[(4 * (lane >> 4) + i) * YS + cbl * 128 + (2 * (wave & 3) + j) * 16 + (lane & 15)] = acc[j][i];
    __syncthreads();
    // FWHT of each member's 128 columns of each column block, * HAD_SCALE * svh_d
    hold(sd);
    const float s0 = h2f((uint16_t)(sd & 0xffffu)), s1 = h2f((uint16_t)(sd >> 16));
    for (int task = wave; task < uv.nm * CBB; task += NW) {
        const int m = task / CBB, c = task % CBB;
        const int n = (cg * CBB + c) * 128 + 2 * lane;
        float v0 = ys[m * YS + c * 128 + 2 * lane], v1 = ys[m * YS + c * 128 + 2 * lane + 1];
        fwht128_w64(v0, v1, lane);
        float* dst = uv.shared ? a.lay.sy + (size_t)m * a.D : a.yroute + (size_t)member_q(a, uv, m) * a.D;
        *reinterpret_cast<float2*>(dst + n) = float2{v0 * HAD_SCALE * s0, v1 * HAD_SCALE * s1};
    }
}

template <int CB, int SCB>
__global__ void __launch_bounds__(DL_THREADS) __attribute__((amdgpu_waves_per_eu(4))) down_kernel(DLArgs a) {
    __shared__ __attribute__((aligned(16))) uint16_t xs[DL_MAXR * DL_RS];
    __shared__ DownSh<DL_WAVES> ds;
    __shared__ int16_t s_mem[DL_MAXR];
    down_block<CB, SCB, false, DL_WAVES>(a, xs, ds, s_mem);
}

// One row: the epilogue folded in (a unit has at most DL_SLOTS members; the grid covers few blocks, so two waves a
// SIMD are enough and the partials and the trellis stay in registers together). Every block of a unit reads the
// unit's gate|up partial sums: a block of eight waves over two column blocks halves those reads with the same waves a
// SIMD. (Sixteen waves over four column blocks measured slower: four waves a SIMD decode one after another.)
constexpr int DL_FOLD_WAVES = 8;
template <int CB, int SCB>
__global__ void __launch_bounds__(64 * DL_FOLD_WAVES) __attribute__((amdgpu_waves_per_eu(2))) down_fold_kernel(DLArgs a) {
    __shared__ __attribute__((aligned(16))) uint16_t xs[DL_MAXR * DL_RS];
    __shared__ DownSh<DL_FOLD_WAVES> ds;
    __shared__ int16_t s_mem[DL_MAXR];
    down_block<CB, SCB, true, DL_FOLD_WAVES>(a, xs, ds, s_mem);
}

// A wave a (row, column block of 128): out = fma chain over the slots in order from 0 of wts * y (a slot whose pick
// is not an expert reads y as it is; exl3_experts.cu:256-267), then + the shared expert (forward.zig:2403).
__global__ void __launch_bounds__(DL_THREADS) combine_kernel(DLArgs a) {
    const int DB = a.D / 128;
    const int w = blockIdx.x * DL_WAVES + (threadIdx.x >> 6), lane = threadIdx.x & 63;
    if (w >= a.R * DB) return;
    const int r = w / DB, n = (w % DB) * 128 + 2 * lane;
    float2 y[DL_SLOTS];
#pragma unroll
    for (int k = 0; k < DL_SLOTS; ++k)
        y[k] = *reinterpret_cast<const float2*>(a.yroute + (size_t)(r * DL_SLOTS + k) * a.D + n);
    float a0 = 0.f, a1 = 0.f;
#pragma unroll
    for (int k = 0; k < DL_SLOTS; ++k) {
        const float wk = a.wts[r * DL_SLOTS + k];
        a0 = __builtin_fmaf(wk, y[k].x, a0);
        a1 = __builtin_fmaf(wk, y[k].y, a1);
    }
    if (a.hs) {
        const float2 sv = *reinterpret_cast<const float2*>(a.lay.sy + (size_t)r * a.D + n);
        a0 = a0 + sv.x;
        a1 = a1 + sv.y;
    }
    *reinterpret_cast<float2*>(a.out + (size_t)r * a.D + n) = float2{a0, a1};
}

// ---- the one-row layer in one launch ---------------------------------------------------------------------------------
// One row routed from logits runs as a single launch of DL_THREADS-thread blocks, one item a block, in two index
// ranges:
//   [0, U GU): gate|up items (unit, column block nh, matrix, k chunk of 256), the shared expert's (unit 0) first;
//   [U GU, U GU + U DB): down items (unit, output column block of 128).
// A gate|up block routes the row up to its unit's pick (the shared expert's items need no routing), stages its 16 k
// tiles x 2 column tiles a wave of trellis in LDS, rotates the row's activations of its chunk, multiplies on MFMA and
// stores its partial sums. The block that completes a (unit, nh) -- the last of its 2 KC items to count in -- sums the
// chunks in order and runs the SwiGLU epilogue of that column block into the unit's down inputs, then counts the
// column block ready. A down block routes the row, stages its unit's down trellis of its column block and waits until
// both column blocks of its unit are ready; it multiplies, rotates and stores the unit's output of the column block.
// The last of the U down blocks of a column block to count in combines it: the slots in order from 0, then the shared
// expert.
// Hand-offs need no fence: data handed on is written with agent-scope stores (coherent across the XCDs' L2s), each wave
// waits for its stores (vmcnt 0), the block meets at a barrier, and only then one thread counts in; readers load with
// agent-scope loads issued after they have seen the count. A down block waits only for items of lower block index,
// which the hardware dispatched before it and which never wait, so every wait ends; it is bounded anyway (a give-up is
// recorded as EA_SYNC_TIMEOUT and the block's output is NaN). Every counter is back at zero when the launch ends: a
// counter's last arrival resets it, and the last down block of a unit resets the unit's ready count.

constexpr int L1_UNITS = 1 + DL_SLOTS;  // the shared expert and the eight picks
constexpr int L1_MAXDB = 256 * DL_MAXKC / 128;  // output column blocks at the largest D

// The counters, one 128-byte line each: gate|up items done per (unit, nh); column blocks ready per unit; down items
// done per unit; units done per output column block.
__device__ __forceinline__ int* l1_gcnt(int* s, int u, int nh) { return s + (u * 2 + nh) * L1_LINE; }
__device__ __forceinline__ int* l1_urdy(int* s, int u) { return s + (2 * L1_UNITS + u) * L1_LINE; }
__device__ __forceinline__ int* l1_dcnt(int* s, int u) { return s + (3 * L1_UNITS + u) * L1_LINE; }
__device__ __forceinline__ int* l1_ccnt(int* s, int cb) { return s + (4 * L1_UNITS + cb) * L1_LINE; }
static_assert((4 * L1_UNITS + L1_MAXDB) * L1_LINE * 4 <= (int)L1_SYNC_BYTES, "the counters fit their region");

struct L1Sh {
    int pick[DL_SLOTS];
    float wts[DL_SLOTS];
    uint64_t tp;  // the block's unit: the trellis address and width of the block's matrix, its expert
    int tk, e;
    int flag;
    __attribute__((aligned(16))) uint16_t xs[DL_RS];  // the row: its rotated activations, or the unit's down inputs
    union {
        struct {
            uint64_t tptr[256];
            int tk2[256];
        } r;  // every expert's table of the block's matrix, loaded with the logits
        __attribute__((aligned(16))) uint32_t stage[DL_WAVES][DL_STAGE_WORDS];
        float gus[2][128];
        float ys[128];
    };
};

// The row's picks up to `need` (need = 8: all of them and their weights) and the tables of matrix `mat` of every
// expert, a thread an expert (E = 256); then the block's unit u's entry (u >= 1: routed unit u - 1, pick u - 1).
__device__ __forceinline__ void l1_route(const DLArgs& a, L1Sh& sh, int mat, int u, int need) {
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
    const uint64_t tp = (uint64_t)a.ptr[mat][t];
    const int tk = a.k2t[mat][t];
    if (wave == (int)(blockIdx.x % DL_WAVES)) topk8_wave(a.logits, a.bias, a.scale, sh.pick, sh.wts, lane, need);
    sh.r.tptr[t] = tp;
    sh.r.tk2[t] = tk;
    __syncthreads();
    if (t == 0) {
        const int e = sh.pick[u - 1];
        sh.e = e;
        sh.tp = sh.r.tptr[e];
        sh.tk = sh.r.tk2[e];
    }
    __syncthreads();
}

// The row's product over NKT k tiles with the wave's two column tiles staged in st: acc[j] (row 0 in lanes 0..15,
// element 0) += xs (A rows 1..15 zero) x the tiles.
template <int CB, int K2, int NKT>
__device__ __forceinline__ void l1_mfma(const uint32_t* st, const LaneQuad& lq, const uint16_t* xs, int lane,
                                        f4v (&acc)[2]) {
    constexpr int TW = 4 * K2;
    const uint32_t* wa = st + lq.w0;
    const uint32_t* wb = st + lq.w1;
    const bool row0 = (lane & 15) == 0;
    const uint16_t* xr = xs + 2 * ((lane >> 4) & 3);
#pragma unroll
    for (int t = 0; t < NKT; t += 2) {
        const uint16_t* xk = xr + t * 16;
        u4v au = {*reinterpret_cast<const uint32_t*>(xk), *reinterpret_cast<const uint32_t*>(xk + 8),
                  *reinterpret_cast<const uint32_t*>(xk + 16), *reinterpret_cast<const uint32_t*>(xk + 24)};
        if (!row0) au = u4v{0u, 0u, 0u, 0u};
        const h8v a = __builtin_bit_cast(h8v, au);
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const int t0 = (2 * t + j) * TW, t1 = (2 * (t + 1) + j) * TW;
            const u2v b0 = decode_quad<K2, CB>(wa[t0], wb[t0], lq.sh);
            const u2v b1 = decode_quad<K2, CB>(wa[t1], wb[t1], lq.sh);
            const h8v bb = __builtin_bit_cast(h8v, (u4v{b0.x, b0.y, b1.x, b1.y}));
            acc[j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, bb, acc[j], 0, 0, 0);
        }
    }
}
template <int CB, int NKT>
__device__ __forceinline__ bool l1_mfma_k2(int k2, const uint32_t* st, const LaneQuad& lq, const uint16_t* xs,
                                           int lane, f4v (&acc)[2]) {
    return EA_K2_SWITCH(k2, 2, 10, (l1_mfma<CB, K2V, NKT>(st, lq, xs, lane, acc)));
}

// Gate|up item (unit u, column block nh, matrix mat, chunk c) of the row. q: the unit's member (the pick's slot, or P
// for the shared expert).
template <int CB, bool SHARED>
__device__ __forceinline__ void l1_gateup(const DLArgs& a, L1Sh& sh, int u, int nh, int mat, int c, int q) {
    const int lane = opaque_lane(threadIdx.x & 63), wave = uniform((int)threadIdx.x >> 6);
    const int KC = a.D / 256, NH = a.I / 128, ns = a.I / 16;
    const int nt0 = nh * 8 + 2 * wave, kt0 = c * DL_KT;
    TileSpan sp;
    int k2;
    const uint16_t* suh;
    if constexpr (SHARED) {
        k2 = a.sh_k2;
        const int TWB = 16 * k2;
        sp.r = buffer_rsrc(mat ? a.sh_w[1] : a.sh_w[0], (uint32_t)((a.D / 16) * ns * TWB));
        sp.off = ((nt0 >> 3) * (a.D / 16) * 8 + kt0 * 8 + (nt0 & 7)) * TWB;
        sp.kstride = 8 * TWB;
        suh = mat ? a.sh_suh[1] : a.sh_suh[0];
    } else {
        k2 = uniform(sh.tk);
        const int TWB = 16 * k2;
        sp.r = buffer_rsrc(uniform(reinterpret_cast<const uint32_t*>(sh.tp)), (uint32_t)((a.D / 16) * ns * TWB));
        sp.off = (kt0 * ns + nt0) * TWB;
        sp.kstride = ns * TWB;
        suh = (mat ? a.suh_u : a.suh_g) + (size_t)uniform(sh.e) * a.D;
    }
    const LaneQuad lq = lane_quad(k2, lane);
    // the row's activations and suh of chunk c (waves 0 and 1 rotate a 128-block each; the others load the same
    // addresses), then the trellis
    const int blk = wave & 1;
    const int k = c * 256 + blk * 128 + 2 * lane;
    const uint32_t xv = *reinterpret_cast<const uint32_t*>(static_cast<const uint16_t*>(a.x) + k);
    const uint32_t sv = *reinterpret_cast<const uint32_t*>(suh + k);
    u4v v[stage_loads<DL_KT>()];
    stage_issue<DL_KT>(sp, k2, lane, v);
    issued();
    uint32_t xh = xv, sh2 = sv;
    hold(xh);
    hold(sh2);
    if (wave < 2) {
        const bool bf = a.x_dtype == BF16;
        const uint16_t xl = (uint16_t)(xh & 0xffffu), xu = (uint16_t)(xh >> 16);
        float v0 = (bf ? bf2f(xl) : h2f(xl)) * h2f((uint16_t)(sh2 & 0xffffu));
        float v1 = (bf ? bf2f(xu) : h2f(xu)) * h2f((uint16_t)(sh2 >> 16));
        fwht128_w64(v0, v1, lane);
        *reinterpret_cast<uint32_t*>(sh.xs + blk * 128 + 2 * lane) =
            (uint32_t)f2h(v0 * HAD_SCALE) | ((uint32_t)f2h(v1 * HAD_SCALE) << 16);
    }
    __syncthreads();
    uint32_t* st = sh.stage[wave];
    stage_store<DL_KT>(st, k2, lane, v);
    f4v acc[2] = {f4v{0.f, 0.f, 0.f, 0.f}, f4v{0.f, 0.f, 0.f, 0.f}};
    const bool ok = l1_mfma_k2<CB, DL_KT>(k2, st, lq, sh.xs, lane, acc);
    if (!ok) {
        if (lane == 0) record_error(a.status, DEV_UNSUPPORTED_WIDTH);
        acc[0] = acc[1] = nan4();
    }
    // row 0's partial sums of this chunk: zp[q][nh][mat][c][128]
    if (lane < 16) {
        float* z = a.lay.zp + ((((size_t)q * NH + nh) * 2 + mat) * KC + c) * 128;
#pragma unroll
        for (int j = 0; j < 2; ++j) st_coh(z + (2 * wave + j) * 16 + lane, acc[j][0]);
    }
}

// The SwiGLU epilogue of (unit, column block nh) of the row's member q, after every chunk's partial sums are in:
// waves 0 and 1 sum the gate's and the up's chunks in order and rotate them (gu_out), wave 0 forms the down inputs.
__device__ __forceinline__ void l1_epilogue(const DLArgs& a, L1Sh& sh, const UnitView& uv, int nh, int q) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int KC = a.D / 256, NH = a.I / 128;
    uint32_t sd = 0;
    if (wave < 2) {
        const uint32_t sv = svh_pair(a, uv, nh, wave, lane);
        sd = suhd_pair(a, uv, nh, lane);
        const float* z = a.lay.zp + (((size_t)q * NH + nh) * 2 + wave) * KC * 128 + 2 * lane;
        float2 zv[DL_MAXKC];
#pragma unroll
        for (int cc = 0; cc < DL_MAXKC; ++cc) zv[cc] = ld_coh2(z + (cc < KC ? cc : KC - 1) * 128);
        const float2 o = gu_out(uv, zp_sum(a, zv), sv, lane);
        *reinterpret_cast<float2*>(&sh.gus[wave][2 * lane]) = o;
    }
    __syncthreads();
    if (wave == 0) {
        const float2 g = *reinterpret_cast<const float2*>(&sh.gus[0][2 * lane]);
        const float2 u = *reinterpret_cast<const float2*>(&sh.gus[1][2 * lane]);
        st_coh(reinterpret_cast<uint32_t*>(a.lay.xd + (size_t)q * a.I + nh * 128 + 2 * lane),
               act_pair(uv, g, u, sd, lane));
    }
}

// Down item (unit u, output column block cb) of the row's member q: its output columns of the unit (y or sy), then
// whether this block combines the column block.
template <int CB, int SCB, int NKT>
__device__ __forceinline__ void l1_down(const DLArgs& a, L1Sh& sh, const UnitView& uv, int u, int cb, int q) {
    const int lane = opaque_lane(threadIdx.x & 63), wave = uniform((int)threadIdx.x >> 6);
    const int NH = a.I / 128, DB = a.D / 128, KT = a.I / 16, ns = a.D / 16;
    const int nt0 = cb * 8 + 2 * wave;
    const int k2 = uv.shared ? a.sh_k2 : uniform(sh.tk), TWB = 16 * k2;
    TileSpan sp;
    if (uv.shared) {
        sp.r = buffer_rsrc(a.sh_w[2], (uint32_t)(KT * ns * TWB));
        sp.off = ((nt0 >> 3) * KT * 8 + (nt0 & 7)) * TWB;
        sp.kstride = 8 * TWB;
    } else {
        sp.r = buffer_rsrc(uniform(reinterpret_cast<const uint32_t*>(sh.tp)), (uint32_t)(KT * ns * TWB));
        sp.off = nt0 * TWB;
        sp.kstride = ns * TWB;
    }
    const LaneQuad lq = lane_quad(k2, lane);
    const uint16_t* svh = uv.shared ? a.sh_svh[2] : a.svh_d + (size_t)uv.e * a.D;
    uint32_t sd = *reinterpret_cast<const uint32_t*>(svh + cb * 128 + 2 * lane);
    u4v v[stage_loads<NKT>()];
    stage_issue<NKT>(sp, k2, lane, v);
    issued();
    hold(sd);
    // both column blocks of the unit's down inputs ready
    if (threadIdx.x == 0) {
        int n = 0;
        while (ld_coh(l1_urdy(a.lay.sync, u)) < NH) {
            if (++n > (1 << 18)) {
                record_error(a.status, DEV_SYNC_TIMEOUT);
                break;
            }
            __builtin_amdgcn_s_sleep(2);
        }
        sh.flag = n > (1 << 18);
    }
    __syncthreads();
    const bool timed_out = sh.flag;
    if (threadIdx.x < a.I / 2)
        reinterpret_cast<uint32_t*>(sh.xs)[threadIdx.x] =
            ld_coh(reinterpret_cast<const uint32_t*>(a.lay.xd + (size_t)q * a.I) + threadIdx.x);
    __syncthreads();
    uint32_t* st = sh.stage[wave];
    stage_store<NKT>(st, k2, lane, v);
    f4v acc[2] = {f4v{0.f, 0.f, 0.f, 0.f}, f4v{0.f, 0.f, 0.f, 0.f}};
    const bool ok = uv.shared ? l1_mfma_k2<SCB, NKT>(k2, st, lq, sh.xs, lane, acc)
                              : l1_mfma_k2<CB, NKT>(k2, st, lq, sh.xs, lane, acc);
    if (!ok || timed_out) {
        if (lane == 0 && !ok) record_error(a.status, DEV_UNSUPPORTED_WIDTH);
        acc[0] = acc[1] = nan4();
    }
    __syncthreads();  // every wave is done with its staging: the column sums take its place
    if (lane < 16) {
#pragma unroll
        for (int j = 0; j < 2; ++j) sh.ys[(2 * wave + j) * 16 + lane] = acc[j][0];
    }
    __syncthreads();
    if (wave == 0) {
        float v0 = sh.ys[2 * lane], v1 = sh.ys[2 * lane + 1];
        fwht128_w64(v0, v1, lane);
        const float s0 = h2f((uint16_t)(sd & 0xffffu)), s1 = h2f((uint16_t)(sd >> 16));
        float* dst = uv.shared ? a.lay.sy : a.yroute + (size_t)q * a.D;
        st_coh2(dst + cb * 128 + 2 * lane, float2{v0 * HAD_SCALE * s0, v1 * HAD_SCALE * s1});
    }
    stores_done();
    __syncthreads();
    if (threadIdx.x == 0) {
        const bool last = count_in(l1_ccnt(a.lay.sync, cb)) == a.U - 1;
        if (last) reset_count(l1_ccnt(a.lay.sync, cb));
        if (count_in(l1_dcnt(a.lay.sync, u)) == DB - 1) {  // every down block of the unit is past its wait
            reset_count(l1_urdy(a.lay.sync, u));
            reset_count(l1_dcnt(a.lay.sync, u));
        }
        sh.flag = last;
    }
    __syncthreads();
    if (sh.flag && wave == 0) {
        // the combine of the column block: the slots in order from 0 (exl3_experts.cu:256-267), then the shared expert
        const int n = cb * 128 + 2 * lane;
        float2 y[DL_SLOTS];
#pragma unroll
        for (int k = 0; k < DL_SLOTS; ++k) y[k] = ld_coh2(a.yroute + (size_t)k * a.D + n);
        float2 sv = a.hs ? ld_coh2(a.lay.sy + n) : float2{0.f, 0.f};
        float a0 = 0.f, a1 = 0.f;
#pragma unroll
        for (int k = 0; k < DL_SLOTS; ++k) {
            a0 = __builtin_fmaf(sh.wts[k], y[k].x, a0);
            a1 = __builtin_fmaf(sh.wts[k], y[k].y, a1);
        }
        if (a.hs) {
            a0 = a0 + sv.x;
            a1 = a1 + sv.y;
        }
        *reinterpret_cast<float2*>(a.out + n) = float2{a0, a1};
    }
}

template <int CB, int SCB>
__global__ void __launch_bounds__(DL_THREADS) __attribute__((amdgpu_waves_per_eu(6))) layer1_kernel(DLArgs a) {
    __shared__ L1Sh sh;
    const int NH = a.I / 128, KC = a.D / 256, DB = a.D / 128;
    const int GU = NH * 2 * KC;  // gate|up items a unit
    const int b = blockIdx.x;
    UnitView uv;
    uv.nm = 1;
    uv.mem = nullptr;
    if (b < a.U * GU) {
        const int u = b / GU, rem = b % GU, nh = rem / (2 * KC), mat = (rem / KC) & 1, c = rem % KC;
        uv.shared = a.hs && u == 0;
        const int q = uv.shared ? DL_SLOTS : u - a.hs;
        if (uv.shared) {
            uv.e = -1;
            l1_gateup<SCB, true>(a, sh, u, nh, mat, c, q);
        } else {
            const bool publisher = b == a.hs * GU;  // hands pick / wts to the caller
            l1_route(a, sh, mat, u - a.hs + 1, publisher ? DL_SLOTS : u - a.hs + 1);
            if (publisher && threadIdx.x < DL_SLOTS) {
                a.pick[threadIdx.x] = sh.pick[threadIdx.x];
                a.wts[threadIdx.x] = sh.wts[threadIdx.x];
            }
            uv.e = uniform(sh.e);
            l1_gateup<CB, false>(a, sh, u, nh, mat, c, q);
        }
        stores_done();
        __syncthreads();
        if (threadIdx.x == 0) {
            const bool last = count_in(l1_gcnt(a.lay.sync, u, nh)) == 2 * KC - 1;
            if (last) reset_count(l1_gcnt(a.lay.sync, u, nh));
            sh.flag = last;
        }
        __syncthreads();
        if (!sh.flag) return;
        l1_epilogue(a, sh, uv, nh, q);
        stores_done();
        __syncthreads();
        if (threadIdx.x == 0) count_in(l1_urdy(a.lay.sync, u));
        return;
    }
    const int d = b - a.U * GU, u = d / DB, cb = d % DB;
    uv.shared = a.hs && u == 0;
    const int q = uv.shared ? DL_SLOTS : u - a.hs;
    // every down block routes the whole row: the last of a column block combines all eight slots with their weights
    l1_route(a, sh, 2, uv.shared ? 1 : u - a.hs + 1, DL_SLOTS);
    uv.e = uv.shared ? -1 : uniform(sh.e);
    if (a.I == 256)
        l1_down<CB, SCB, 16>(a, sh, uv, u, cb, q);
    else
        l1_down<CB, SCB, 8>(a, sh, uv, u, cb, q);
}

// ---- host side ----------------------------------------------------------------------------------------------------

static size_t align256(size_t n) { return (n + 255) & ~(size_t)255; }

// Region offsets for a scratch of `rows` rows (capacity), in bytes from the region's base.
struct DLCarve {
    size_t sync, zp, xd, sy, ws, total;
    size_t U, NH, DB;
};

static DLCarve dl_carve(uint32_t rows, uint32_t D, uint32_t I, uint32_t E) {
    DLCarve c{};
    const size_t P = (size_t)rows * DL_SLOTS, Q = P + rows;
    c.U = 1 + (P < E ? P : E);
    c.NH = I / 128;
    c.DB = D / 128;
    const size_t KC = D / 256;
    size_t off = 0;
    auto take = [&](size_t bytes) {
        const size_t at = off;
        off += align256(bytes);
        return at;
    };
    c.sync = take(L1_SYNC_BYTES);
    c.zp = take(Q * c.NH * 2 * KC * 128 * 4);
    c.xd = take(Q * I * 2);
    c.sy = take((size_t)rows * D * 4);
    c.ws = take((size_t)DL_MAXP * 3 * 8 + ((size_t)DL_MAXP + 1 + (size_t)DL_MAXP * DL_MAXR + 4 * DL_MAXP) * 4);
    c.total = off;
    return c;
}

static bool dl_shape_ok(uint32_t rows, uint32_t slots, uint32_t D, uint32_t I, uint32_t E) {
    return rows >= 1 && rows <= DL_MAXR && slots == DL_SLOTS && D >= 256 && D % 256 == 0 && D <= 256 * DL_MAXKC &&
           (I == 128 || I == DL_MAXI) && E >= 1 && E <= DL_MAXE;
}

// Bytes of the two launches' region in a moe scratch of `rows` rows: zero when the shape has no such path.
size_t dl_region_bytes(uint32_t rows, uint32_t slots, uint32_t D, uint32_t I, uint32_t E) {
    return dl_shape_ok(rows, slots, D, I, E) ? dl_carve(rows, D, I, E).total : 0;
}

static DLLayout dl_layout(uint64_t base, uint32_t rows, uint32_t D, uint32_t I, uint32_t E) {
    const DLCarve c = dl_carve(rows, D, I, E);
    DLLayout l;
    l.sync = dptr<int>(base + c.sync);
    l.zp = dptr<float>(base + c.zp);
    l.xd = dptr<uint16_t>(base + c.xd);
    l.sy = dptr<float>(base + c.sy);
    l.tptr = dptr<uint64_t>(base + c.ws);  // 256-byte aligned
    int* ws = dptr<int>(base + c.ws + (size_t)DL_MAXP * 3 * 8);
    l.uids = ws;
    l.ucount = ws + DL_MAXP;
    l.members = l.ucount + 1;
    l.mcount = l.members + DL_MAXP * DL_MAXR;
    l.tk2 = l.mcount + DL_MAXP;
    return l;
}

// Stage events for benchmarks (ea_profile_enable): recorded on the call's stream around the layer's stages (route
// and gate|up, epilogue, down, combine).
constexpr int DL_STAGES = 4;
struct DLProfile {
    bool on = false, recorded = false;
    hipEvent_t ev[DL_STAGES + 1] = {};
};
static DLProfile g_prof[64];

static DLProfile* profile_of(int device) { return device >= 0 && device < 64 ? &g_prof[device] : nullptr; }

static void mark_stage(hipStream_t s, int device, int k) {
    DLProfile* p = profile_of(device);
    if (p && p->on) {
        (void)hipEventRecord(p->ev[k], s);
        if (k == DL_STAGES) p->recorded = true;
    }
}

template <int CB, int SCB>
static int dl_launch(hipStream_t s, const DLArgs& a, int cus, int device) {
    static int per_cu = 0, per_cu_wide = 0;  // resident gate|up blocks a CU, once per instantiation
    if (per_cu == 0) {
        int n = 0;
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, gateup_kernel<CB, SCB>, DL_THREADS, 0) != hipSuccess ||
            n < 1)
            n = 1;
        per_cu = n;
        n = 0;
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, gateup_wide_kernel<CB, SCB>, 2 * DL_THREADS, 0) !=
                hipSuccess ||
            n < 1)
            n = 1;
        per_cu_wide = n;
    }
    const int NH = a.I / 128, KC = a.D / 256, DB = a.D / 128;
    mark_stage(s, device, 0);
    if (a.router_w) {
        // the router's logits first (ops.router: ea_router's launch), into the caller's logits buffer
        const int r = launch_router(s, a.x, a.x_dtype, (uint32_t)a.x_stride, a.router_w, nullptr,
                                    const_cast<float*>(a.logits), (uint32_t)a.R, (uint32_t)a.D, 256u);
        if (r) return r;
    }
    if (a.R == 1 && a.logits) {
        // one row routed from logits: the whole layer in one launch (the stage events then all follow it)
        layer1_kernel<CB, SCB><<<a.U * NH * 2 * KC + a.U * DB, DL_THREADS, 0, s>>>(a);
        const int r = launched();
        if (r) return r;
        for (int k = 1; k <= DL_STAGES; ++k) mark_stage(s, device, k);
        return EA_OK;
    }
    const bool wide = a.R > 1 && NH == 2;  // items over both column blocks
    const int items = a.U * (wide ? 1 : NH) * 2 * KC;
    int grid = (wide ? per_cu_wide : per_cu) * cus;
    if (grid > items) grid = items;
    if (a.R > 1) {
        route_kernel<<<1, DL_ROUTE_THREADS, 0, s>>>(a);
        const int r = launched();
        if (r) return r;
    }
    if (wide)
        gateup_wide_kernel<CB, SCB><<<grid, 2 * DL_THREADS, 0, s>>>(a);
    else
        gateup_kernel<CB, SCB><<<grid, DL_THREADS, 0, s>>>(a);
    int r = launched();
    if (r) return r;
    mark_stage(s, device, 1);
    constexpr int FCB = DL_FOLD_WAVES / 4;  // column blocks a fold block
    if (a.R == 1 && DB % FCB == 0) {
        // one row: the down launch computes its own inputs (the epilogue stage is empty)
        mark_stage(s, device, 2);
        down_fold_kernel<CB, SCB><<<a.U * (DB / FCB), 64 * DL_FOLD_WAVES, 0, s>>>(a);
        if ((r = launched())) return r;
    } else {
        epilogue_kernel<<<a.U * NH * ((a.R + DL_WAVES - 1) / DL_WAVES), DL_THREADS, 0, s>>>(a);
        if ((r = launched())) return r;
        mark_stage(s, device, 2);
        down_kernel<CB, SCB><<<a.U * DB, DL_THREADS, 0, s>>>(a);
        if ((r = launched())) return r;
    }
    mark_stage(s, device, 3);
    combine_kernel<<<(a.R * DB + DL_WAVES - 1) / DL_WAVES, DL_THREADS, 0, s>>>(a);
    if ((r = launched())) return r;
    mark_stage(s, device, 4);
    return EA_OK;
}

// The decode layer in three to five launches: routing from logits (when given), the routed experts of `ex`, the shared expert
// (when given) and their sum into out [R, D]. EA_UNPORTED_GROUPED_VARIANT when the shape, widths or codebooks are
// not instantiated here; the caller then runs the launch sequence.
int decode_layer(hipStream_t s, const void* x, int x_dtype, uint32_t x_stride, const float* logits,
                 const float* bias, float scale, int32_t* pick, float* wts, const ea_routed* ex,
                 const ea_linear* const* shared, const ea_moe_scratch* sc, float* out, uint32_t R,
                 const void* router_w) {
    EA_REQUIRE_CTX(c);
    const uint32_t D = ex->dims, I = ex->width, E = ex->count, slots = sc->slots;
    if (!sc->fused || R > sc->rows || !dl_shape_ok(sc->rows, slots, D, I, E)) return EA_UNPORTED_GROUPED_VARIANT;
    if (ex->k2_gu[0] < 2 || ex->k2_gu[1] > 10 || ex->k2_d[0] < 2 || ex->k2_d[1] > 10) return EA_UNPORTED_GROUPED_VARIANT;
    if (logits && E != 256) return EA_UNPORTED_GROUPED_VARIANT;
    if (x_dtype != EA_F16 && x_dtype != EA_BF16) return EA_UNPORTED_GROUPED_VARIANT;
    // activation rows are read a word (two values) at a time
    if ((reinterpret_cast<uintptr_t>(x) & 3) || (x_stride & 1)) return EA_UNPORTED_GROUPED_VARIANT;
    if (router_w) {
        // the router launch's own conditions, checked before anything is launched
        if (!logits || E != 256) return EA_BAD_ARGUMENT;
        if (D % 512 != 0) return EA_UNEVEN_SPLIT;
        if (x_stride < D || x_stride % 4 != 0) return EA_BAD_ROW_STRIDE;
        if ((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(router_w)) & 7) return EA_BAD_ARGUMENT;
    }
    int scb = (int)ex->cb;
    DLArgs a{};
    if (shared) {
        const ea_linear *g = shared[0], *u = shared[1], *d = shared[2];
        if (!g || !u || !d) return EA_BAD_ARGUMENT;
        if (g->k != D || u->k != D || g->n != I || u->n != I || d->k != I || d->n != D) return EA_BAD_WIDTH;
        if (g->k2 != u->k2 || g->k2 != d->k2 || g->cb != u->cb || g->cb != d->cb) return EA_UNPORTED_GROUPED_VARIANT;
        if (g->k2 < 2 || g->k2 > 10) return EA_UNPORTED_GROUPED_VARIANT;
        scb = (int)g->cb;
        a.hs = 1;
        a.sh_k2 = (int)g->k2;
        for (int m = 0; m < 3; ++m) {
            a.sh_w[m] = dptr<const uint32_t>(shared[m]->words);
            a.sh_suh[m] = dptr<const uint16_t>(shared[m]->suh);
            a.sh_svh[m] = dptr<const uint16_t>(shared[m]->svh);
        }
    }
    a.logits = logits;
    a.router_w = router_w;
    a.bias = bias;
    a.scale = scale;
    a.pick = pick;
    a.wts = wts;
    a.x = x;
    a.x_dtype = x_dtype;
    a.x_stride = (int)x_stride;
    for (int m = 0; m < 3; ++m) {
        a.ptr[m] = dptr<const int64_t>(ex->ptr[m]);
        a.k2t[m] = dptr<const int32_t>(ex->k2[m]);
    }
    a.suh_g = dptr<const uint16_t>(ex->suh_g);
    a.suh_u = dptr<const uint16_t>(ex->suh_u);
    a.svh_g = dptr<const uint16_t>(ex->svh_g);
    a.svh_u = dptr<const uint16_t>(ex->svh_u);
    a.suh_d = dptr<const uint16_t>(ex->suh_d);
    a.svh_d = dptr<const uint16_t>(ex->svh_d);
    a.E = (int)E;
    a.out = out;
    a.yroute = dptr<float>(sc->y);
    a.lay = dl_layout(sc->fused, sc->rows, D, I, E);
    a.R = (int)R;
    a.D = (int)D;
    a.I = (int)I;
    const uint32_t P = R * DL_SLOTS;
    a.U = a.hs + (int)(P < E ? P : E);
    a.status = c->status;
    const int rcb = (int)ex->cb;
    if (rcb == 1 && scb == 1) return dl_launch<1, 1>(s, a, c->cus, c->device);
    if (rcb == 1 && scb == 2) return dl_launch<1, 2>(s, a, c->cus, c->device);
    if (rcb == 2 && scb == 2) return dl_launch<2, 2>(s, a, c->cus, c->device);
    if (rcb == 2 && scb == 1) return dl_launch<2, 1>(s, a, c->cus, c->device);
    return EA_UNPORTED_GROUPED_VARIANT;
}

// ---- the allocation-free variant's scratch --------------------------------------------------------------------------

// The scratch of ea_ffn_moe_decode_static: the per-pair down outputs and the decode layer's region, carved for
// DL_MAXR rows of the call's layer shape. The largest shape the decode layer takes (D 6144, I 256) needs 10.7 MB.
// Every call on a device shares that device's copy, which holds the last call's contents: the layer writes every
// value it reads back within a call, and the one-row launch's counters, which must start at zero, are cleared by
// ea_init and left at zero by every launch.
constexpr size_t DL_STATIC_BYTES = (size_t)12 << 20;
static __device__ __align__(256) uint8_t scratch[DL_STATIC_BYTES];

// The byte offsets of the per-pair outputs and the region in the static scratch for a layer shape; false when the
// layout does not fit.
static bool dl_static_carve(uint32_t D, uint32_t I, uint32_t E, size_t& y_off, size_t& region_off) {
    if (!dl_shape_ok(DL_MAXR, DL_SLOTS, D, I, E)) return false;
    region_off = 0;  // the region first: its counters then sit at the array's start for every layer shape
    y_off = dl_carve(DL_MAXR, D, I, E).total;
    return y_off + align256((size_t)DL_MAXP * D * 4) <= DL_STATIC_BYTES;
}

int dl_static_setup(DevCtx& c) {
    void* p = nullptr;
    int r = hip_status(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
    if (r) return r;
    if (!p) return EA_HIP_FAILED;
    r = hip_status(hipMemset(p, 0, DL_STATIC_BYTES));
    if (r) return r;
    c.static_scratch = p;
    return EA_OK;
}

}  // namespace ea

using namespace ea;

extern "C" {

int ea_ffn_moe_decode_static(ea_stream_t stream, const void* x, int x_dtype, uint32_t x_stride, const float* logits,
                             const float* bias, float scale, int32_t* pick, float* wts, const ea_routed* ex,
                             const ea_linear* const* shared, float* out, uint32_t R) {
    EA_REQUIRE_CTX(c);
    if (!x || !logits || !bias || !pick || !wts || !ex || !out) return EA_BAD_ARGUMENT;
    if (!c->static_scratch) return EA_NOT_INITIALIZED;
    if (R > (uint32_t)DL_MAXR) return EA_SCRATCH_TOO_SMALL;
    size_t y_off = 0, region_off = 0;
    if (!dl_static_carve(ex->dims, ex->width, ex->count, y_off, region_off)) return EA_SCRATCH_TOO_SMALL;
    if (R == 0) return EA_OK;
    const uint64_t base = reinterpret_cast<uintptr_t>(c->static_scratch);
    ea_moe_scratch sc{};
    sc.y = base + y_off;
    sc.fused = base + region_off;
    sc.rows = DL_MAXR;
    sc.slots = DL_SLOTS;
    return decode_layer(as_stream(stream), x, x_dtype, x_stride, logits, bias, scale, pick, wts, ex, shared, &sc, out,
                        R, nullptr);
}

int ea_profile_enable(int on) {
    EA_REQUIRE_CTX(c);
    DLProfile* p = profile_of(c->device);
    if (!p) return EA_BAD_ARGUMENT;
    if (on && !p->ev[0])
        for (int k = 0; k <= DL_STAGES; ++k) {
            const int r = hip_status(hipEventCreate(&p->ev[k]));
            if (r) return r;
        }
    p->on = on != 0;
    p->recorded = false;
    return EA_OK;
}

int ea_profile_stages(float* ms, uint32_t n) {
    EA_REQUIRE_CTX(c);
    DLProfile* p = profile_of(c->device);
    if (!p || !ms || n < (uint32_t)DL_STAGES) return EA_BAD_ARGUMENT;
    if (!p->recorded) return EA_INVALID;
    int r = hip_status(hipEventSynchronize(p->ev[DL_STAGES]));
    if (r) return r;
    for (int k = 0; k < DL_STAGES; ++k) {
        r = hip_status(hipEventElapsedTime(&ms[k], p->ev[k], p->ev[k + 1]));
        if (r) return r;
    }
    return EA_OK;
}

int ea_ffn_moe_decode(ea_stream_t stream, const void* x, int x_dtype, uint32_t x_stride, const float* logits,
                      const float* bias, float scale, int32_t* pick, float* wts, const ea_routed* ex,
                      const ea_linear* const* shared, const ea_moe_scratch* sc, float* out, uint32_t R) {
    EA_REQUIRE_CTX(c);
    if (!x || !logits || !bias || !pick || !wts || !ex || !sc || !out) return EA_BAD_ARGUMENT;
    if (R > sc->rows) return EA_SCRATCH_TOO_SMALL;
    if (R == 0) return EA_OK;
    return decode_layer(as_stream(stream), x, x_dtype, x_stride, logits, bias, scale, pick, wts, ex, shared, sc, out,
                        R, nullptr);
}

int ea_ffn_moe_decode_router(ea_stream_t stream, const void* x, int x_dtype, uint32_t x_stride, const void* router_w,
                             float* logits, const float* bias, float scale, int32_t* pick, float* wts,
                             const ea_routed* ex, const ea_linear* const* shared, const ea_moe_scratch* sc, float* out,
                             uint32_t R) {
    EA_REQUIRE_CTX(c);
    if (!x || !router_w || !logits || !bias || !pick || !wts || !ex || !sc || !out) return EA_BAD_ARGUMENT;
    if (R > sc->rows) return EA_SCRATCH_TOO_SMALL;
    if (R == 0) return EA_OK;
    return decode_layer(as_stream(stream), x, x_dtype, x_stride, logits, bias, scale, pick, wts, ex, shared, sc, out,
                        R, router_w);
}

}  // extern "C"
