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
#include "ea_stamps.hpp"

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
constexpr size_t L1_SYNC_BYTES = 16384;      // the one-row launch's epoch and check-in words

// The one-row launch's tagged slots (8 bytes each: a value's bits, then the launch's tag), at offsets fixed for every
// layer shape: sized for the largest one (9 units, I 256, D 6144).
constexpr int L1_UNITS = 1 + DL_SLOTS;                  // the shared expert and the eight picks
constexpr int L1_MAXNH = DL_MAXI / 128;                 // gate|up column blocks of 128
constexpr int L1_MAXDB = 256 * DL_MAXKC / 128;          // output column blocks of 128
constexpr int L1_MAXB = 1 + L1_UNITS * (L1_MAXNH * 2 * DL_MAXKC + L1_MAXDB);  // blocks of the largest launch
constexpr int L1_CHK = 64;                              // words before the check-in words (the epoch word's line)
constexpr size_t L1_TZ = (size_t)L1_UNITS * L1_MAXNH * 2 * DL_MAXKC * 128;  // gate|up partial sums
constexpr size_t L1_TXD = (size_t)L1_UNITS * DL_MAXI / 2;                   // down inputs, two fp16 a slot
constexpr size_t L1_TY = (size_t)L1_UNITS * 256 * DL_MAXKC;                 // down outputs
constexpr size_t L1_TAG_BYTES = (L1_TZ + L1_TXD + L1_TY) * 8;
constexpr int L1_RT = 1024;                             // u64 slots before the routing slots (byte 8192)
constexpr int L1_RT_SLOTS = 2 * DL_SLOTS + 3 * DL_SLOTS * 3;  // picks, weights, each pick's three tables
static_assert((L1_CHK + L1_MAXB + 1) * 4 <= L1_RT * 8, "the check-in words end before the routing slots");
static_assert((L1_RT + L1_RT_SLOTS) * 8 <= (int)L1_SYNC_BYTES, "the routing slots fit the sync region");

// Scratch of the layer's launches, carved on the host for the scratch's row capacity (any R up to it runs).
struct DLLayout {
    int* sync;          // the one-row launch's epoch word and check-in words (first in the region)
    uint64_t* tz;       // the one-row launch's tagged slots: [U, NH, 2, KC, 128] gate|up partial sums,
    uint64_t* txd;      //   [U, I / 2] down inputs,
    uint64_t* ty;       //   [U, D] down outputs (all right after the sync words)
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
// Every entry of the three matrices is read (all three tables are always set), before any is stored: reads chosen
// between LDS and memory by one expression became flat loads that waited one by one.
__device__ __forceinline__ void route_tables(const DLArgs& a, RouteSh& sh, int mats) {
    for (int u = threadIdx.x; u < sh.ucount; u += DL_THREADS) {
        const int e = sh.uids[u];
        uint64_t p[3];
        int k[3];
        if (a.logits) {
#pragma unroll
            for (int m = 0; m < 3; ++m) {
                p[m] = sh.r.tptr[m][e];
                k[m] = sh.r.tk2[m][e];
            }
        } else {
#pragma unroll
            for (int m = 0; m < 3; ++m) {
                p[m] = (uint64_t)a.ptr[m][e];
                k[m] = a.k2t[m][e];
            }
        }
#pragma unroll
        for (int m = 0; m < 3; ++m)
            if (m < mats) {
                sh.uptr[u][m] = p[m];
                sh.uk2[u][m] = k[m];
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

// An item's loads in flight: the members' activations and suh of its k chunk (a wave a (row, 128-block) task), then
// its trellis words.
template <int NW>
struct GuFetch {
    static constexpr int MT = 2 * DL_MAXR / NW;
    uint32_t xv[MT], sv[MT];
    u4v v[stage_loads<DL_KT>()];
};

// The item's loads: activations and suh first, then the trellis (loads complete in order, so the rotation waits only
// for the first ones while the trellis is in flight).
template <int NW>
__device__ __forceinline__ void gateup_issue(const DLArgs& a, const UnitView& uv, const TileSpan& sp, int k2,
                                             const uint16_t* suh, int c, int lane, int wave, GuFetch<NW>& f) {
    constexpr int MT = GuFetch<NW>::MT;
    const int ntask = 2 * uv.nm;
#pragma unroll
    for (int i = 0; i < MT; ++i) {
        const int task = min(wave + NW * i, ntask - 1);  // unconditional (see stage_issue); extra lanes repeat
        const int m = task >> 1, blk = task & 1;
        const int k = c * 256 + blk * 128 + 2 * lane;
        const uint16_t* xr = static_cast<const uint16_t*>(a.x) + (size_t)member_row(uv, m) * a.x_stride;
        f.xv[i] = *reinterpret_cast<const uint32_t*>(xr + k);
        f.sv[i] = *reinterpret_cast<const uint32_t*>(suh + k);
    }
    stage_issue<DL_KT>(sp, k2, lane, f.v);
    issued();
}

// The item's product from its loads: rotate the activations of the k chunk into xs (xs[m][k] = fp16(((x * suh) @ H) *
// HAD_SCALE)), then, after the block barrier, the trellis into the wave's LDS region and the MFMAs.
template <int CB, int NW>
__device__ __forceinline__ bool gateup_consume(const DLArgs& a, const UnitView& uv, int k2, GuFetch<NW>& f,
                                               uint16_t* xs, uint32_t* st, int lane, int wave, f4v (&acc)[2]) {
    constexpr int MT = GuFetch<NW>::MT;
    const LaneQuad lq = lane_quad(k2, lane);
    const int ntask = 2 * uv.nm;
    const bool bf = a.x_dtype == BF16;
#pragma unroll
    for (int i = 0; i < MT; ++i) {
        const int task = wave + NW * i;
        if (task < ntask) {
            const int m = task >> 1, blk = task & 1;
            const uint16_t xl = (uint16_t)(f.xv[i] & 0xffffu), xh = (uint16_t)(f.xv[i] >> 16);
            const float x0 = bf ? bf2f(xl) : h2f(xl);
            const float x1 = bf ? bf2f(xh) : h2f(xh);
            float v0 = x0 * h2f((uint16_t)(f.sv[i] & 0xffffu));
            float v1 = x1 * h2f((uint16_t)(f.sv[i] >> 16));
            fwht128_w64(v0, v1, lane);
            *reinterpret_cast<uint32_t*>(xs + m * DL_RS + blk * 128 + 2 * lane) =
                (uint32_t)f2h(v0 * HAD_SCALE) | ((uint32_t)f2h(v1 * HAD_SCALE) << 16);
        }
    }
    __syncthreads();
    stage_store<DL_KT>(st, k2, lane, f.v);
    return mfma_tiles_k2<CB, DL_KT>(k2, st, lq, xs, uv.nm, lane, acc);
}

// The item's product for one width: its loads, then (the trellis still in flight) the rotation and the MFMAs.
template <int CB, int NW>
__device__ __forceinline__ bool gateup_product(const DLArgs& a, const UnitView& uv, const TileSpan& sp, int k2,
                                               const uint16_t* suh, int c, uint16_t* xs, uint32_t* st,
                                               f4v (&acc)[2]) {
    const int lane = opaque_lane(threadIdx.x & 63), wave = uniform((int)threadIdx.x >> 6);
    GuFetch<NW> f;
    gateup_issue<NW>(a, uv, sp, k2, suh, c, lane, wave, f);
#pragma unroll
    for (int i = 0; i < GuFetch<NW>::MT; ++i) {
        hold(f.xv[i]);
        hold(f.sv[i]);
    }
    return gateup_consume<CB, NW>(a, uv, k2, f, xs, st, lane, wave, acc);
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
// A gate|up item: its unit, the wave's column tiles and where its matrix's tiles are.
struct GuItem {
    UnitView uv;
    TileSpan sp;
    int k2, nh, mat, c, wl;
    const uint16_t* suh;
};
template <bool SHARED, int NW>
__device__ __forceinline__ GuItem gateup_describe(const DLArgs& a, RouteSh& sh, int u, int nh, int mat, int c) {
    static_assert(NW == DL_WAVES || NW == 2 * DL_WAVES, "one or both column blocks of 128");
    const int wave = uniform((int)threadIdx.x >> 6);
    GuItem it;
    it.wl = wave & (DL_WAVES - 1);  // the wave within its column block
    if (NW != DL_WAVES) nh = wave / DL_WAVES;
    it.nh = nh;
    it.mat = mat;
    it.c = c;
    it.uv.shared = SHARED;
    const int ur = u - a.hs;
    it.uv.nm = SHARED ? a.R : uniform(sh.mcount[ur]);
    it.uv.e = SHARED ? -1 : uniform(sh.uids[ur]);
    it.uv.mem = SHARED ? nullptr : sh.members[ur];
    // wave w: n tiles nh * 8 + 2w, + 1 over the 16 k tiles of chunk c
    const int nt0 = nh * 8 + 2 * it.wl, kt0 = c * DL_KT;
    // matrix D x I: routed in the expert layout (tile (kt, nt) at (kt * I / 16 + nt) * TW words), the shared expert
    // in strips ([I / 128][D / 16][8][TW])
    const int ns = a.I / 16;
    if constexpr (SHARED) {
        it.k2 = a.sh_k2;
        const int TWB = 16 * it.k2;  // bytes a tile
        it.sp.r = buffer_rsrc(mat ? a.sh_w[1] : a.sh_w[0], (uint32_t)((a.D / 16) * ns * TWB));
        it.sp.off = ((nt0 >> 3) * (a.D / 16) * 8 + kt0 * 8 + (nt0 & 7)) * TWB;
        it.sp.kstride = 8 * TWB;
        it.suh = mat ? a.sh_suh[1] : a.sh_suh[0];
    } else {
        it.k2 = uniform(sh.uk2[ur][mat]);
        const uint32_t* T = uniform(reinterpret_cast<const uint32_t*>(sh.uptr[ur][mat]));
        const int TWB = 16 * it.k2;
        it.sp.r = buffer_rsrc(T, (uint32_t)((a.D / 16) * ns * TWB));
        it.sp.off = (kt0 * ns + nt0) * TWB;
        it.sp.kstride = ns * TWB;
        it.suh = (mat ? a.suh_u : a.suh_g) + (size_t)it.uv.e * a.D;
    }
    return it;
}

// The item's partial sums of its chunk: zp[q][nh][mat][c][128] (NaN when the width had no decoder).
__device__ __forceinline__ void gateup_store(const DLArgs& a, const GuItem& it, bool ok, f4v (&acc)[2], int lane) {
    const int KC = a.D / 256, NH = a.I / 128;
    if (!ok) {
        if (lane == 0) record_error(a.status, DEV_UNSUPPORTED_WIDTH);
        acc[0] = acc[1] = nan4();
    }
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int m = 4 * (lane >> 4) + i;
            if (m < it.uv.nm) {
                const int col = (2 * it.wl + j) * 16 + (lane & 15);
                a.lay.zp[((((size_t)member_q(a, it.uv, m) * NH + it.nh) * 2 + it.mat) * KC + it.c) * 128 + col] =
                    acc[j][i];
            }
        }
}

template <int CB, bool SHARED, int NW = DL_WAVES>
__device__ __forceinline__ void gateup_item(const DLArgs& a, RouteSh& sh, int u, int nh, int mat, int c,
                                            uint16_t* xs, uint32_t* st) {
    const int lane = threadIdx.x & 63;
    const GuItem it = gateup_describe<SHARED, NW>(a, sh, u, nh, mat, c);
    f4v acc[2] = {f4v{0.f, 0.f, 0.f, 0.f}, f4v{0.f, 0.f, 0.f, 0.f}};
    const bool ok = gateup_product<CB, NW>(a, it.uv, it.sp, it.k2, it.suh, c, xs, st, acc);
    gateup_store(a, it, ok, acc, lane);
}

// A block's routed items it, it + G, it + 2G, ... (G = gridDim.x) over both column blocks (NW = 2 DL_WAVES), each
// item's loads issued before the previous item's product runs, so an item's load latency hides behind its
// predecessor's decode and MFMAs instead of standing between them.
template <int CB, int NW>
__device__ __forceinline__ void gateup_routed_pipelined(const DLArgs& a, RouteSh& sh, int it, int items, int units,
                                                        uint16_t* xs, uint32_t* st, int& dirty) {
    const int lane = opaque_lane(threadIdx.x & 63), wave = uniform((int)threadIdx.x >> 6);
    const int KC = a.D / 256, per_unit = 2 * KC, G = (int)gridDim.x;
    auto valid = [&](int i) { return i < items && i / per_unit < units; };
    auto describe = [&](int i) {
        const int rem = i % per_unit;
        return gateup_describe<false, NW>(a, sh, i / per_unit, 0, rem / KC, rem % KC);
    };
    auto run = [&](const GuItem& cur, GuFetch<NW>& f) __attribute__((always_inline)) {
        const int nm = cur.uv.nm;
        if (nm < dirty) zero_rows<64 * NW>(xs, nm, dirty);
        f4v acc[2] = {f4v{0.f, 0.f, 0.f, 0.f}, f4v{0.f, 0.f, 0.f, 0.f}};
        // the lane id made opaque in every item: the widths' lane constants are then formed in the item, not held
        // across the loop
        const int ln = opaque_lane(threadIdx.x & 63);
        const bool ok = gateup_consume<CB, NW>(a, cur.uv, cur.k2, f, xs, st, ln, wave, acc);
        gateup_store(a, cur, ok, acc, ln);
        dirty = nm;
        __syncthreads();
    };
    if (!valid(it)) return;
    GuFetch<NW> fa, fb;
    GuItem ca = describe(it), cb;
    gateup_issue<NW>(a, ca.uv, ca.sp, ca.k2, ca.suh, ca.c, lane, wave, fa);
    for (;;) {
        int nx = it + G;
        bool more = valid(nx);
        if (more) {
            cb = describe(nx);
            gateup_issue<NW>(a, cb.uv, cb.sp, cb.k2, cb.suh, cb.c, lane, wave, fb);
        }
        run(ca, fa);
        if (!more) break;
        it = nx;
        nx = it + G;
        more = valid(nx);
        if (more) {
            ca = describe(nx);
            gateup_issue<NW>(a, ca.uv, ca.sp, ca.k2, ca.suh, ca.c, lane, wave, fa);
        }
        run(cb, fb);
        if (!more) break;
        it = nx;
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
__global__ void __launch_bounds__(2 * DL_THREADS) __attribute__((amdgpu_waves_per_eu(4)))
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
    gateup_routed_pipelined<CB, NW>(a, sh, it, items, a.hs + sh.ucount, xs, st, dirty);
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
// One row routed from logits runs as a single launch of DL_THREADS-thread blocks, one item a block:
//   block 0: the router: the row's top-8 from the logits, published with each pick's weight and its three
//     matrices' trellis addresses and widths (loaded with the logits, a thread an expert);
//   then U GU gate|up items (unit, column block nh, matrix, k chunk of 256), the shared expert's (unit 0) first;
//   then U DB down items (unit, output column block of 128).
// A gate|up block routes the row up to its unit's pick (the shared expert's items need no routing); a down block,
// which has time until its inputs are ready, waits for its pick's entry from the router (one wave polls four slots),
// so that the down blocks' top-8 rounds do not compete with the gate|up blocks' at the start of the launch. A gate|up
// block stages its 16 k tiles x 2 column tiles a wave of trellis in LDS, rotates the row's activations of its chunk,
// multiplies on MFMA and stores its partial sums. The last item of a (unit, nh) in block order then waits for the other items' sums, adds the
// chunks in order and runs the SwiGLU epilogue of that column block into the unit's down inputs. A down block stages
// its unit's down trellis of its column block, waits for both column blocks of its unit's down inputs, multiplies,
// rotates and stores the unit's output of the column block; the down block of the last unit combines the column
// block: the slots in order from 0, then the shared expert.
//
// Hand-offs are tagged slots: a value handed to another block is stored together with the launch's tag in one 8-byte
// agent-scope store (the value's bits low, the tag high; coherent across the XCDs' L2s), and the reader polls the slots
// themselves with agent-scope loads until every tag is the launch's. Once the data has landed, a reader needs one
// round trip, and a writer never waits for its stores. The tag comes from the epoch word at the start of the region:
// a block reads it once and checks in by storing the tag in its own word; the last block of the launch, once every
// other block has checked in, advances the epoch, so the next launch (after this one, on the stream) tags with the
// next value and no slot is ever cleared. The slots sit at fixed offsets for every layer shape, their tag halves hold
// nothing but tags, and a scratch's tags only grow (0, what a cleared scratch holds, is never one): a slot not yet
// written in this launch never carries its tag.
// Every wait is on blocks of lower index, which the hardware dispatched before the waiting block and which never wait
// on it, so every wait ends; each is bounded anyway: a give-up is recorded as EA_SYNC_TIMEOUT and the values it would
// have produced are NaN.

constexpr int L1_POLLS = 1 << 18;  // polls before a wait gives up

__device__ __forceinline__ uint32_t l1_next(uint32_t e) { return e == 0xffffffffu ? 1u : e + 1u; }
__device__ __forceinline__ uint32_t* l1_epoch(const DLArgs& a) { return reinterpret_cast<uint32_t*>(a.lay.sync); }
__device__ __forceinline__ uint32_t* l1_checkin(const DLArgs& a) { return l1_epoch(a) + L1_CHK; }
__device__ __forceinline__ void st_tag(uint64_t* p, uint32_t bits, uint32_t tag) {
    __hip_atomic_store(p, ((uint64_t)tag << 32) | bits, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint64_t ld_tag(const uint64_t* p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ bool tag_is(uint64_t v, uint32_t tag) { return (uint32_t)(v >> 32) == tag; }
__device__ __forceinline__ float tag_val(uint64_t v) { return __uint_as_float((uint32_t)v); }
__device__ __forceinline__ bool wave_all(bool ok) { return __builtin_amdgcn_ballot_w64(!ok) == 0; }
// An opaque copy of a pointer: a poll loop then forms its addresses in each pass instead of holding them all.
template <typename T>
__device__ __forceinline__ const T* opaque_ptr(const T* p) {
    asm volatile("" : "+v"(p));
    return p;
}

// The epoch, read by thread 0 at the block's start (the other threads' value is unused).
__device__ __forceinline__ uint32_t l1_epoch_load(const DLArgs& a) {
    return threadIdx.x == 0 ? ld_coh(l1_epoch(a)) : 0u;
}

// The last block of the launch: once every other block has checked in with this launch's tag, the epoch advances to
// it. Run by one wave.
__device__ __forceinline__ void l1_advance(const DLArgs& a, uint32_t tag, int lane) {
    constexpr int PER = (L1_MAXB + 63) / 64;
    const int others = (int)gridDim.x - 1;
    const uint32_t* chk = l1_checkin(a);
    for (int n = 0;; ++n) {
        // every word loaded before any is checked (a check beside each load made each load wait for the one before)
        uint32_t v[PER];
#pragma unroll
        for (int k = 0; k < PER; ++k) v[k] = ld_coh(chk + lane + 64 * k);  // inside the sync words for every k
        bool ok = true;
#pragma unroll
        for (int k = 0; k < PER; ++k) ok &= lane + 64 * k >= others || v[k] == tag;
        if (wave_all(ok)) break;
        if (n >= L1_POLLS) {
            if (lane == 0) record_error(a.status, DEV_SYNC_TIMEOUT);
            break;
        }
        __builtin_amdgcn_s_sleep(2);
    }
    if (lane == 0) st_coh(l1_epoch(a), tag);
}

struct L1Sh {
    int pick[DL_SLOTS];
    float wts[DL_SLOTS];
    uint64_t tp;  // the block's unit: the trellis address and width of the block's matrix, its expert
    int tk, e;
    int flag;
    uint32_t tag;
    __attribute__((aligned(16))) uint16_t xs[DL_RS];  // the row: its rotated activations, or the unit's down inputs
    union {
        struct {
            uint64_t tptr[3][256];
            int tk2[3][256];
        } r;  // the router's tables of every expert, loaded with the logits
        __attribute__((aligned(16))) uint32_t stage[DL_WAVES][DL_STAGE_WORDS];
        struct {
            float half[2][128];  // the gate's and the up's sums over the first half of the chunks
            float gus[2][128];   // their outputs
        } ep;
        float ys[128];
    };
};

__device__ __forceinline__ uint64_t* l1_route_slots(const DLArgs& a) {
    return reinterpret_cast<uint64_t*>(a.lay.sync) + L1_RT;
}

// Block 0: the row's top-8 and weights, every expert's tables of the three matrices (a thread an expert, E = 256,
// loaded with the logits), then the routing slots: pick k, weight k, and (matrix m, pick k)'s trellis address (two
// slots) and width; and the caller's pick / wts.
__device__ __forceinline__ void l1_router(const DLArgs& a, L1Sh& sh, uint32_t e0) {
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
    uint64_t tp[3];
    int tk[3];
#pragma unroll
    for (int m = 0; m < 3; ++m) {
        tp[m] = (uint64_t)a.ptr[m][t];
        tk[m] = a.k2t[m][t];
    }
    if (wave == 0) topk8_wave(a.logits, a.bias, a.scale, sh.pick, sh.wts, lane);
#pragma unroll
    for (int m = 0; m < 3; ++m) {
        sh.r.tptr[m][t] = tp[m];
        sh.r.tk2[m][t] = tk[m];
    }
    if (t == 0) {
        const uint32_t tag = l1_next(e0);
        sh.tag = tag;
        st_coh(l1_checkin(a) + blockIdx.x, tag);
    }
    __syncthreads();
    if (t < DL_SLOTS) {
        const uint32_t tag = sh.tag;
        const int e = sh.pick[t];
        const float w = sh.wts[t];
        uint64_t* rt = l1_route_slots(a);
        st_tag(rt + t, (uint32_t)e, tag);
        st_tag(rt + DL_SLOTS + t, __float_as_uint(w), tag);
#pragma unroll
        for (int m = 0; m < 3; ++m) {
            const uint64_t p = sh.r.tptr[m][e];
            uint64_t* q = rt + 2 * DL_SLOTS + (m * DL_SLOTS + t) * 3;
            st_tag(q, (uint32_t)p, tag);
            st_tag(q + 1, (uint32_t)(p >> 32), tag);
            st_tag(q + 2, (uint32_t)sh.r.tk2[m][e], tag);
        }
        a.pick[t] = e;
        a.wts[t] = w;
    }
}

// A gate|up item routes the row itself, up to its pick k (k + 1 top-8 rounds), with the tables of matrix `mat` of
// every expert loaded with the logits; its unit's entry into sh.e / sh.tp / sh.tk. (Waiting for the router's slots
// instead measured slower for the gate|up items: the slots land 1-2 us after the router stores them.)
__device__ __forceinline__ void l1_route_self(const DLArgs& a, L1Sh& sh, int mat, int k) {
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
    const uint64_t tp = (uint64_t)a.ptr[mat][t];
    const int tk = a.k2t[mat][t];
    if (wave == (int)(blockIdx.x % DL_WAVES)) topk8_wave(a.logits, a.bias, a.scale, sh.pick, sh.wts, lane, k + 1);
    sh.r.tptr[0][t] = tp;
    sh.r.tk2[0][t] = tk;
    __syncthreads();
    if (t == 0) {
        const int e = sh.pick[k];
        sh.e = e;
        sh.tp = sh.r.tptr[0][e];
        sh.tk = sh.r.tk2[0][e];
    }
    __syncthreads();
}

// A down item's wait for the router (wave 0; the caller's barrier follows): pick k's expert and its matrix `mat`'s
// trellis address and width into sh.e / sh.tp / sh.tk, and with `weights` every pick's weight into sh.wts. Lanes 0..3
// poll the pick's four slots, lanes 4..11 the weights; a give-up is recorded and leaves expert 0's entry (the
// product is then NaN through `timed_out`).
__device__ __forceinline__ bool l1_route_wait(const DLArgs& a, L1Sh& sh, int k, int mat, uint32_t tag, bool weights,
                                              int lane) {
    const uint64_t* rt = l1_route_slots(a);
    const int at = lane == 0 ? k
                 : lane < 4 ? 2 * DL_SLOTS + (mat * DL_SLOTS + k) * 3 + lane - 1
                 : lane < 12 ? DL_SLOTS + lane - 4 : 0;
    const bool used = lane < (weights ? 12 : 4);
    uint64_t v = 0;
    bool timed_out = false;
    for (int n = 0;; ++n) {
        v = ld_tag(rt + at);
        if (wave_all(!used || tag_is(v, tag))) break;
        if (n >= L1_POLLS) {
            timed_out = true;
            if (lane == 0) record_error(a.status, DEV_SYNC_TIMEOUT);
            break;
        }
        __builtin_amdgcn_s_sleep(1);
    }
    const uint32_t lo = (uint32_t)v;
    const int e = __builtin_amdgcn_readlane((int)lo, 0);
    const uint32_t plo = (uint32_t)__builtin_amdgcn_readlane((int)lo, 1);
    const uint32_t phi = (uint32_t)__builtin_amdgcn_readlane((int)lo, 2);
    const int k2 = __builtin_amdgcn_readlane((int)lo, 3);
    if (lane == 0) {
        const bool ok = !timed_out && e >= 0 && e < a.E;
        sh.e = ok ? e : 0;
        sh.tp = ok ? ((uint64_t)phi << 32 | plo) : (uint64_t)a.ptr[mat][0];
        sh.tk = ok ? k2 : 0;  // no decoder: the product stores NaN
    }
    if (weights && lane >= 4 && lane < 12) sh.wts[lane - 4] = __uint_as_float(lo);
    return timed_out;
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

// A down item's wait for both column blocks of its unit's down inputs: wave 0 polls their slots and moves them to
// sh.xs; every wave meets at the barrier. True when the wait gave up. (Every wave polling, staggered by a quarter
// round trip, measured slower: the waits are bound by the round trip, not by how often a poll is issued.)
__device__ __forceinline__ bool l1_down_wait(const DLArgs& a, L1Sh& sh, int u, uint32_t tag, int lane) {
    const int NH = a.I / 128;
    if (threadIdx.x < 64) {
        const uint64_t* xd = a.lay.txd + (size_t)u * (a.I / 2) + lane;
        uint64_t p[L1_MAXNH];
        bool timed_out = false;
        for (int n = 0;; ++n) {
            bool ok = true;
#pragma unroll
            for (int j = 0; j < L1_MAXNH; ++j) {
                p[j] = ld_tag(xd + j * 64);  // j >= NH: another unit's slot, not used
                ok &= j >= NH || tag_is(p[j], tag);
            }
            if (wave_all(ok)) break;
            if (n >= L1_POLLS) {
                timed_out = true;
                if (lane == 0) record_error(a.status, DEV_SYNC_TIMEOUT);
                break;
            }
            __builtin_amdgcn_s_sleep(1);
        }
#pragma unroll
        for (int j = 0; j < L1_MAXNH; ++j)
            if (j < NH) reinterpret_cast<uint32_t*>(sh.xs)[j * 64 + lane] = (uint32_t)p[j];
        if (lane == 0) sh.flag = timed_out;
    }
    __syncthreads();
    return sh.flag;
}

// The down product of a down item, around its wait: the first PRE k-tile pairs of the wave's two column tiles are
// decoded into MFMA operands (registers) while the unit's down inputs are still being produced; l1_down_wait then
// brings the inputs to sh.xs, and the MFMAs run, the remaining pairs decoded as they go. Returns the wait's result.
// The one-row layer pre-decodes every pair (PRE = NKT / 2): once the inputs land, a down item is 16 MFMAs, the FWHT
// and a store (2.0 us of decode after the wait measured without it; 1.0 us with half of it pre-decoded).
template <int CB, int K2, int NKT, int PRE>
__device__ __forceinline__ bool l1_down_product(const DLArgs& a, L1Sh& sh, int u, uint32_t tag, const uint32_t* st,
                                                const LaneQuad& lq, int lane, f4v (&acc)[2]) {
    static_assert(PRE <= NKT / 2, "pre-decoded pairs of k tiles");
    constexpr int TW = 4 * K2;
    const uint32_t* wa = st + lq.w0;
    const uint32_t* wb = st + lq.w1;
    u4v pb[PRE > 0 ? PRE : 1][2];
#pragma unroll
    for (int tp = 0; tp < PRE; ++tp)
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const int t0 = (4 * tp + j) * TW, t1 = (4 * tp + 2 + j) * TW;
            const u2v b0 = decode_quad<K2, CB>(wa[t0], wb[t0], lq.sh);
            const u2v b1 = decode_quad<K2, CB>(wa[t1], wb[t1], lq.sh);
            pb[tp][j] = u4v{b0.x, b0.y, b1.x, b1.y};
        }
#pragma unroll
    for (int tp = 0; tp < PRE; ++tp)
#pragma unroll
        for (int j = 0; j < 2; ++j) hold(pb[tp][j]);  // decoded before the wait, not after it
    EA_STAMP(2, threadIdx.x == 0);  // wave 0's pre-decode done
    const bool r = l1_down_wait(a, sh, u, tag, lane);
    EA_STAMP(3, threadIdx.x == 0);  // the down inputs seen
    __builtin_amdgcn_s_setprio(2);  // the pre-decode ran at the lowest priority, beside the gate|up decode
    const bool row0 = (lane & 15) == 0;
    const uint16_t* xr = sh.xs + 2 * ((lane >> 4) & 3);
#pragma unroll
    for (int tp = 0; tp < NKT / 2; ++tp) {
        const uint16_t* xk = xr + 2 * tp * 16;
        u4v au = {*reinterpret_cast<const uint32_t*>(xk), *reinterpret_cast<const uint32_t*>(xk + 8),
                  *reinterpret_cast<const uint32_t*>(xk + 16), *reinterpret_cast<const uint32_t*>(xk + 24)};
        if (!row0) au = u4v{0u, 0u, 0u, 0u};
        const h8v a = __builtin_bit_cast(h8v, au);
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            u4v bq;
            if (tp < PRE) {
                bq = pb[tp < PRE ? tp : 0][j];
            } else {
                const int t0 = (4 * tp + j) * TW, t1 = (4 * tp + 2 + j) * TW;
                const u2v b0 = decode_quad<K2, CB>(wa[t0], wb[t0], lq.sh);
                const u2v b1 = decode_quad<K2, CB>(wa[t1], wb[t1], lq.sh);
                bq = u4v{b0.x, b0.y, b1.x, b1.y};
            }
            acc[j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, __builtin_bit_cast(h8v, bq), acc[j], 0, 0, 0);
        }
    }
    return r;
}

// Gate|up item (unit u, column block nh, matrix mat, chunk c) of the row; e0: the epoch thread 0 read. Its partial
// sums go to the tagged slots tz[u][nh][mat][c][128].
template <int CB, bool SHARED>
__device__ __forceinline__ void l1_gateup(const DLArgs& a, L1Sh& sh, int u, int nh, int mat, int c, uint32_t e0) {
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
    if (threadIdx.x == 0) {  // the launch's tag, and the check-in
        const uint32_t t = l1_next(e0);
        sh.tag = t;
        st_coh(l1_checkin(a) + blockIdx.x, t);
    }
    __syncthreads();
    const uint32_t tag = (uint32_t)uniform((int)sh.tag);
    uint32_t* st = sh.stage[wave];
    stage_store<DL_KT>(st, k2, lane, v);
    EA_STAMP(5, threadIdx.x == 0);  // the activations rotated, wave 0's trellis landed
    f4v acc[2] = {f4v{0.f, 0.f, 0.f, 0.f}, f4v{0.f, 0.f, 0.f, 0.f}};
    const bool ok = l1_mfma_k2<CB, DL_KT>(k2, st, lq, sh.xs, lane, acc);
    EA_STAMP(6, threadIdx.x == 0);  // wave 0's tiles decoded and multiplied
    if (!ok) {
        if (lane == 0) record_error(a.status, DEV_UNSUPPORTED_WIDTH);
        acc[0] = acc[1] = nan4();
    }
    // row 0's partial sums of this chunk
    if (lane < 16) {
        uint64_t* z = a.lay.tz + ((((size_t)u * NH + nh) * 2 + mat) * KC + c) * 128;
#pragma unroll
        for (int j = 0; j < 2; ++j) st_tag(z + (2 * wave + j) * 16 + lane, __float_as_uint(acc[j][0]), tag);
    }
}

// The SwiGLU epilogue of (unit u, column block nh), run by the unit's last gate|up item of nh once its own sums are
// stored: waves 0 / 2 take the gate's first / second half of the chunks, waves 1 / 3 the up's, each polling its
// chunks' slots (two columns a lane); the sums run over the chunks in order, the first half's handed on through LDS;
// then FWHT, svh and SwiGLU into the unit's tagged down inputs.
__device__ __forceinline__ void l1_epilogue(const DLArgs& a, L1Sh& sh, const UnitView& uv, int u, int nh) {
    constexpr int HC = DL_MAXKC / 2;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int KC = a.D / 256, NH = a.I / 128;
    const int mat = wave & 1, h = wave >> 1, half = (KC + 1) >> 1;
    const int c0 = h ? half : 0, nc = h ? KC - half : half;
    const uint32_t tag = (uint32_t)uniform((int)sh.tag);
    const uint32_t sv = svh_pair(a, uv, nh, mat, lane);
    const uint32_t sd = suhd_pair(a, uv, nh, lane);
    __syncthreads();  // every wave is done with its staged trellis: the sums take its place
    const uint64_t* z = a.lay.tz + (((size_t)u * NH + nh) * 2 + mat) * KC * 128 + (size_t)c0 * 128 + 2 * lane;
    uint64_t p[HC][2];
    bool timed_out = false;
    if (nc > 0) {
        for (int n = 0;; ++n) {
            bool ok = true;
            const uint64_t* zb = opaque_ptr(z);  // addresses formed inside the loop, not held across it
#pragma unroll
            for (int i = 0; i < HC; ++i) {
                p[i][0] = ld_tag(zb + i * 128);  // chunks past nc: other slots of the array, not used
                p[i][1] = ld_tag(zb + i * 128 + 1);
                ok &= i >= nc || (tag_is(p[i][0], tag) && tag_is(p[i][1], tag));
            }
            if (wave_all(ok)) break;
            if (n >= L1_POLLS) {
                timed_out = true;
                if (lane == 0) record_error(a.status, DEV_SYNC_TIMEOUT);
                break;
            }
            __builtin_amdgcn_s_sleep(1);
        }
    }
    float s0 = 0.f, s1 = 0.f;
    if (h == 0) {
#pragma unroll
        for (int i = 0; i < HC; ++i)
            if (i < nc) {
                s0 += tag_val(p[i][0]);
                s1 += tag_val(p[i][1]);
            }
        if (timed_out) s0 = s1 = __builtin_nanf("");
        *reinterpret_cast<float2*>(&sh.ep.half[mat][2 * lane]) = float2{s0, s1};
    }
    __syncthreads();
    EA_STAMP(3, threadIdx.x == 0);  // every wave's polls done
    if (h == 1) {
        const float2 f = *reinterpret_cast<const float2*>(&sh.ep.half[mat][2 * lane]);
        s0 = f.x;
        s1 = f.y;
#pragma unroll
        for (int i = 0; i < HC; ++i)
            if (i < nc) {
                s0 += tag_val(p[i][0]);
                s1 += tag_val(p[i][1]);
            }
        if (timed_out) s0 = s1 = __builtin_nanf("");
        *reinterpret_cast<float2*>(&sh.ep.gus[mat][2 * lane]) = gu_out(uv, float2{s0, s1}, sv, lane);
    }
    __syncthreads();
    if (wave == 2) {
        const float2 g = *reinterpret_cast<const float2*>(&sh.ep.gus[0][2 * lane]);
        const float2 up = *reinterpret_cast<const float2*>(&sh.ep.gus[1][2 * lane]);
        st_tag(a.lay.txd + (size_t)u * (a.I / 2) + nh * 64 + lane, act_pair(uv, g, up, sd, lane), tag);
        EA_STAMP(4, lane == 0);  // the down inputs stored
    }
}

// Down item (unit u, output column block cb) of the row (sh.tag holds the launch's tag). Its outputs go to the tagged
// slots ty[u][D]; the last unit's block combines the column block instead.
template <int CB, int SCB, int NKT>
__device__ __forceinline__ void l1_down(const DLArgs& a, L1Sh& sh, const UnitView& uv, int u, int cb) {
    const int lane = opaque_lane(threadIdx.x & 63), wave = uniform((int)threadIdx.x >> 6);
    const int NH = a.I / 128, KT = a.I / 16, ns = a.D / 16;
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
    const uint32_t tag = (uint32_t)uniform((int)sh.tag);  // set by thread 0 before the block's first barrier
    if (wave == 0) {
        if (lane == 0) st_coh(l1_checkin(a) + blockIdx.x, tag);
        if (blockIdx.x == gridDim.x - 1) l1_advance(a, tag, lane);
    }
    uint32_t* st = sh.stage[wave];
    stage_store<NKT>(st, k2, lane, v);
    f4v acc[2] = {f4v{0.f, 0.f, 0.f, 0.f}, f4v{0.f, 0.f, 0.f, 0.f}};
    bool timed_out = false;
    const bool ok =
        uv.shared ? EA_K2_SWITCH(k2, 2, 10,
                                 (timed_out = l1_down_product<SCB, K2V, NKT, NKT / 2>(a, sh, u, tag, st, lq, lane, acc)))
                  : EA_K2_SWITCH(k2, 2, 10,
                                 (timed_out = l1_down_product<CB, K2V, NKT, NKT / 2>(a, sh, u, tag, st, lq, lane, acc)));
    if (!ok) timed_out = l1_down_wait(a, sh, u, tag, lane);  // no decoder for the width: the block still meets its barrier
    if (!ok || timed_out) {
        if (lane == 0 && !ok) record_error(a.status, DEV_UNSUPPORTED_WIDTH);
        acc[0] = acc[1] = nan4();
    }
    __syncthreads();  // every wave is done with its staging: the column sums take its place
    EA_STAMP(4, threadIdx.x == 0);  // every wave's MFMAs done
    if (lane < 16) {
#pragma unroll
        for (int j = 0; j < 2; ++j) sh.ys[(2 * wave + j) * 16 + lane] = acc[j][0];
    }
    __syncthreads();
    if (wave != 0) return;
    float v0 = sh.ys[2 * lane], v1 = sh.ys[2 * lane + 1];
    fwht128_w64(v0, v1, lane);
    v0 = v0 * HAD_SCALE * h2f((uint16_t)(sd & 0xffffu));
    v1 = v1 * HAD_SCALE * h2f((uint16_t)(sd >> 16));
    const int n = cb * 128 + 2 * lane;
    if (u != a.U - 1) {
        uint64_t* y = a.lay.ty + (size_t)u * a.D + n;
        st_tag(y, __float_as_uint(v0), tag);
        st_tag(y + 1, __float_as_uint(v1), tag);
        EA_STAMP(5, lane == 0);  // the outputs stored
        return;
    }
    // the combine of the column block (the last unit is the last slot's): the other units' outputs, then the slots
    // in order from 0 (exl3_experts.cu:256-267), then the shared expert
    uint64_t p[L1_UNITS - 1][2];
    bool timed_out2 = false;
    for (int it = 0;; ++it) {
        bool all = true;
        const uint64_t* yb = opaque_ptr(a.lay.ty + n);
#pragma unroll
        for (int w = 0; w < L1_UNITS - 1; ++w) {
            const uint64_t* y = yb + (size_t)w * a.D;  // w >= U - 1: a slot not used
            p[w][0] = ld_tag(y);
            p[w][1] = ld_tag(y + 1);
            all &= w >= a.U - 1 || (tag_is(p[w][0], tag) && tag_is(p[w][1], tag));
        }
        if (wave_all(all)) break;
        if (it >= L1_POLLS) {
            timed_out2 = true;
            if (lane == 0) record_error(a.status, DEV_SYNC_TIMEOUT);
            break;
        }
        __builtin_amdgcn_s_sleep(1);
    }
    EA_STAMP(5, lane == 0);  // the other units' outputs seen
    // slot k is unit hs + k (U = hs + 8): slots 0..6 from the tagged slots, slot 7 this block's own
    const bool hs = a.hs;
    float a0 = 0.f, a1 = 0.f;
#pragma unroll
    for (int k = 0; k < DL_SLOTS - 1; ++k) {
        a0 = __builtin_fmaf(sh.wts[k], tag_val(hs ? p[k + 1][0] : p[k][0]), a0);
        a1 = __builtin_fmaf(sh.wts[k], tag_val(hs ? p[k + 1][1] : p[k][1]), a1);
    }
    a0 = __builtin_fmaf(sh.wts[DL_SLOTS - 1], v0, a0);
    a1 = __builtin_fmaf(sh.wts[DL_SLOTS - 1], v1, a1);
    if (hs) {
        a0 = a0 + tag_val(p[0][0]);
        a1 = a1 + tag_val(p[0][1]);
    }
    if (timed_out2) a0 = a1 = __builtin_nanf("");
    *reinterpret_cast<float2*>(a.out + n) = float2{a0, a1};
    EA_STAMP(6, lane == 0);  // the column block combined
}

// Five waves a SIMD: the down items hold their whole pre-decoded product (64 VGPRs) through their wait.
template <int CB, int SCB>
__global__ void __launch_bounds__(DL_THREADS) __attribute__((amdgpu_waves_per_eu(5))) layer1_kernel(DLArgs a) {
    __shared__ L1Sh sh;
    const int NH = a.I / 128, KC = a.D / 256, DB = a.D / 128;
    const int GU = NH * 2 * KC;  // gate|up items a unit
    EA_STAMP(0, threadIdx.x == 0);  // the block's start
    const uint32_t e0 = l1_epoch_load(a);
    if (blockIdx.x == 0) {
        l1_router(a, sh, e0);
        EA_STAMP(1, threadIdx.x == 0);  // the picks published
        EA_STAMP_VALUE(STAMP_POINTS - 1, 1, threadIdx.x == 0);
        return;
    }
    const int b = blockIdx.x - 1, lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    UnitView uv;
    uv.nm = 1;
    uv.mem = nullptr;
    if (b < a.U * GU) {
        const int u = b / GU, rem = b % GU, nh = rem / (2 * KC), mat = (rem / KC) & 1, c = rem % KC;
        uv.shared = a.hs && u == 0;
        // descriptor: 2 shared / 3 routed gate|up item, unit, column block, matrix, chunk
        EA_STAMP_VALUE(STAMP_POINTS - 1, (uint64_t)(uv.shared ? 2 : 3) | (uint64_t)u << 8 | (uint64_t)nh << 16 |
                                          (uint64_t)mat << 20 | (uint64_t)c << 24, threadIdx.x == 0);
        if (uv.shared) {
            uv.e = -1;
            __builtin_amdgcn_s_setprio(2);
            l1_gateup<SCB, true>(a, sh, u, nh, mat, c, e0);
        } else {
            l1_route_self(a, sh, mat, u - a.hs);
            EA_STAMP(1, threadIdx.x == 0);  // routed up to its pick
            uv.e = uniform(sh.e);
            __builtin_amdgcn_s_setprio(2);  // the gate|up decode is on the layer's critical path
            l1_gateup<CB, false>(a, sh, u, nh, mat, c, e0);
        }
        EA_STAMP(2, threadIdx.x == 0);  // its partial sums stored
        if (mat == 1 && c == KC - 1) l1_epilogue(a, sh, uv, u, nh);
        return;
    }
    const int d = b - a.U * GU, u = d / DB, cb = d % DB;
    uv.shared = a.hs && u == 0;
    // descriptor: 4 down item, 5 the combining one (the last unit's), unit, output column block
    EA_STAMP_VALUE(STAMP_POINTS - 1, (uint64_t)(u == a.U - 1 ? 5 : 4) | (uint64_t)u << 8 | (uint64_t)cb << 16,
                threadIdx.x == 0);
    if (threadIdx.x == 0) sh.tag = l1_next(e0);
    // the last unit's block combines the column block: it takes every weight
    if (!uv.shared && wave == 0)
        l1_route_wait(a, sh, u - a.hs, 2, l1_next((uint32_t)uniform((int)e0)), u == a.U - 1, lane);  // lane 0 is thread 0
    __syncthreads();
    EA_STAMP(1, threadIdx.x == 0);  // the router's slots seen
    uv.e = uv.shared ? -1 : uniform(sh.e);
    if (a.I == 256)
        l1_down<CB, SCB, 16>(a, sh, uv, u, cb);
    else
        l1_down<CB, SCB, 8>(a, sh, uv, u, cb);
}

// ---- host side ----------------------------------------------------------------------------------------------------

static size_t align256(size_t n) { return (n + 255) & ~(size_t)255; }

// Region offsets for a scratch of `rows` rows (capacity), in bytes from the region's base.
struct DLCarve {
    size_t sync, tags, zp, xd, sy, ws, total;
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
    c.tags = take(L1_TAG_BYTES);
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
    l.tz = dptr<uint64_t>(base + c.tags);
    l.txd = l.tz + L1_TZ;
    l.ty = l.txd + L1_TXD;
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
        layer1_kernel<CB, SCB><<<1 + a.U * NH * 2 * KC + a.U * DB, DL_THREADS, 0, s>>>(a);
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
    int scb = ex->cb == 0 ? 1 : (int)ex->cb;  // without a shared expert any built pairing (its codebook is unused)
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
    // routed 3inst experts (the reference's grouped kernel takes every codebook, exl3_experts.cu:306-309) beside a
    // shared expert in one of the codebooks its linear takes (mcg, mul1)
    if (rcb == 0 && scb == 1) return dl_launch<0, 1>(s, a, c->cus, c->device);
    if (rcb == 0 && scb == 2) return dl_launch<0, 2>(s, a, c->cus, c->device);
    return EA_UNPORTED_GROUPED_VARIANT;
}

// ---- the allocation-free variant's scratch --------------------------------------------------------------------------

// The scratch of ea_ffn_moe_decode_static: the per-pair down outputs and the decode layer's region, carved for
// DL_MAXR rows of the call's layer shape. The largest shape the decode layer takes (D 6144, I 256) needs 12.06 MB.
// Every call on a device shares that device's copy, which holds the last call's contents: the layer writes every
// value it reads back within a call, and the one-row launch's epoch word, check-in words and tagged slots start at
// zero (ea_init clears the array) and are never cleared again: each launch tags with the next epoch.
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

#ifdef EA_STAMPS
// The timeline build only: the stamp region of the decode layer kernels (ea_stamps.hpp).
int ea_stamps_attach_layer(void* region) { return stamp_attach(region); }
#endif

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
