// Routed experts of prompt chunks (hundreds to thousands of rows): route the pairs into items of at most IPM pairs
// of one expert, then per item one MFMA GEMM that decodes each trellis tile once for all of the item's rows
// (prompt_experts.cu / prompt_experts.zig of the reference give the interface and the item scheme).
//
// A pass over <= 4096 rows: route -> per-pair input rotation -> item GEMM gate|up -> gate/up epilogue -> item GEMM
// down -> [down epilogue + slot-ordered combine] [-> bf16 rounding]. Every row's arithmetic is independent of which
// item or M-tile it lands in (MFMA rows do not mix). With a pair plane (the reference's deterministic mode 2) the
// down GEMM writes each pair's row and the combine adds the slots in order, so the output is the same on every run.
// Without one (modes 0 and 1, the reference's default) the down GEMM's epilogue adds each pair into its row of out
// with fp32 (or packed fp16) atomics in arrival order; the rotation launch clears out first.
#include <hip/hip_runtime.h>

#include "ea_device.hpp"
#include "ea_experts.hpp"
#include "ea_gemm.hpp"
#include "ea_host.hpp"

namespace ea {

// Routed pairs an item at most. The reference's items hold up to 112 (prompt_experts.cu:55-58, TF_PE_GPM), as do
// this library's for the register-streaming GEMM of widths above 10 (IPM_WIDE); the staged GEMMs (widths 2..10) take
// items of up to 80 (five row tiles): against 48 the same at 512 rows and 3-4 % faster at 2048 (a heavy expert
// decoded in fewer items), against 112 (seven row tiles, more accumulators) faster at both; 64 and 96 measured between.
// A pair's sums do not depend on its item. The register-streaming GEMM keeps the reference's 112 (7 row tiles); its
// index arithmetic is the same for any number of row tiles (a 3-tile build once summed wrong at widths 12-16: the
// decoder's half-register fp16 adds lacked the wait states their readers need, which cb_pair now carries).
constexpr int IPM = 80;
constexpr int IPM_TILES = IPM / 16;
constexpr int IPM_WIDE = 112;
constexpr int IPM_WIDE_TILES = IPM_WIDE / 16;
constexpr uint32_t CHUNK_ROWS = 4096;  // rows a pass at most (prompt_experts.zig:17)
constexpr int ROUTE_THREADS = 1024;
constexpr int ROUTE_HELD = 16;  // picks a route thread holds in registers: 16,384 pairs (2,048 rows of 8 slots)

constexpr int SMALL_ROWS = 16;     // items of at most this many pairs: the kernels holding one row tile

// Item i of list `big` (0: items of at most SMALL_ROWS pairs, from the front of items[]; 1: the others, from its
// back), or false past the list's count.
__device__ __forceinline__ bool item_at(const int* __restrict__ items, const int* __restrict__ count, int big,
                                        int max_items, int i, int& e, int& first, int& cnt) {
    if (i >= count[big]) return false;
    const int at = big ? max_items - 1 - i : i;
    e = items[3 * at];
    first = items[3 * at + 1];
    cnt = items[3 * at + 2];
    return true;
}

// One block: per-expert counts; exclusive scans over experts of the counts and of both lists' items; items
// (e, first, cnt <= ipm) of an expert in pair order, each into its list; sorted[] = pair ids grouped by expert (order
// within an expert: arrival); pclass[pair] = 1 when the pair's item is in the list of larger items. (prompt_experts.cu:
// 162-244 with by_count off; the two lists are this library's: they let a launch size its registers for its items'
// rows, and the larger items split K.)
__global__ void __launch_bounds__(ROUTE_THREADS) route_kernel(const int* __restrict__ pick, int n, int E,
                                                             int* __restrict__ sorted, int* __restrict__ items,
                                                             int* __restrict__ item_count, int* __restrict__ pclass,
                                                             int max_items, int ipm) {
    extern __shared__ int sh[];
    int* cnt = sh;          // [E]
    int* cur = sh + E;      // [E]
    int* start = sh + 2 * E;  // [E]
    __shared__ int wsum[ROUTE_THREADS / 64][3];
    for (int e = threadIdx.x; e < E; e += ROUTE_THREADS) cnt[e] = 0;
    // the first ROUTE_HELD * ROUTE_THREADS picks are loaded once, all loads in flight together, and held in
    // registers for both passes (a load then an atomic a pair waited for every load in turn); later ones are re-read
    int held[ROUTE_HELD];
#pragma unroll
    for (int j = 0; j < ROUTE_HELD; ++j) {
        const int i = j * ROUTE_THREADS + (int)threadIdx.x;
        held[j] = i < n ? pick[i] : -1;
    }
    __syncthreads();
#pragma unroll
    for (int j = 0; j < ROUTE_HELD; ++j)
        if (held[j] >= 0 && held[j] < E) atomicAdd(&cnt[held[j]], 1);
    for (int i = ROUTE_HELD * ROUTE_THREADS + threadIdx.x; i < n; i += ROUTE_THREADS) {
        const int e = pick[i];
        if (e >= 0 && e < E) atomicAdd(&cnt[e], 1);
    }
    __syncthreads();
    const int per = (E + ROUTE_THREADS - 1) / ROUTE_THREADS;
    const int e0 = threadIdx.x * per;
    int own[3] = {0, 0, 0};  // pairs, small items, large items of this thread's experts
    for (int q = 0; q < per; ++q) {
        const int e = e0 + q;
        if (e < E) {
            const int c = cnt[e], full = c / ipm, rem = c - full * ipm;
            own[0] += c;
            own[1] += rem > 0 && rem <= SMALL_ROWS;
            own[2] += full + (rem > SMALL_ROWS);
        }
    }
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    int inc[3] = {own[0], own[1], own[2]};
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
#pragma unroll
        for (int v = 0; v < 3; ++v) {
            const int a = __shfl_up(inc[v], o, 64);
            if (lane >= o) inc[v] += a;
        }
    }
    if (lane == 63)
#pragma unroll
        for (int v = 0; v < 3; ++v) wsum[wave][v] = inc[v];
    __syncthreads();
    if (wave == 0) {
#pragma unroll
        for (int v = 0; v < 3; ++v) {
            const int a = lane < ROUTE_THREADS / 64 ? wsum[lane][v] : 0;
            int sa = a;
#pragma unroll
            for (int o = 1; o < 64; o <<= 1) {
                const int x = __shfl_up(sa, o, 64);
                if (lane >= o) sa += x;
            }
            if (lane < ROUTE_THREADS / 64) wsum[lane][v] = sa - a;
            if (v > 0 && lane == ROUTE_THREADS / 64 - 1) item_count[v - 1] = min(sa, max_items);
        }
    }
    __syncthreads();
    int off = wsum[wave][0] + inc[0] - own[0];
    int si = wsum[wave][1] + inc[1] - own[1], bi = wsum[wave][2] + inc[2] - own[2];
    for (int q = 0; q < per; ++q) {
        const int e = e0 + q;
        if (e >= E) break;
        const int c = cnt[e];
        cur[e] = off;
        start[e] = off;
        for (int f = 0; f < c; f += ipm) {
            const int m = min(ipm, c - f);
            const int at = m <= SMALL_ROWS ? si++ : max_items - 1 - bi++;
            if (at >= 0 && at < max_items) {
                items[3 * at] = e;
                items[3 * at + 1] = off + f;
                items[3 * at + 2] = m;
            }
        }
        off += c;
    }
    __syncthreads();
    auto place = [&](int i, int e) __attribute__((always_inline)) {
        int big = 0;
        if (e >= 0 && e < E) {
            const int at = atomicAdd(&cur[e], 1);
            sorted[at] = i;
            const int f = (at - start[e]) / ipm * ipm;  // the first pair of its item, within the expert
            big = min(ipm, cnt[e] - f) > SMALL_ROWS;
        }
        pclass[i] = big;
    };
#pragma unroll
    for (int j = 0; j < ROUTE_HELD; ++j) {
        const int i = j * ROUTE_THREADS + (int)threadIdx.x;
        if (i < n) place(i, held[j]);
    }
    for (int i = ROUTE_HELD * ROUTE_THREADS + threadIdx.x; i < n; i += ROUTE_THREADS) place(i, pick[i]);
}

// ---- the down epilogue without a pair plane ---------------------------------------------------------------------

constexpr int ES = 128 + 4;  // LDS row stride of a row tile's epilogue buffer, floats (rows 4 apart on other banks)

// Where the atomic down epilogue adds: out [rows, D] fp32 (fp16 with half), the expert's svh_d row, the item's pairs
// and routing weights (LDS), and a double buffer of one row tile x 128 columns in LDS.
struct DnAtomic {
    void* out;
    const uint16_t* svh;  // svh_d + e * D
    const int* pair_sh;   // the item's pairs, -1 past its count
    const float* wts_sh;  // their routing weights
    float* ebuf;          // [2][16][ES]
    int D, slots, half;
};

// The down items' epilogue without a pair plane (prompt_experts.cu:719-797, modes 0 and 1): for each occupied row
// tile, the block's four waves hand their 16 rows x 32 columns (two column tiles each, MFMA accumulator layout) to LDS,
// then thread (row r, lane l16) takes the row's columns g + 16 j (g = h8_group(l16)) of the 128-column block cb: the
// FWHT over the block (fwht128_x8: column bits 4, 5, 6 inside the thread, bits 0..3 across the row's 16 lanes), the
// output scale svh_d * HAD_SCALE (sv, loaded by the caller) and the pair's routing weight, then an atomic add into
// its row of out: fp32, 16 lanes a row covering 64 contiguous bytes an instruction; or, with half, packed fp16 pairs
// once the lanes of a column pair have traded values. The slots of a row meet in out in arrival order, so the sums' bits may differ run to run.
// The buffer halves alternate (eb), so one barrier a row tile suffices: a half is written again only after the
// barrier that follows every thread's reads of it.
template <int MT>
__device__ __forceinline__ void dn_atomic(const f4v (&acc)[MT][2], int mts, int wave, int lane, int cb,
                                          const uint32_t (&sv)[4], const DnAtomic& a, int& eb) {
    const int r = (int)threadIdx.x >> 4, l16 = lane & 15, g = h8_group(lane);
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
        if (mt >= mts) break;  // uniform
        float* E = a.ebuf + eb * 16 * ES;
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int i = 0; i < 4; ++i) E[(4 * (lane >> 4) + i) * ES + 32 * wave + 16 * j + l16] = acc[mt][j][i];
        __syncthreads();
        float v[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) v[j] = E[r * ES + 16 * j + g];
        eb ^= 1;
        const float sg = fwht128_x8(v, lane);  // the values' sign, folded into the scale (exact)
        const int idx = mt * 16 + r, p = a.pair_sh[idx];
        const float w = p >= 0 ? a.wts_sh[idx] : 0.f;
#pragma unroll
        for (int j = 0; j < 8; ++j) v[j] = v[j] * (sg * (h2f((uint16_t)(sv[j >> 1] >> (16 * (j & 1)))) * HAD_SCALE)) * w;
        const size_t ro = (size_t)(p >= 0 ? p / a.slots : 0) * a.D + (size_t)cb * 128;
        if (!a.half) {
            if (p >= 0) {
                float* o = static_cast<float*>(a.out) + ro + g;
#pragma unroll
                for (int j = 0; j < 8; ++j)
                    __builtin_amdgcn_global_atomic_fadd_f32((__attribute__((address_space(1))) float*)(o + 16 * j),
                                                            v[j]);
            }
        } else {
            // lane pair (l16, l16 ^ 1) holds columns (16 j + even, 16 j + odd) (its groups differ in bit 0 only): the
            // even column's lane adds j = 0..3, the odd one's j = 4..7, each as one packed pair at the even column
            // (static indices only: both lanes' pairs are formed and one is chosen)
            const bool odd = g & 1;
            uint16_t* base = static_cast<uint16_t*>(a.out) + ro + (g & ~1);
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const float oe = lane_xor<1>(v[q]), oo = lane_xor<1>(v[q + 4]);  // the partner's values
                const float lo = odd ? oo : v[q], hi = odd ? v[q + 4] : oe;
                const h2v hv = __builtin_bit_cast(h2v, (uint32_t)f2h(lo) | ((uint32_t)f2h(hi) << 16));
                if (p >= 0)
                    __builtin_amdgcn_global_atomic_fadd_v2f16(
                        (__attribute__((address_space(1))) h2v*)(base + 16 * (odd ? q + 4 : q)), hv);
            }
        }
    }
}

// svh_d of thread (r, l16)'s eight columns g + 16 j (g = h8_group(l16)) of column block cb, two fp16 a word (j even
// low).
__device__ __forceinline__ void dn_atomic_scales(const uint16_t* svh, int cb, int lane, uint32_t (&sv)[4]) {
#pragma unroll
    for (int q = 0; q < 4; ++q)
        sv[q] = (uint32_t)svh[cb * 128 + 32 * q + h8_group(lane)] |
                ((uint32_t)svh[cb * 128 + 32 * q + 16 + h8_group(lane)] << 16);
}

// Block (item, n block of NW * NTW tiles, matrix): wave w covers NTW n tiles over the whole K range for all of the
// item's rows (IPM_WIDE_TILES groups of 16), so each trellis tile is decoded once per item. Z[mat][pair][n] fp32.
template <int CB, int LO, int HI, int NTW, int NW, bool ATOM>
__global__ void __launch_bounds__(NW * 64) item_gemm_kernel(
    const uint16_t* __restrict__ X0, const uint16_t* __restrict__ X1, const int64_t* __restrict__ TP0,
    const int64_t* __restrict__ TP1, const int* __restrict__ K2_0, const int* __restrict__ K2_1,
    const int* __restrict__ sorted, const int* __restrict__ items, const int* __restrict__ item_count,
    float* __restrict__ Z, int K, int N, int P, int big, int max_items, int* __restrict__ status,
    const float* __restrict__ wts, const uint16_t* __restrict__ svh_d, void* __restrict__ out, int slots, int half) {
    static_assert(!ATOM || NTW * NW == 8, "the atomic epilogue takes 128-column blocks of four waves");
    int e, first, cnt;
    if (!item_at(items, item_count, big, max_items, blockIdx.x, e, first, cnt)) return;
    const int mat = blockIdx.z;
    const uint16_t* X = mat ? X1 : X0;
    const uint32_t* T = reinterpret_cast<const uint32_t*>(mat ? TP1[e] : TP0[e]);
    const int k2 = mat ? K2_1[e] : K2_0[e];
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    __shared__ int pair_sh[IPM_WIDE];
    constexpr int EWORDS = ATOM ? 2 * 16 * ES : 1;
    constexpr int WWORDS = ATOM ? IPM_WIDE : 1;
    __shared__ float ebuf[EWORDS];
    __shared__ float wts_sh[WWORDS];
    if (threadIdx.x < IPM_WIDE) pair_sh[threadIdx.x] = (int)threadIdx.x < cnt ? sorted[first + threadIdx.x] : -1;
    if constexpr (ATOM)
        if (threadIdx.x < IPM_WIDE) wts_sh[threadIdx.x] = (int)threadIdx.x < cnt ? wts[sorted[first + threadIdx.x]] : 0.f;
    __syncthreads();
    const int nt0 = (blockIdx.y * NW + wave) * NTW;
    if (!ATOM && nt0 * 16 >= N) return;  // ATOM: N % 128 == 0 (host-checked), every wave in range
    const uint16_t* xrow[IPM_WIDE_TILES];
#pragma unroll
    for (int m = 0; m < IPM_WIDE_TILES; ++m) {
        const int p = pair_sh[m * 16 + (lane & 15)];
        xrow[m] = p >= 0 ? X + (size_t)p * K : nullptr;
    }
    f4v acc[IPM_WIDE_TILES][NTW];
#pragma unroll
    for (int m = 0; m < IPM_WIDE_TILES; ++m)
#pragma unroll
        for (int j = 0; j < NTW; ++j) acc[m][j] = f4v{0.f, 0.f, 0.f, 0.f};
    const int ns = N >> 4;
    const uint32_t* base = T + (size_t)nt0 * 4 * k2;
    const bool ok = EA_K2_SWITCH(k2, LO, HI,
                                 (wave_tiles<CB, K2V, NTW, IPM_WIDE_TILES>(base, (size_t)ns * 4 * K2V, K >> 4, 0, xrow,
                                                                      lane, acc)));
    if (!ok) {
        if (lane == 0) record_error(status, DEV_UNSUPPORTED_WIDTH);
#pragma unroll
        for (int m = 0; m < IPM_WIDE_TILES; ++m)
#pragma unroll
            for (int j = 0; j < NTW; ++j) acc[m][j] = nan4();
    }
    if constexpr (ATOM) {
        uint32_t sv[4];
        dn_atomic_scales(svh_d + (size_t)e * N, (int)blockIdx.y, lane, sv);
        int eb = 0;
        const DnAtomic at{out, svh_d + (size_t)e * N, pair_sh, wts_sh, ebuf, N, slots, half};
        dn_atomic<IPM_WIDE_TILES>(acc, (cnt + 15) >> 4, wave, lane, (int)blockIdx.y, sv, at, eb);
        return;
    }
    float* Zm = Z + (size_t)mat * P * N;
#pragma unroll
    for (int m = 0; m < IPM_WIDE_TILES; ++m)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int row = m * 16 + 4 * (lane >> 4) + i;
            const int p = pair_sh[row];
            if (p < 0) continue;
#pragma unroll
            for (int j = 0; j < NTW; ++j) Zm[(size_t)p * N + (nt0 + j) * 16 + (lane & 15)] = acc[m][j][i];
        }
}

// ---- the staged item GEMM (widths 2..10) -------------------------------------------------------------------

constexpr int PK = 8;                             // k tiles a chunk: 128 k
constexpr int PXS = PK * 16 + 8;                  // LDS row stride of a staged activation chunk, halves (272 bytes)
constexpr int PW = 4;                             // waves a block: 8 column tiles, 128 columns
constexpr int PSTAGE = PK * 2 * 4 * STAGE_MAXK2;  // a wave's staged trellis words a chunk
constexpr int DNG = 16;  // down matrix: column blocks of 128 a block, small items (8, 24 and 48 measured slower at 512 rows)
constexpr int DNG_BIG = 2;  // the same for the larger items: more blocks for fewer items (4: 1 % slower at 512 rows)
constexpr int DNG_BIG_LONG = 4;   // passes of more than LONG_ROWS rows: 1.5 % faster at 2048 rows
constexpr int LONG_ROWS = 1024;
constexpr int GU_SPLIT = 2;                       // K splits of a larger item's gate|up (4 and 8 measured slower)
// The number of K splits of a larger item's gate|up over K (at most one a chunk).
static int gu_splits(int K) { return K / (PK * 16) < GU_SPLIT ? K / (PK * 16) : GU_SPLIT; }
constexpr int DXS = 2 * PK * 16 + 8;              // down matrix: LDS row stride of the activations (K up to 256)

// An activation piece (8 halves: column 8 q8 .. +7 of a chunk row) into LDS. Within each 32-k step of the row
// (16 words) word d goes to 4 (d & 3) + (d >> 2), so the words of a lane's MFMA operand (g, g + 4, g + 8, g + 12 of
// the step: the k order in which the trellis quads fill the B operand) are one 16-byte read.
__device__ __forceinline__ void put_a(uint16_t* row, int q8, const u4v& v) {
    uint32_t* w = reinterpret_cast<uint32_t*>(row) + 16 * (q8 >> 2) + (q8 & 3);
#pragma unroll
    for (int r = 0; r < 4; ++r) w[4 * r] = v[r];
}

// One chunk (PK k tiles) of a wave: its two column tiles times the item's first mts (<= MT) row tiles. The trellis
// words are staged in st (tile (t, j) at word (2 t + j) * 4 K2), the activations in xa (row stride xs halves, laid
// out by put_a); each tile pair decodes once and feeds all row tiles.
template <int CB, int K2, int MT>
__device__ __forceinline__ void item_chunk(const uint32_t* st, const LaneQuad& lq, const uint16_t* xa, int mts,
                                           int lane, f4v (&acc)[MT][2], int xs) {
    constexpr int TW = 4 * K2;
    const uint32_t* wa = st + lq.w0;
    const uint32_t* wb = st + lq.w1;
    const uint16_t* xr = xa + (lane & 15) * xs + 8 * ((lane >> 4) & 3);
#pragma unroll
    for (int t = 0; t < PK; t += 2) {
        h8v bb[2];
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const int t0 = (2 * t + j) * TW, t1 = (2 * (t + 1) + j) * TW;
            const u2v b0 = decode_quad<K2, CB>(wa[t0], wb[t0], lq.sh);
            const u2v b1 = decode_quad<K2, CB>(wa[t1], wb[t1], lq.sh);
            bb[j] = __builtin_bit_cast(h8v, (u4v{b0.x, b0.y, b1.x, b1.y}));
        }
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
            if (mt >= mts) break;  // the item's occupied row tiles only (uniform)
            const h8v a = *reinterpret_cast<const h8v*>(xr + mt * 16 * xs + t * 16);
            acc[mt][0] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, bb[0], acc[mt][0], 0, 0, 0);
            acc[mt][1] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, bb[1], acc[mt][1], 0, 0, 0);
        }
    }
}

// One chunk for a single row tile with the LDS reads one k step ahead: the trellis words and the activation operand
// of k step t + 1 are read before k step t decodes, so each read's latency overlaps a step of decoding.
template <int CB, int K2>
__device__ __forceinline__ void item_chunk1(const uint32_t* st, const LaneQuad& lq, const uint16_t* xa, int lane,
                                            f4v (&acc)[1][2], int xs) {
    constexpr int TW = 4 * K2;
    const uint32_t* wa = st + lq.w0;
    const uint32_t* wb = st + lq.w1;
    const uint16_t* xr = xa + (lane & 15) * xs + 8 * ((lane >> 4) & 3);
    uint32_t w[2][4][2];  // [buffer][tile: (t, j0), (t + 1, j0), (t, j1), (t + 1, j1)][word]
    h8v a[2];
    auto read = [&](int t, int b) __attribute__((always_inline)) {
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                const int o = (2 * (t + h) + j) * TW;
                w[b][2 * j + h][0] = wa[o];
                w[b][2 * j + h][1] = wb[o];
            }
        a[b] = *reinterpret_cast<const h8v*>(xr + t * 16);
    };
    read(0, 0);
#pragma unroll
    for (int t = 0; t < PK; t += 2) {
        const int b = (t >> 1) & 1;
        if (t + 2 < PK) read(t + 2, b ^ 1);
        issued();
        h8v bb[2];
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const u2v b0 = decode_quad<K2, CB>(w[b][2 * j][0], w[b][2 * j][1], lq.sh);
            const u2v b1 = decode_quad<K2, CB>(w[b][2 * j + 1][0], w[b][2 * j + 1][1], lq.sh);
            bb[j] = __builtin_bit_cast(h8v, (u4v{b0.x, b0.y, b1.x, b1.y}));
        }
        acc[0][0] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[b], bb[0], acc[0][0], 0, 0, 0);
        acc[0][1] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[b], bb[1], acc[0][1], 0, 0, 0);
    }
}

// The chunk loop of a gate|up block for one width: the activations one chunk ahead, the trellis two, two barriers a
// chunk (the activations are shared by the block's waves). Loads complete in issue order and every load is issued (a
// chunk past the last re-reads the last), so the waits stay exact.
template <int CB, int K2, int MT>
__device__ __forceinline__ void gu_loop(__amdgpu_buffer_rsrc_t xrs, const uint32_t (&aoff)[MT], const int (&lofs)[MT],
                                        const TileSpan& sp, uint16_t* xa, uint32_t* st, int lane, int q8, int mts,
                                        int c0, int nch, f4v (&acc)[MT][2]) {
    constexpr int NL = stage_loads_k<PK, K2>();
    const LaneQuad lq = lane_quad_k<K2>(lane);
    u4v av[MT], ta[NL], tb[NL];
    auto issue_a = [&](int c) __attribute__((always_inline)) {
        c = c0 + (c < nch ? c : nch - 1);
#pragma unroll
        for (int i = 0; i < MT; ++i)
            av[i] = __builtin_bit_cast(u4v, __builtin_amdgcn_raw_buffer_load_b128(xrs, aoff[i], c * PK * 32, 0));
    };
    auto issue_t = [&](int c, u4v (&tv)[NL]) __attribute__((always_inline)) {
        c = c0 + (c < nch ? c : nch - 1);
        TileSpan sc = sp;
        sc.off = sp.off + c * PK * sp.kstride;
        stage_issue_k<PK, K2>(sc, lane, tv);
    };
    auto step = [&](int c, u4v (&tv)[NL]) __attribute__((always_inline)) {
        __syncthreads();  // the previous chunk's reads of xa are done
#pragma unroll
        for (int i = 0; i < MT; ++i)
            if (i < mts) put_a(xa + lofs[i], q8, av[i]);
        stage_store_k<PK, K2>(st, lane, tv);  // only this wave reads its region, in order
        issue_a(c + 1);
        issue_t(c + 2, tv);
        __syncthreads();  // the chunk's activations are in LDS
        item_chunk<CB, K2, MT>(st, lq, xa, mts, lane, acc, PXS);
    };
    issue_t(0, ta);
    issue_t(1, tb);
    issue_a(0);
    // two steps an iteration with no exit between them, so every load's wait is counted the same on each pass
    int c = 0;
    for (; c + 1 < nch; c += 2) {
        step(c, ta);
        step(c + 1, tb);
    }
    if (c < nch) step(c, ta);  // uniform
}

// Block b of a launch over (items, C column blocks, Z slices) in XCD order. Blocks are dispatched to the 8 XCDs in
// turn (block b on XCD b mod 8); group g = item Z + slice takes blocks on XCD g mod 8 for all C of its column blocks
// (the item's activations of the slice come into that XCD's L2 once), and slice z of an expert's consecutive items
// lands on the XCDs (i Z + z) mod 8, 8 / gcd(Z, 8) of them (two for Z = 4 or 12), whose L2s then hold its trellis
// for the expert's later items. 2048 rows: 719 -> 691 us a layer (item order: a slice's blocks on all 8 XCDs, each
// fetching the slice). Blocks: ceil(items Z / 8) 8 C, those past the list's count return at once.
__device__ __forceinline__ void xcd_order(int b, int C, int Z, int& item, int& cb, int& z) {
    const int q = b >> 3;
    cb = q % C;
    const int g = (q / C) * 8 + (b & 7);
    item = g / Z;
    z = g % Z;
}
static unsigned xcd_blocks(int items, int C, int Z) { return (unsigned)((items * Z + 7) / 8 * 8 * C); }

// Block (item of the larger items' list, 128 columns, (matrix, K split)), in XCD order: the item's rows (up to
// IPM_TILES row tiles) times its expert's matrix over split s of K's chunks of 128 (splits [s nch / nsplit,
// (s + 1) nch / nsplit)).
// A chunk's activations go to LDS once for the block's four waves; each wave's two column tiles of the chunk come in
// as 16-byte loads staged in the wave's own LDS region. Only the item's occupied row tiles are loaded and multiplied;
// rows past the item's count read the item's first pair and are not stored (MFMA rows do not mix). Split 0 goes to
// Z[mat][pair][n], split s > 0 to Zp[s - 1][mat][pair][n] (fp32), each accumulated from zero (stored as 0 + sum).
template <int CB>
__global__ void __launch_bounds__(PW * 64) __attribute__((amdgpu_waves_per_eu(2)))
item_gu_kernel(const uint16_t* __restrict__ X0, const uint16_t* __restrict__ X1, const int64_t* __restrict__ TP0,
               const int64_t* __restrict__ TP1, const int* __restrict__ K2_0, const int* __restrict__ K2_1,
               const int* __restrict__ sorted, const int* __restrict__ items, const int* __restrict__ item_count,
               float* __restrict__ Z, float* __restrict__ Zp, int K, int N, int P, int nsplit, int mats, int max_items,
               int* __restrict__ status) {
    constexpr int MT = IPM_TILES;
    int e, first, cnt;
    int item, cb, zs;
    xcd_order((int)blockIdx.x, N / (16 * 2 * PW), mats * nsplit, item, cb, zs);
    if (!item_at(items, item_count, 1, max_items, item, e, first, cnt)) return;
    const int mat = zs / nsplit, split = zs % nsplit;
    const uint16_t* X = mat ? X1 : X0;
    const uint32_t* T = reinterpret_cast<const uint32_t*>(mat ? TP1[e] : TP0[e]);
    const int k2 = mat ? K2_1[e] : K2_0[e];
    // the wave index in a scalar register: the trellis offsets built from it are then scalar (a buffer load's soffset)
    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    __shared__ int pair_sh[MT * 16];
    __shared__ __attribute__((aligned(16))) uint16_t xa[MT * 16 * PXS];
    __shared__ __attribute__((aligned(16))) uint32_t st[PW][PSTAGE];
    if (tid < MT * 16) pair_sh[tid] = tid < cnt ? sorted[first + tid] : -1;
    __syncthreads();
    // this thread's activation pieces of every chunk: piece i is row 16 i + (tid >> 4), halves 8 (tid & 15) .. +7;
    // a piece past the item's row tiles reads row tile 0's address (a cache hit) and is not stored
    const int mts = (cnt + 15) >> 4;
    uint32_t aoff[MT];
    int lofs[MT];
#pragma unroll
    for (int i = 0; i < MT; ++i) {
        const int row = i * 16 + (tid >> 4);
        const int rr = i < mts ? row : (tid >> 4);
        const int p = pair_sh[rr] >= 0 ? pair_sh[rr] : pair_sh[0];
        aoff[i] = ((uint32_t)p * (uint32_t)K + 8u * (tid & 15)) * 2u;
        lofs[i] = row * PXS;
    }
    const __amdgpu_buffer_rsrc_t xrs = buffer_rsrc(X, (uint32_t)((size_t)P * K * 2));
    const int nt0 = cb * (2 * PW) + 2 * wave;
    const int ns = N >> 4, TWB = 16 * k2;
    TileSpan sp;
    sp.r = buffer_rsrc(T, (uint32_t)((K >> 4) * ns * TWB));
    sp.off = nt0 * TWB;
    sp.kstride = ns * TWB;
    f4v acc[MT][2];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) acc[mt][0] = acc[mt][1] = f4v{0.f, 0.f, 0.f, 0.f};
    const int nch = K / (PK * 16);
    const int c0 = split * nch / nsplit, nc = (split + 1) * nch / nsplit - c0;  // nsplit <= nch: nc >= 1
    const bool ok = EA_K2_SWITCH(
        k2, 2, 10, (gu_loop<CB, K2V, MT>(xrs, aoff, lofs, sp, xa, st[wave], lane, tid & 15, mts, c0, nc, acc)));
    if (!ok) {
        if (lane == 0) record_error(status, DEV_UNSUPPORTED_WIDTH);
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) acc[mt][0] = acc[mt][1] = nan4();
    }
    float* Zm = (split ? Zp + (size_t)(split - 1) * 2 * P * N : Z) + (size_t)mat * P * N;
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int p = pair_sh[mt * 16 + 4 * (lane >> 4) + i];
            if (p < 0) continue;
#pragma unroll
            for (int j = 0; j < 2; ++j) Zm[(size_t)p * N + (nt0 + j) * 16 + (lane & 15)] = 0.f + acc[mt][j][i];
        }
}

// Items of at most 16 pairs: a block is NW waves, one a column-tile pair of one matrix, over all of K. The block's
// waves share each chunk of activations through a ring of RING_S chunk slots in LDS, filled and freed with LDS
// counters instead of barriers, so a wave can run up to RING_S - RING_L - 1 chunks ahead of the slowest:
//   filled[s]: pieces stored into slot s, over all the chunks it has held (NW a chunk);
//   done[s]:   waves that have finished a chunk of slot s, over all its chunks (NW a chunk).
// At its step c a wave stores its piece of chunk p = c + RING_L into slot p % RING_S once every wave is done with
// that slot's previous chunk (done >= NW (p / RING_S)), waits until chunk c is complete in its slot
// (filled >= NW (c / RING_S + 1)), computes it, and counts itself done. The slowest wave can always go on (every
// chunk it waits for was stored at a step no later than its own, and every slot it stores into was freed before),
// so every wait ends. Each wave's trellis goes through its own LDS region as in gu_loop; the activation piece of a
// chunk (1/NW of it) and the trellis are loaded two chunks ahead. The nch chunks are summed as nsum splits
// ([s nch / nsum, (s + 1) nch / nsum)), each accumulated from zero and added in order into tot (from zero): the bits
// of a K-split item's sum of its split planes (item_gu_kernel, summed by the epilogue), so a pair's sums do not
// depend on which list its item is in.
constexpr int RING_S = 6;  // activation chunk slots
constexpr int RING_L = 2;  // a wave stores its piece of chunk c + RING_L at its step c

template <int NW>
struct RingPiece {  // a lane's words of a chunk: 16 rows x 64 words over NW waves
    static constexpr int WORDS = 16 * 64 / (NW * 64);
};

__device__ __forceinline__ int lds_load_acquire(const int* p) {
    return __hip_atomic_load(p, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_WORKGROUP);
}
// One count for the whole wave: only its first lane adds (the wait before the add covers every lane's accesses).
__device__ __forceinline__ void lds_add_release(int* p, int v, int lane) {
    if (lane == 0) __hip_atomic_fetch_add(p, v, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_WORKGROUP);
}
// Wait until *p >= target. Every count waited for is reached (see above); the wait is still bounded (about 2^20
// sleeps, tens of milliseconds): past the bound it gives up, returns false and the kernel reports EA_SYNC_TIMEOUT.
__device__ __forceinline__ bool lds_wait_geq(const int* p, int target) {
    for (int n = 0; lds_load_acquire(p) < target; ++n) {
        if (n >= (1 << 20)) return false;
        __builtin_amdgcn_s_sleep(1);
    }
    return true;
}

template <int CB, int K2, int NW>
__device__ __forceinline__ void ring_loop(__amdgpu_buffer_rsrc_t xrs, uint32_t aoff, int lofs, const TileSpan& sp,
                                          uint16_t* ring, int* filled, int* done, uint32_t* st, int lane, int nch,
                                          int nsum, f4v (&acc)[1][2], f4v (&tot)[1][2], bool& synced) {
    constexpr int NL = stage_loads_k<PK, K2>();
    constexpr int W = RingPiece<NW>::WORDS;  // 2 or 4
    constexpr int SLOT = 16 * PXS;
    using pv = uint32_t __attribute__((ext_vector_type(W)));
    const LaneQuad lq = lane_quad_k<K2>(lane);
    pv pa, pb;
    u4v ta[NL], tb[NL];
    int sn = 1;  // the next split's index
    auto issue_p = [&](int c, pv& v) __attribute__((always_inline)) {
        c = c < nch ? c : nch - 1;
        if constexpr (W == 4)
            v = __builtin_bit_cast(pv, __builtin_amdgcn_raw_buffer_load_b128(xrs, aoff, c * PK * 32, 0));
        else
            v = __builtin_bit_cast(pv, __builtin_amdgcn_raw_buffer_load_b64(xrs, aoff, c * PK * 32, 0));
    };
    auto issue_t = [&](int c, u4v (&tv)[NL]) __attribute__((always_inline)) {
        c = c < nch ? c : nch - 1;
        TileSpan sc = sp;
        sc.off = sp.off + c * PK * sp.kstride;
        stage_issue_k<PK, K2>(sc, lane, tv);
    };
    // the piece's words d .. d + W - 1 of its row (d = lofs & 63) at their transposed places (see put_a)
    auto put = [&](int p, const pv& v) __attribute__((always_inline)) {
        const int sl = p % RING_S;
        synced = synced && lds_wait_geq(&done[sl], NW * (p / RING_S));  // after a give-up no more waits
        uint32_t* w = reinterpret_cast<uint32_t*>(ring + sl * SLOT + (lofs >> 6) * PXS);
        const int d = lofs & 63;
#pragma unroll
        for (int r = 0; r < W; ++r) {
            const int dd = (d & 15) + r;  // word within its 32-k step
            w[16 * (d >> 4) + 4 * (dd & 3) + (dd >> 2)] = v[r];
        }
        lds_add_release(&filled[sl], 1, lane);
    };
    auto step = [&](int c, u4v (&tv)[NL], pv& v) __attribute__((always_inline)) {
        if (c + RING_L < nch) put(c + RING_L, v);  // uniform
        issue_p(c + RING_L + 2, v);
        stage_store_k<PK, K2>(st, lane, tv);
        issue_t(c + 2, tv);
        const int sl = c % RING_S;
        synced = synced && lds_wait_geq(&filled[sl], NW * (c / RING_S + 1));
        item_chunk1<CB, K2>(st, lq, ring + sl * SLOT, lane, acc, PXS);
        lds_add_release(&done[sl], 1, lane);  // after the chunk's reads of the slot have returned
        if (c + 1 == sn * nch / nsum) {  // the end of a split (uniform)
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                tot[0][j] += acc[0][j];
                acc[0][j] = f4v{0.f, 0.f, 0.f, 0.f};
            }
            ++sn;
        }
    };
    // chunks 0 .. RING_L - 1 go in before the loop; pa / pb then carry chunks RING_L and RING_L + 1
    for (int p = 0; p < RING_L && p < nch; ++p) {
        pv v;
        issue_p(p, v);
        put(p, v);
    }
    issue_p(RING_L, pa);
    issue_t(0, ta);
    issue_p(RING_L + 1, pb);
    issue_t(1, tb);
    int c = 0;
    for (; c + 1 < nch; c += 2) {  // two steps an iteration with no exit between them
        step(c, ta, pa);
        step(c + 1, tb, pb);
    }
    if (c < nch) step(c, ta, pa);  // uniform
}

template <int CB, int NW>
__global__ void __launch_bounds__(NW * 64) __attribute__((amdgpu_waves_per_eu(4)))
item_ring_kernel(const uint16_t* __restrict__ X0, const uint16_t* __restrict__ X1, const int64_t* __restrict__ TP0,
                 const int64_t* __restrict__ TP1, const int* __restrict__ K2_0, const int* __restrict__ K2_1,
                 const int* __restrict__ sorted, const int* __restrict__ items, const int* __restrict__ item_count,
                 float* __restrict__ Z, int K, int N, int P, int nsum, int max_items, int* __restrict__ status) {
    int e, first, cnt;
    if (!item_at(items, item_count, 0, max_items, blockIdx.x, e, first, cnt)) return;
    const int mat = blockIdx.z;
    const uint16_t* X = mat ? X1 : X0;
    const uint32_t* T = reinterpret_cast<const uint32_t*>(mat ? TP1[e] : TP0[e]);
    const int k2 = mat ? K2_1[e] : K2_0[e];
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    __shared__ int pair_sh[16];
    __shared__ int filled[RING_S], done[RING_S];
    __shared__ __attribute__((aligned(16))) uint16_t ring[RING_S * 16 * PXS];
    __shared__ __attribute__((aligned(16))) uint32_t st[NW][PSTAGE];
    if (threadIdx.x < 16) pair_sh[threadIdx.x] = (int)threadIdx.x < cnt ? sorted[first + threadIdx.x] : -1;
    if (threadIdx.x < RING_S) filled[threadIdx.x] = done[threadIdx.x] = 0;
    __syncthreads();
    // this lane's piece of every chunk: words [d, d + W) of row r (word index lofs = 64 r + d over the chunk);
    // a row past the count reads the first pair's row
    constexpr int W = RingPiece<NW>::WORDS;
    const int lofs = (wave * 64 + lane) * W;
    const int row = lofs >> 6;
    const int p = pair_sh[row] >= 0 ? pair_sh[row] : pair_sh[0];
    const uint32_t aoff = ((uint32_t)p * (uint32_t)K + 2u * (uint32_t)(lofs & 63)) * 2u;
    const __amdgpu_buffer_rsrc_t xrs = buffer_rsrc(X, (uint32_t)((size_t)P * K * 2));
    const int nt0 = blockIdx.y * (2 * NW) + 2 * wave;
    const int ns = N >> 4, TWB = 16 * k2;
    TileSpan sp;
    sp.r = buffer_rsrc(T, (uint32_t)((K >> 4) * ns * TWB));
    sp.off = nt0 * TWB;
    sp.kstride = ns * TWB;
    f4v acc[1][2], tot[1][2];
    acc[0][0] = acc[0][1] = tot[0][0] = tot[0][1] = f4v{0.f, 0.f, 0.f, 0.f};
    const int nch = K / (PK * 16);
    bool synced = true;
    const bool ok = EA_K2_SWITCH(k2, 2, 10,
                                 (ring_loop<CB, K2V, NW>(xrs, aoff, lofs, sp, ring, filled, done, st[wave], lane, nch,
                                                         nsum, acc, tot, synced)));
    if (!ok || !synced) {
        if (lane == 0) record_error(status, ok ? DEV_SYNC_TIMEOUT : DEV_UNSUPPORTED_WIDTH);
        tot[0][0] = tot[0][1] = nan4();
    }
    float* Zm = Z + (size_t)mat * P * N;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int pp = pair_sh[4 * (lane >> 4) + i];
        if (pp < 0) continue;
#pragma unroll
        for (int j = 0; j < 2; ++j) Zm[(size_t)pp * N + (nt0 + j) * 16 + (lane & 15)] = tot[0][j][i];
    }
}

// The column blocks of a down block for one width: step s is column block s / nch, chunk s % nch; the trellis two
// steps ahead; each column block's rows are stored when its last chunk is done.
template <int CB, int K2, int MT, int NG, bool ATOM>
__device__ __forceinline__ void dn_loop(const TileSpan& sp, const uint16_t* xa, uint32_t* st, int lane, int wave,
                                        int mts, int nch, int nb0, const int* pair_sh, float* __restrict__ Z, int N,
                                        const DnAtomic& at) {
    constexpr int NL = stage_loads_k<PK, K2>();
    constexpr int TWB = 16 * K2;
    const LaneQuad lq = lane_quad_k<K2>(lane);
    const int steps = NG * nch;  // even (NG even, or nch = 2: the caller's choice): two steps an iteration
    u4v ta[NL], tb[NL];
    f4v acc[MT][2];
    uint32_t sv[4];  // ATOM: svh_d of this thread's epilogue columns, loaded at a column block's first chunk
    int eb = 0;
    auto issue_t = [&](int s2, u4v (&tv)[NL]) __attribute__((always_inline)) {
        s2 = s2 < steps ? s2 : steps - 1;
        TileSpan sc = sp;
        sc.off = sp.off + (s2 / nch) * 8 * TWB + (s2 % nch) * PK * sp.kstride;
        stage_issue_k<PK, K2>(sc, lane, tv);
    };
    auto step = [&](int s2, u4v (&tv)[NL]) __attribute__((always_inline)) {
        const int c = s2 % nch;
        if (c == 0) {
#pragma unroll
            for (int mt = 0; mt < MT; ++mt) acc[mt][0] = acc[mt][1] = f4v{0.f, 0.f, 0.f, 0.f};
            if constexpr (ATOM) dn_atomic_scales(at.svh, nb0 + s2 / nch, lane, sv);
        }
        stage_store_k<PK, K2>(st, lane, tv);  // only this wave reads its region, in order
        issue_t(s2 + 2, tv);
        item_chunk<CB, K2, MT>(st, lq, xa + c * PK * 16, mts, lane, acc, DXS);
        if (c == nch - 1 && ATOM) {
            if constexpr (ATOM) dn_atomic<MT>(acc, mts, wave, lane, nb0 + s2 / nch, sv, at, eb);
        } else if (c == nch - 1) {
            const int nt0 = (nb0 + s2 / nch) * 8 + 2 * wave;
#pragma unroll
            for (int mt = 0; mt < MT; ++mt)
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const int p = pair_sh[mt * 16 + 4 * (lane >> 4) + i];
                    if (p < 0) continue;
#pragma unroll
                    for (int j = 0; j < 2; ++j) Z[(size_t)p * N + (nt0 + j) * 16 + (lane & 15)] = acc[mt][j][i];
                }
        }
    };
    issue_t(0, ta);
    issue_t(1, tb);
    for (int s2 = 0; s2 < steps; s2 += 2) {  // steps = NG nch is even: two steps an iteration, no exit between
        step(s2, ta);
        step(s2 + 1, tb);
    }
}

// The down matrix (K = I of 128 or 256: one or two chunks): a block (item of list MT > 2, NG column blocks of 128)
// loads the item's activations for all of K into LDS once, then its waves run the column blocks independently. WB = 8
// (the larger items with a pair plane): two groups of four waves, each over NG / 2 of the column blocks, share one copy
// of the activations, so two blocks fit a CU's LDS at four waves a SIMD (four-wave blocks: three at three).
template <int CB, int MT, int NG, bool ATOM, int WB = PW>
__global__ void __launch_bounds__(WB * 64) __attribute__((amdgpu_waves_per_eu(MT > 2 && WB == PW ? 2 : 4)))
item_dn_kernel(const uint16_t* __restrict__ X, const int64_t* __restrict__ TP, const int* __restrict__ K2T,
               const int* __restrict__ sorted, const int* __restrict__ items, const int* __restrict__ item_count,
               float* __restrict__ Z, int K, int N, int P, int max_items, int* __restrict__ status,
               const float* __restrict__ wts, const uint16_t* __restrict__ svh_d, void* __restrict__ out, int slots,
               int half) {
    int e, first, cnt;
    // the larger items' blocks in XCD order (a column group's slice of an expert on the same XCDs for all of the
    // expert's items); the small items' (one item an expert) item by item
    int item = blockIdx.x, grp = blockIdx.y;
    if constexpr (MT > 2) {
        int cb_unused;
        xcd_order((int)blockIdx.x, 1, N / 128 / NG, item, cb_unused, grp);
    }
    if (!item_at(items, item_count, MT > 2, max_items, item, e, first, cnt)) return;
    const uint32_t* T = reinterpret_cast<const uint32_t*>(TP[e]);
    const int k2 = K2T[e];
    // the wave index in a scalar register: the trellis offsets built from it are then scalar (a buffer load's soffset)
    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    __shared__ int pair_sh[MT * 16];
    __shared__ __attribute__((aligned(16))) uint16_t xa[MT * 16 * DXS];
    static_assert(WB == PW || (WB == 2 * PW && !ATOM && NG % 2 == 0), "two wave groups: pair-plane blocks");
    __shared__ __attribute__((aligned(16))) uint32_t st[WB][PSTAGE];
    constexpr int EWORDS = ATOM ? 2 * 16 * ES : 1;
    constexpr int WWORDS = ATOM ? MT * 16 : 1;
    __shared__ float ebuf[EWORDS];
    __shared__ float wts_sh[WWORDS];
    if (tid < MT * 16) pair_sh[tid] = tid < cnt ? sorted[first + tid] : -1;
    if constexpr (ATOM)
        if (tid < MT * 16) wts_sh[tid] = tid < cnt ? wts[sorted[first + tid]] : 0.f;
    __syncthreads();
    const int mts = (cnt + 15) >> 4;
    const int nch = K / (PK * 16);  // 1 or 2
    DnAtomic at{};
    if constexpr (ATOM) at = DnAtomic{out, svh_d + (size_t)e * N, pair_sh, wts_sh, ebuf, N, slots, half};
    {
        // 256 threads cover a chunk of a row tile; with eight waves each half of the block loads one chunk
        constexpr int CPT = WB == PW ? 2 : 1;  // chunks a thread loads
        const int lt = tid & 255, c0 = WB == PW ? 0 : tid >> 8;
        const __amdgpu_buffer_rsrc_t xrs = buffer_rsrc(X, (uint32_t)((size_t)P * K * 2));
        u4v av[CPT][MT];
#pragma unroll
        for (int q = 0; q < CPT; ++q)
#pragma unroll
            for (int i = 0; i < MT; ++i) {
                const int rr = i < mts ? i * 16 + (lt >> 4) : (lt >> 4);
                const int p = pair_sh[rr] >= 0 ? pair_sh[rr] : pair_sh[0];
                const int cc = c0 + q < nch ? c0 + q : 0;
                av[q][i] = __builtin_bit_cast(
                    u4v, __builtin_amdgcn_raw_buffer_load_b128(
                             xrs, ((uint32_t)p * (uint32_t)K + (uint32_t)(cc * PK * 16 + 8 * (lt & 15))) * 2u, 0, 0));
            }
#pragma unroll
        for (int q = 0; q < CPT; ++q)
#pragma unroll
            for (int i = 0; i < MT; ++i)
                if (c0 + q < nch && i < mts)
                    put_a(xa + (i * 16 + (lt >> 4)) * DXS + (c0 + q) * PK * 16, lt & 15, av[q][i]);
    }
    constexpr int NGW = WB == PW ? NG : NG / 2;  // column blocks a wave group runs
    const int ns = N >> 4, TWB = 16 * k2;
    const int w4 = wave & (PW - 1);
    const int nb0 = grp * NG + (wave / PW) * NGW;  // the wave group's first column block
    TileSpan sp;
    sp.r = buffer_rsrc(T, (uint32_t)((K >> 4) * ns * TWB));
    sp.off = (nb0 * 8 + 2 * w4) * TWB;
    sp.kstride = ns * TWB;
    __syncthreads();  // the activations are in LDS
    const bool ok = EA_K2_SWITCH(
        k2, 2, 10, (dn_loop<CB, K2V, MT, NGW, ATOM>(sp, xa, st[wave], lane, w4, mts, nch, nb0, pair_sh, Z, N, at)));
    if (!ok) {  // no product ran: the item's outputs of the block's column blocks are NaN
        if (lane == 0) record_error(status, DEV_UNSUPPORTED_WIDTH);
        for (int g = 0; g < NGW; ++g)
            for (int i = 0; i < MT * 16; ++i) {
                const int p = pair_sh[i];
                if (p < 0) continue;
                const size_t o = (size_t)(nb0 + g) * 128 + w4 * 32 + (lane & 31);
                if (!ATOM) Z[(size_t)p * N + o] = __builtin_nanf("");
                else if (!half) static_cast<float*>(out)[(size_t)(p / slots) * N + o] = __builtin_nanf("");
                else static_cast<uint16_t*>(out)[(size_t)(p / slots) * N + o] = 0x7E00;
            }
    }
}

// The down epilogue and slot combine of a prompt pass. Block (row r, 2048 columns): a thread holds 8 consecutive
// columns of one 128-block (16 lanes a block, lane l the columns 8 h8_group(l) .. + 7); for each slot in order
// y = FWHT(plane[pair]) * HAD_SCALE * svh_d[e], then out = fma(w, y, out) from zero, a slot without an expert adding
// w * 0. These are the operations and the order of down_combine_kernel with one split (the butterflies over
// value-index bits 0..6, three inside a lane and four across lanes: fwht128_x8), so the same bits (a zero y's sign
// does not reach out, which starts at +0); the rotated plane is not written back (nothing reads it after the combine).
// (prompt_experts.cu's deterministic combine; exl3_experts.cu:186-214 for the epilogue.)
__global__ void __launch_bounds__(256) prompt_combine_kernel(const float* __restrict__ Z, const int* __restrict__ pick,
                                                             const uint16_t* __restrict__ svh_d,
                                                             const float* __restrict__ wts, float* __restrict__ out,
                                                             int D, int E, int slots) {
    const int r = blockIdx.x, lane = threadIdx.x & 63;
    const int k = blockIdx.y * 2048 + 128 * ((int)threadIdx.x >> 4) + 8 * h8_group(lane);
    if (k >= D) return;  // whole 16-lane groups (D % 128 == 0)
    float a[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) a[j] = 0.f;
    // four slots at a time: their picks and weights, then all their plane and svh loads in flight before the first
    // slot's rotation (a slot without an expert loads pair 0's row and expert 0's scales, and adds w * 0)
    constexpr int QB = 4;
    for (int q0 = 0; q0 < slots; q0 += QB) {
        int ev[QB];
        float wv[QB];
        f4v z0[QB], z1[QB];
        u4v sv[QB];
#pragma unroll
        for (int j = 0; j < QB; ++j) {
            const int p = r * slots + (q0 + j < slots ? q0 + j : q0), e = pick[p];
            wv[j] = wts[p];
            ev[j] = e >= 0 && e < E ? p : -1;
            const size_t zo = (size_t)(ev[j] >= 0 ? p : r * slots) * D + k;
            z0[j] = *reinterpret_cast<const f4v*>(Z + zo);
            z1[j] = *reinterpret_cast<const f4v*>(Z + zo + 4);
            sv[j] = *reinterpret_cast<const u4v*>(svh_d + (size_t)(ev[j] >= 0 ? e : 0) * D + k);
        }
        issued();
#pragma unroll
        for (int j = 0; j < QB; ++j) {
            if (q0 + j >= slots) break;  // uniform
            float o[8];
            if (ev[j] >= 0) {  // uniform over the block
                float v[8];
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    v[i] = 0.f + z0[j][i];  // the split sum from zero
                    v[4 + i] = 0.f + z1[j][i];
                }
                const float sc = fwht128_x8(v, lane) * HAD_SCALE;  // the values' sign folded into the scale (exact)
#pragma unroll
                for (int i = 0; i < 8; ++i) o[i] = v[i] * sc * h2f((uint16_t)(sv[j][i >> 1] >> (16 * (i & 1))));
            } else {
#pragma unroll
                for (int i = 0; i < 8; ++i) o[i] = 0.f;
            }
#pragma unroll
            for (int i = 0; i < 8; ++i) a[i] = __builtin_fmaf(wv[j], o[i], a[i]);
        }
    }
    *reinterpret_cast<f4v*>(out + (size_t)r * D + k) = f4v{a[0], a[1], a[2], a[3]};
    *reinterpret_cast<f4v*>(out + (size_t)r * D + k + 4) = f4v{a[4], a[5], a[6], a[7]};
}

// out fp32 -> bf16 -> fp32 in place (prompt_experts.zig:246).
__global__ void round_kernel(float* __restrict__ out, size_t n) {
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x)
        out[i] = bf16r(out[i]);
}

static size_t align256(size_t n) { return (n + 255) & ~(size_t)255; }

struct PromptLayout {
    size_t sorted, items, count, xd, plane, xg, xu, z, zp, pclass, total;
    uint32_t rows, max_items;
    bool has_plane;
};

// Whether a pass without a pair plane covers the layer's shape: the atomic epilogue of the staged down GEMM takes
// K = I of at most 256 and whole pairs of 128-column blocks (D % 256 == 0). Other shapes keep the plane.
static bool atomic_down_fits(const ea_routed* ex) { return ex->width <= 2 * PK * 16 && ex->dims % 256 == 0; }

static PromptLayout prompt_layout(const ea_routed* ex, uint32_t rows, uint32_t slots, int planes) {
    PromptLayout l{};
    l.has_plane = planes || !atomic_down_fits(ex);
    const uint32_t r = rows < CHUNK_ROWS ? rows : CHUNK_ROWS;
    const size_t n = (size_t)r * slots, D = ex->dims, I = ex->width;
    l.rows = r;
    l.max_items = (uint32_t)(n / IPM + (n < ex->count ? n : ex->count));  // IPM <= IPM_WIDE: room for either
    size_t off = 0;
    auto take = [&](size_t b) {
        const size_t at = off;
        off += align256(b);
        return at;
    };
    l.sorted = take(n * 4);
    l.items = take(3 * (size_t)l.max_items * 4);
    l.count = take(16);
    l.xd = take(n * I * 2);
    l.plane = l.has_plane ? take(n * D * 4) : 0;  // per-pair down outputs (the reference's pair plane)
    l.xg = take(n * D * 2);
    l.xu = take(n * D * 2);
    l.z = take(2 * n * I * 4);
    l.zp = take((size_t)(gu_splits((int)D) - 1) * 2 * n * I * 4);
    l.pclass = take(n * 4);
    l.total = off;
    return l;
}

// The atomic epilogue's arguments for a down launch (out null: the pair plane Z instead).
struct DownOut {
    const float* wts = nullptr;
    const uint16_t* svh_d = nullptr;
    void* out = nullptr;
    int slots = 0, half = 0;
};

template <int CB, int LO, int HI>
static void item_gemm(hipStream_t s, const uint16_t* X0, const uint16_t* X1, const int64_t* TP0, const int64_t* TP1,
                      const int* B0, const int* B1, const int* sorted, const int* items, const int* count, float* Z,
                      int K, int N, int P, int mats, uint32_t max_items, int* status, const DownOut& d = DownOut{}) {
    constexpr int NTW = 2, NW = 4;
    dim3 grid(max_items, (N / 16 + NTW * NW - 1) / (NTW * NW), mats);
    for (int big = 1; big >= 0; --big) {
        if (d.out)
            item_gemm_kernel<CB, LO, HI, NTW, NW, true><<<grid, NW * 64, 0, s>>>(
                X0, X1, TP0, TP1, B0, B1, sorted, items, count, Z, K, N, P, big, (int)max_items, status, d.wts,
                d.svh_d, d.out, d.slots, d.half);
        else
            item_gemm_kernel<CB, LO, HI, NTW, NW, false><<<grid, NW * 64, 0, s>>>(
                X0, X1, TP0, TP1, B0, B1, sorted, items, count, Z, K, N, P, big, (int)max_items, status, nullptr,
                nullptr, nullptr, 0, 0);
    }
}

// What one item list's pass reads and writes: the rotated activations, the three matrices' trellis tables and
// widths, the items, the pair classes and the per-pair planes (z and zp: gate|up partial sums, xd: down inputs,
// plane: down outputs). The two lists' pairs are disjoint, so their passes touch disjoint rows of every plane.
struct ListPass {
    const uint16_t *xg, *xu;
    const int64_t* tp[3];
    const int* k2[3];
    const int *sorted, *items, *count, *pclass, *pick;
    const uint16_t *svh_g, *svh_u, *suh_d;
    float *z, *zp, *plane;
    uint16_t* xd;
    int D, I, P, rows, slots, E, mi;
    int* status;
    DownOut down;  // out set: no pair plane, the down items add into out (fp32, or fp16 with half)
};

// One item list from its gate|up product to its down product, in order on q: big = 1 takes the larger items (the
// gate|up K split into zp; the down matrix by blocks of DNG_BIG column blocks), big = 0 the items of at most
// SMALL_ROWS pairs (the ring kernel; DNG column blocks). The down matrix takes the resident-activation kernel when
// its K and N fit, the chunked ones otherwise. The two lists run on two streams: the small items' blocks leave room
// on many CUs, the larger items' blocks are few and long, and each list's down product starts when its own
// epilogue is done.
template <int CB>
static int list_pass(hipStream_t q, const ListPass& a, int big) {
    const int ns = gu_splits(a.D);
    if (big)
        item_gu_kernel<CB><<<xcd_blocks(a.mi, a.I / (16 * 2 * PW), 2 * ns), PW * 64, 0, q>>>(
            a.xg, a.xu, a.tp[0], a.tp[1], a.k2[0], a.k2[1], a.sorted, a.items, a.count, a.z, a.zp, a.D, a.I, a.P, ns,
            2, a.mi, a.status);
    else  // blocks of 4 waves over 128 columns (8 waves over 256 measured 1 % slower at 512 rows, the same at 2048)
        item_ring_kernel<CB, 4><<<dim3(a.mi, a.I / 128, 2), 4 * 64, 0, q>>>(
            a.xg, a.xu, a.tp[0], a.tp[1], a.k2[0], a.k2[1], a.sorted, a.items, a.count, a.z, a.D, a.I, a.P, ns, a.mi,
            a.status);
    int r = launched();
    if (r) return r;
    r = launch_gateup_epilogue(q, a.z, a.pick, a.svh_g, a.svh_u, a.suh_d, a.xd, (uint32_t)a.rows, (uint32_t)a.P,
                               (uint32_t)a.I, 1, (uint32_t)a.slots, (uint32_t)a.E, __builtin_inff(), 1, a.pclass, a.zp,
                               (uint32_t)ns, big);
    if (r) return r;
    if (a.down.out) {  // no pair plane: the atomic epilogue (atomic_down_fits holds)
        const DownOut& d = a.down;
        const int nb = a.D / 128;
        if (big && a.rows > LONG_ROWS && nb % DNG_BIG_LONG == 0)
            item_dn_kernel<CB, IPM_TILES, DNG_BIG_LONG, true><<<xcd_blocks(a.mi, 1, nb / DNG_BIG_LONG), PW * 64, 0, q>>>(
                a.xd, a.tp[2], a.k2[2], a.sorted, a.items, a.count, nullptr, a.I, a.D, a.P, a.mi, a.status, d.wts,
                d.svh_d, d.out, d.slots, d.half);
        else if (big)
            item_dn_kernel<CB, IPM_TILES, DNG_BIG, true><<<xcd_blocks(a.mi, 1, nb / DNG_BIG), PW * 64, 0, q>>>(
                a.xd, a.tp[2], a.k2[2], a.sorted, a.items, a.count, nullptr, a.I, a.D, a.P, a.mi, a.status, d.wts,
                d.svh_d, d.out, d.slots, d.half);
        else if (nb % DNG == 0)
            item_dn_kernel<CB, SMALL_ROWS / 16, DNG, true><<<dim3(a.mi, nb / DNG, 1), PW * 64, 0, q>>>(
                a.xd, a.tp[2], a.k2[2], a.sorted, a.items, a.count, nullptr, a.I, a.D, a.P, a.mi, a.status, d.wts,
                d.svh_d, d.out, d.slots, d.half);
        else
            item_dn_kernel<CB, SMALL_ROWS / 16, 2, true><<<dim3(a.mi, nb / 2, 1), PW * 64, 0, q>>>(
                a.xd, a.tp[2], a.k2[2], a.sorted, a.items, a.count, nullptr, a.I, a.D, a.P, a.mi, a.status, d.wts,
                d.svh_d, d.out, d.slots, d.half);
    } else if (a.I <= 2 * PK * 16 && (a.D / 128) % DNG == 0) {
        if (big && a.rows > LONG_ROWS && (a.D / 128) % DNG_BIG_LONG == 0)
            item_dn_kernel<CB, IPM_TILES, DNG_BIG_LONG, false, 2 * PW>
                <<<xcd_blocks(a.mi, 1, a.D / 128 / DNG_BIG_LONG), 2 * PW * 64, 0, q>>>(
                a.xd, a.tp[2], a.k2[2], a.sorted, a.items, a.count, a.plane, a.I, a.D, a.P, a.mi, a.status, nullptr,
                nullptr, nullptr, 0, 0);
        else if (big && a.I == 2 * PK * 16)  // two chunks of K: a wave group's one column block is an even step count
            item_dn_kernel<CB, IPM_TILES, DNG_BIG, false, 2 * PW>
                <<<xcd_blocks(a.mi, 1, a.D / 128 / DNG_BIG), 2 * PW * 64, 0, q>>>(
                a.xd, a.tp[2], a.k2[2], a.sorted, a.items, a.count, a.plane, a.I, a.D, a.P, a.mi, a.status, nullptr,
                nullptr, nullptr, 0, 0);
        else if (big)
            item_dn_kernel<CB, IPM_TILES, DNG_BIG, false><<<xcd_blocks(a.mi, 1, a.D / 128 / DNG_BIG), PW * 64, 0, q>>>(
                a.xd, a.tp[2], a.k2[2], a.sorted, a.items, a.count, a.plane, a.I, a.D, a.P, a.mi, a.status, nullptr,
                nullptr, nullptr, 0, 0);
        else
            item_dn_kernel<CB, SMALL_ROWS / 16, DNG, false><<<dim3(a.mi, a.D / 128 / DNG, 1), PW * 64, 0, q>>>(
                a.xd, a.tp[2], a.k2[2], a.sorted, a.items, a.count, a.plane, a.I, a.D, a.P, a.mi, a.status, nullptr,
                nullptr, nullptr, 0, 0);
    } else if (big) {
        item_gu_kernel<CB><<<xcd_blocks(a.mi, a.D / (16 * 2 * PW), 1), PW * 64, 0, q>>>(
            a.xd, a.xd, a.tp[2], a.tp[2], a.k2[2], a.k2[2], a.sorted, a.items, a.count, a.plane, nullptr, a.I, a.D,
            a.P, 1, 1, a.mi, a.status);
    } else {
        item_ring_kernel<CB, 4><<<dim3(a.mi, a.D / 128, 1), 4 * 64, 0, q>>>(
            a.xd, a.xd, a.tp[2], a.tp[2], a.k2[2], a.k2[2], a.sorted, a.items, a.count, a.plane, a.I, a.D, a.P, 1,
            a.mi, a.status);
    }
    return launched();
}

// Both lists at once, joined once before the combine. The list whose blocks are dispatched first: the larger items
// up to LONG_ROWS rows a pass (512 rows: 339 us a layer against 355 with the small items first), the small items
// above it (2048 rows: 734 against 767 us), where the larger items fill the GPU for most of the pass and the small
// items' chain would otherwise wait for CUs at each of its steps. Launched eagerly, the side stream's list is
// enqueued (and dispatched) first; a captured graph's replay runs the main stream's branch first, so under capture
// the first list goes on the main stream.
static int list_passes(hipStream_t s, uint32_t cb, const ListPass& a) {
    auto pass = [&](hipStream_t q, int big) {
        return cb == 1 ? list_pass<1>(q, a, big) : cb == 2 ? list_pass<2>(q, a, big) : list_pass<0>(q, a, big);
    };
    hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(s, &cap) != hipSuccess) {
        cap = hipStreamCaptureStatusNone;
        (void)hipGetLastError();  // the query's own error is not a launch's
    }
    const int first = a.rows > LONG_ROWS ? 0 : 1;
    const int side = cap == hipStreamCaptureStatusActive ? 1 - first : first;
    return fork_join(
        s, [&](hipStream_t q) { return pass(q, side); }, [&](hipStream_t q) { return pass(q, 1 - side); });
}

// Widths above 10 (three trellis words a lane): the register-streaming GEMM, both lists in turn on s.
static void wide_gemm(hipStream_t s, uint32_t cb, const uint16_t* X0, const uint16_t* X1, const int64_t* TP0,
                      const int64_t* TP1, const int* B0, const int* B1, const int* sorted, const int* items,
                      const int* count, float* Z, int K, int N, int P, int mats, uint32_t max_items, int* status,
                      const DownOut& d = DownOut{}) {
    if (cb == 1) {
        item_gemm<1, 2, 16>(s, X0, X1, TP0, TP1, B0, B1, sorted, items, count, Z, K, N, P, mats, max_items, status, d);
    } else if (cb == 2) {
        item_gemm<2, 2, 16>(s, X0, X1, TP0, TP1, B0, B1, sorted, items, count, Z, K, N, P, mats, max_items, status, d);
    } else {
        item_gemm<0, 2, 16>(s, X0, X1, TP0, TP1, B0, B1, sorted, items, count, Z, K, N, P, mats, max_items, status, d);
    }
}

// A decode window of more than 16 rows through the prefill path (ea_moe_routed): the moe scratch holds a prompt
// scratch with the pair plane (the slots added in order, so a window's rows get the same bits on every run) in its
// region; both follow from the layer's shape.
size_t prompt_region_bytes(const ea_routed* ex, uint32_t rows, uint32_t slots) {
    return prompt_layout(ex, rows, slots, 1).total;
}

int prompt_region_carve(const ea_routed* ex, uint32_t rows, uint32_t slots, uint64_t base, ea_prompt_scratch* s) {
    const PromptLayout l = prompt_layout(ex, rows, slots, 1);
    s->sorted = base + l.sorted;
    s->items = base + l.items;
    s->count = base + l.count;
    s->xd = base + l.xd;
    s->plane = base + l.plane;
    s->xg = base + l.xg;
    s->xu = base + l.xu;
    s->z = base + l.z;
    s->zp = base + l.zp;
    s->pclass = base + l.pclass;
    s->rows = l.rows;
    s->slots = slots;
    s->max_items = l.max_items;
    return EA_OK;
}

}  // namespace ea

using namespace ea;

extern "C" {

int ea_prompt_experts_supported(const ea_routed* ex, int* ok) {
    EA_REQUIRE_CTX(c);
    if (!ex || !ok) return EA_BAD_ARGUMENT;
    *ok = 0;
    if (ex->cb > 2 || ex->width % 128 || ex->dims % 128 || ex->count == 0) return EA_OK;
    for (int m = 0; m < 3; ++m) {
        int32_t* k2 = new int32_t[ex->count];
        const int r = hip_status(hipMemcpy(k2, dptr<void>(ex->k2[m]), ex->count * 4, hipMemcpyDeviceToHost));
        bool good = r == EA_OK;
        for (uint32_t e = 0; good && e < ex->count; ++e) good = k2[e] >= 2 && k2[e] <= 16;
        delete[] k2;
        if (r) return r;
        if (!good) return EA_OK;
    }
    *ok = 1;
    return EA_OK;
}

size_t ea_prompt_scratch_bytes(const ea_routed* ex, uint32_t rows, uint32_t slots, int planes) {
    if (!ex || rows == 0 || slots == 0) return 0;
    return prompt_layout(ex, rows, slots, planes).total;
}

int ea_prompt_scratch_init(ea_stream_t stream, ea_prompt_scratch* s, void* base, size_t bytes, const ea_routed* ex,
                           uint32_t rows, uint32_t slots, int planes) {
    EA_REQUIRE_CTX(c);
    if (!s || !base || !ex || rows == 0 || slots == 0 || slots > 32) return EA_BAD_ARGUMENT;
    if (reinterpret_cast<uintptr_t>(base) & 255) return EA_BAD_ARGUMENT;
    const PromptLayout l = prompt_layout(ex, rows, slots, planes);
    if (bytes < l.total) return EA_SCRATCH_TOO_SMALL;
    const uint64_t b = reinterpret_cast<uintptr_t>(base);
    s->sorted = b + l.sorted;
    s->items = b + l.items;
    s->count = b + l.count;
    s->xd = b + l.xd;
    s->plane = l.has_plane ? b + l.plane : 0;
    s->xg = b + l.xg;
    s->xu = b + l.xu;
    s->z = b + l.z;
    s->zp = b + l.zp;
    s->pclass = b + l.pclass;
    s->rows = l.rows;
    s->slots = slots;
    s->max_items = l.max_items;
    // only the count word needs a defined start (prompt_experts.zig:109-110)
    return fill_words(as_stream(stream), dptr<void>(s->count), 0u, 4);
}

int ea_prompt_experts_run(ea_stream_t stream, const void* x, int x_dtype, uint32_t xstride, const int32_t* pick,
                          const float* wts, const ea_routed* ex, const ea_prompt_scratch* sc, void* out, uint32_t R,
                          int do_round, int half_sums) {
    EA_REQUIRE_CTX(c);
    if (half_sums && do_round) return EA_INVALID;  // prompt_experts.zig:147
    if (half_sums && sc && sc->plane) return EA_INVALID;  // prompt_experts.zig:155: the pair plane takes fp32 rows only
    if (!x || !pick || !wts || !ex || !sc || !out) return EA_BAD_ARGUMENT;
    if (x_dtype < 0 || x_dtype > 2 || sc->slots == 0) return EA_BAD_ARGUMENT;
    if (ex->width % 128 || ex->dims % 128) return EA_BAD_WIDTH;
    // no pair plane: the down items add each slot into out with atomics (packed fp16 pairs with half_sums), which a
    // scratch made for this layer's shape allows (atomic_down_fits) and which needs out 4-byte aligned
    const bool atom = sc->plane == 0;
    if (atom && (!atomic_down_fits(ex) || (reinterpret_cast<uintptr_t>(out) & 3))) return EA_BAD_ARGUMENT;
    hipStream_t s = as_stream(stream);
    const uint32_t D = ex->dims, I = ex->width, E = ex->count, S = sc->slots;
    const size_t xb = x_dtype == 2 ? 4 : 2;
    const size_t ob = half_sums ? 2 : 4;
    const bool wide = ex->k2_gu[1] > 10 || ex->k2_d[1] > 10;
    for (uint32_t r0 = 0; r0 < R; r0 += sc->rows) {
        const uint32_t n = R - r0 < sc->rows ? R - r0 : sc->rows;
        const uint32_t pairs = n * S;
        const int ipm = wide ? IPM_WIDE : IPM;
        const uint32_t items_n = (uint32_t)(pairs / ipm + (pairs < E ? pairs : E));
        const uint32_t max_items = items_n < sc->max_items ? items_n : sc->max_items;
        const char* xs = static_cast<const char*>(x) + (size_t)r0 * xstride * xb;
        const int32_t* pk = pick + (size_t)r0 * S;
        const float* wt = wts + (size_t)r0 * S;
        route_kernel<<<1, ROUTE_THREADS, 3 * E * sizeof(int), s>>>(pk, (int)pairs, (int)E, dptr<int>(sc->sorted),
                                                                  dptr<int>(sc->items), dptr<int>(sc->count),
                                                                  dptr<int>(sc->pclass), (int)max_items, ipm);
        int r = launched();
        if (r) return r;
        // without a plane the pass's rows of out are cleared by the rotation launch, before any down item adds
        char* opass = static_cast<char*>(out) + (size_t)r0 * D * ob;
        r = launch_rot_in(s, xs, x_dtype, xstride, pk, dptr<const uint16_t>(ex->suh_g), dptr<const uint16_t>(ex->suh_u),
                          dptr<uint16_t>(sc->xg), dptr<uint16_t>(sc->xu), n, D, S, E, atom ? opass : nullptr,
                          half_sums);
        if (r) return r;
        DownOut down;
        if (atom) {
            down.wts = wt;
            down.svh_d = dptr<const uint16_t>(ex->svh_d);
            down.out = opass;
            down.slots = (int)S;
            down.half = half_sums;
        }
        if (!wide) {
            ListPass a{};
            a.xg = dptr<const uint16_t>(sc->xg);
            a.xu = dptr<const uint16_t>(sc->xu);
            for (int m = 0; m < 3; ++m) {
                a.tp[m] = dptr<const int64_t>(ex->ptr[m]);
                a.k2[m] = dptr<const int>(ex->k2[m]);
            }
            a.sorted = dptr<const int>(sc->sorted);
            a.items = dptr<const int>(sc->items);
            a.count = dptr<const int>(sc->count);
            a.pclass = dptr<const int>(sc->pclass);
            a.pick = pk;
            a.svh_g = dptr<const uint16_t>(ex->svh_g);
            a.svh_u = dptr<const uint16_t>(ex->svh_u);
            a.suh_d = dptr<const uint16_t>(ex->suh_d);
            a.z = dptr<float>(sc->z);
            a.zp = dptr<float>(sc->zp);
            a.plane = dptr<float>(sc->plane);
            a.xd = dptr<uint16_t>(sc->xd);
            a.D = (int)D;
            a.I = (int)I;
            a.P = (int)pairs;
            a.rows = (int)n;
            a.slots = (int)S;
            a.E = (int)E;
            a.mi = (int)max_items;
            a.status = c->status;
            a.down = down;
            r = list_passes(s, ex->cb, a);
        } else {
            wide_gemm(s, ex->cb, dptr<const uint16_t>(sc->xg), dptr<const uint16_t>(sc->xu),
                      dptr<const int64_t>(ex->ptr[0]), dptr<const int64_t>(ex->ptr[1]), dptr<const int>(ex->k2[0]),
                      dptr<const int>(ex->k2[1]), dptr<const int>(sc->sorted), dptr<const int>(sc->items),
                      dptr<const int>(sc->count), dptr<float>(sc->z), (int)D, (int)I, (int)pairs, 2, max_items,
                      c->status);
            r = launched();
            if (r) return r;
            r = launch_gateup_epilogue(s, dptr<const float>(sc->z), pk, dptr<const uint16_t>(ex->svh_g),
                                       dptr<const uint16_t>(ex->svh_u), dptr<const uint16_t>(ex->suh_d),
                                       dptr<uint16_t>(sc->xd), n, pairs, I, 1, S, E, __builtin_inff(), 1);
            if (r) return r;
            wide_gemm(s, ex->cb, dptr<const uint16_t>(sc->xd), dptr<const uint16_t>(sc->xd),
                      dptr<const int64_t>(ex->ptr[2]), dptr<const int64_t>(ex->ptr[2]), dptr<const int>(ex->k2[2]),
                      dptr<const int>(ex->k2[2]), dptr<const int>(sc->sorted), dptr<const int>(sc->items),
                      dptr<const int>(sc->count), dptr<float>(sc->plane), (int)I, (int)D, (int)pairs, 1, max_items,
                      c->status, down);
            r = launched();
        }
        if (r) return r;
        if (atom) {  // every slot is in out already
            if (do_round) {
                round_kernel<<<1024, 256, 0, s>>>(reinterpret_cast<float*>(opass), (size_t)n * D);
                r = launched();
                if (r) return r;
            }
            continue;
        }
        // the pair plane summed in slot order (fp32 rows only: half sums were refused above); slots without an
        // expert add nothing (the reference's route skips them)
        float* o32 = reinterpret_cast<float*>(opass);
        if ((reinterpret_cast<uintptr_t>(o32) & 15) == 0) {  // 16-byte stores
            prompt_combine_kernel<<<dim3(n, (D + 2047) / 2048), 256, 0, s>>>(dptr<const float>(sc->plane), pk,
                                                                             dptr<const uint16_t>(ex->svh_d), wt, o32,
                                                                             (int)D, (int)E, (int)S);
            r = launched();
        } else {
            r = launch_down_combine(s, dptr<const float>(sc->plane), pk, dptr<const uint16_t>(ex->svh_d),
                                    dptr<float>(sc->plane), wt, o32, n, pairs, D, 1, S, E, true);
        }
        if (r) return r;
        if (do_round) {
            round_kernel<<<1024, 256, 0, s>>>(o32, (size_t)n * D);
            r = launched();
        }
        if (r) return r;
    }
    return EA_OK;
}

}  // extern "C"
