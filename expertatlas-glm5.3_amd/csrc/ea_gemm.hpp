// The MFMA core shared by the expert GEMV / GEMM and the EXL3 linear: a wavefront multiplies up to MG groups of 16
// activation rows by a strip of trellis tiles, decoding each tile once into v_mfma_f32_16x16x32_f16 B operands.
#pragma once

#include "ea_device.hpp"

namespace ea {

typedef const __attribute__((address_space(1))) uint32_t* gptr_u32;

// A global-memory load the compiler can see is global (not flat): trellis tables hold plain 64-bit addresses.
__device__ __forceinline__ uint32_t gload(const uint32_t* p) { return *(gptr_u32)(p); }

// A lane's constant view of any tile for K2 (its word indices and funnel shift; see quad_of / quad3_of).
template <int K2, int CB>
struct TileLane {
    static constexpr int NW = K2 <= 10 ? 2 : 3;  // words a lane reads from a tile
    int w0, w1, w2, sh;
    __device__ __forceinline__ explicit TileLane(int lane) {
        if constexpr (K2 <= 10) {
            const Quad q = quad_of<K2>(mfma_lane_p0(lane));
            w0 = q.wa;
            w1 = q.wb;
            w2 = 0;
            sh = q.sh;
        } else {
            const Quad3 q = quad3_of<K2>(mfma_lane_p0(lane));
            w0 = q.w0;
            w1 = q.w1;
            w2 = q.w2;
            sh = q.sh;
        }
    }
    // This lane's words of the tile starting at `tile`.
    __device__ __forceinline__ void fetch(const uint32_t* __restrict__ tile, uint32_t (&w)[NW]) const {
        w[0] = gload(tile + w0);
        w[1] = gload(tile + w1);
        if constexpr (NW == 3) w[2] = gload(tile + w2);
    }
    // The same through a buffer resource: the tile starts `soff` bytes into it (a scalar offset), so the addressing
    // costs no vector registers beyond the lane's word offsets.
    __device__ __forceinline__ void fetch(__amdgpu_buffer_rsrc_t r, int soff, uint32_t (&w)[NW]) const {
        w[0] = __builtin_amdgcn_raw_buffer_load_b32(r, 4 * w0, soff, 0);
        w[1] = __builtin_amdgcn_raw_buffer_load_b32(r, 4 * w1, soff, 0);
        if constexpr (NW == 3) w[2] = __builtin_amdgcn_raw_buffer_load_b32(r, 4 * w2, soff, 0);
    }
    // The four values as two packed words (values 0, 1 in .x; 2, 3 in .y).
    __device__ __forceinline__ u2v decode(const uint32_t (&w)[NW]) const {
        if constexpr (K2 <= 10) return decode_quad<K2, CB>(w[0], w[1], sh);
        else return decode_quad3<K2, CB>(w[0], w[1], w[2], sh);
    }
    // This lane's four B values of the tile starting at `tile`.
    __device__ __forceinline__ u2v decode_at(const uint32_t* __restrict__ tile) const {
        uint32_t w[NW];
        fetch(tile, w);
        return decode(w);
    }
};

// The lane's A operand of a two-tile k step at k = k0 (16x16x32): rows k0 + 2g, +1, +8, +9 and the same 16 later,
// g = lane >> 4; the same k permutation as the decoded B operand.
__device__ __forceinline__ h8v load_a8(const uint16_t* __restrict__ xrow, int k0, int lane) {
    if (!xrow) return h8v{0, 0, 0, 0, 0, 0, 0, 0};
    const uint16_t* xk = xrow + k0 + 2 * ((lane >> 4) & 3);
    const u4v au = {*reinterpret_cast<const uint32_t*>(xk), *reinterpret_cast<const uint32_t*>(xk + 8),
                    *reinterpret_cast<const uint32_t*>(xk + 16), *reinterpret_cast<const uint32_t*>(xk + 24)};
    return __builtin_bit_cast(h8v, au);
}

__device__ __forceinline__ h4v load_a4(const uint16_t* __restrict__ xrow, int k0, int lane) {
    if (!xrow) return h4v{0, 0, 0, 0};
    const uint16_t* xk = xrow + k0 + 2 * ((lane >> 4) & 3);
    const u2v au = {*reinterpret_cast<const uint32_t*>(xk), *reinterpret_cast<const uint32_t*>(xk + 8)};
    return __builtin_bit_cast(h4v, au);
}

// acc[m][j] += rows(m) @ tiles: tile (t, j) of the strip at base + t * kstride + j * TW words for t in [0, nkt);
// xrow[m]: this lane's activation row (lane & 15) of row group m, or nullptr; k0: the k of tile 0.
// Output layout of acc[m][j]: lane l holds D[4 (l >> 4) + i][l & 15] (row, column within the 16 x 16 tile).
// Software-pipelined: the trellis words of the next two-tile step are in flight while this step decodes.
template <int CB, int K2, int NTW, int MG>
__device__ __forceinline__ void wave_tiles(const uint32_t* __restrict__ base, size_t kstride, int nkt, int k0,
                                           const uint16_t* const (&xrow)[MG], int lane, f4v (&acc)[MG][NTW]) {
    constexpr int TW = 4 * K2;
    using TL = TileLane<K2, CB>;
    constexpr int NWD = TL::NW;
    const TL tl(lane);
    uint32_t wa[NTW][2][NWD], wb[NTW][2][NWD];
    auto fetch = [&](uint32_t (&w)[NTW][2][NWD], int t) __attribute__((always_inline)) {
        const uint32_t* t0 = base + (size_t)t * kstride;
#pragma unroll
        for (int j = 0; j < NTW; ++j) {
            tl.fetch(t0 + j * TW, w[j][0]);
            tl.fetch(t0 + kstride + j * TW, w[j][1]);
        }
    };
    // the activations of a step are loaded before the next step's trellis words, so waiting for them leaves the
    // trellis prefetch in flight (loads complete in issue order)
    auto load_a = [&](h8v (&a)[MG], int t) __attribute__((always_inline)) {
#pragma unroll
        for (int m = 0; m < MG; ++m) a[m] = load_a8(xrow[m], k0 + t * 16, lane);
    };
    auto compute = [&](uint32_t (&w)[NTW][2][NWD], const h8v (&a)[MG]) __attribute__((always_inline)) {
#pragma unroll
        for (int j = 0; j < NTW; ++j) {
            const u2v b0 = tl.decode(w[j][0]);
            const u2v b1 = tl.decode(w[j][1]);
            const h8v b = __builtin_bit_cast(h8v, (u4v{b0.x, b0.y, b1.x, b1.y}));
#pragma unroll
            for (int m = 0; m < MG; ++m) acc[m][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[m], b, acc[m][j], 0, 0, 0);
        }
    };
    const int steps = nkt >> 1;
    if (steps > 0) fetch(wa, 0);
    int s = 0;
    for (; s + 2 <= steps; s += 2) {
        h8v a0[MG], a1[MG];
        load_a(a0, 2 * s);
        fetch(wb, 2 * s + 2);
        asm volatile("" ::: "memory");  // keep the prefetch issued ahead of this step's decode
        compute(wa, a0);
        load_a(a1, 2 * s + 2);
        if (s + 2 < steps) fetch(wa, 2 * s + 4);
        asm volatile("" ::: "memory");
        compute(wb, a1);
    }
    if (s < steps) {
        h8v a0[MG];
        load_a(a0, 2 * s);
        compute(wa, a0);
    }
    if (nkt & 1) {
        const int t = nkt - 1;
        h4v a[MG];
#pragma unroll
        for (int m = 0; m < MG; ++m) a[m] = load_a4(xrow[m], k0 + t * 16, lane);
        const uint32_t* t0 = base + (size_t)t * kstride;
#pragma unroll
        for (int j = 0; j < NTW; ++j) {
            const h4v b = __builtin_bit_cast(h4v, tl.decode_at(t0 + j * TW));
#pragma unroll
            for (int m = 0; m < MG; ++m) acc[m][j] = __builtin_amdgcn_mfma_f32_16x16x16f16(a[m], b, acc[m][j], 0, 0, 0);
        }
    }
}

__device__ __forceinline__ void record_error(int* status, int code) { atomicCAS(status, 0, code); }

// ---- hand-offs between blocks of one launch ------------------------------------------------------------------------
// Data handed to another block is written with agent-scope stores (coherent across the XCDs' L2s); the writer waits for
// its stores (stores_done), meets its block at a barrier, and only then one thread counts in; a reader loads the data
// with agent-scope loads issued after it has seen the count.
__device__ __forceinline__ void st_coh(float* p, float v) { __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); }
__device__ __forceinline__ void st_coh(uint32_t* p, uint32_t v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_coh2(float* p, float2 v) {
    __hip_atomic_store(reinterpret_cast<uint64_t*>(p), __builtin_bit_cast(uint64_t, v), __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint32_t ld_coh(const uint32_t* p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float2 ld_coh2(const float* p) {
    return __builtin_bit_cast(float2, __hip_atomic_load(reinterpret_cast<const uint64_t*>(p), __ATOMIC_RELAXED,
                                                        __HIP_MEMORY_SCOPE_AGENT));
}
__device__ __forceinline__ int ld_coh(const int* p) { return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); }
__device__ __forceinline__ int count_in(int* c) { return __hip_atomic_fetch_add(c, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); }
__device__ __forceinline__ void reset_count(int* c) { __hip_atomic_store(c, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); }
// Every store this wave issued has completed (and, being agent-scope, is visible to every block).
__device__ __forceinline__ void stores_done() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }

// A product that could not run (a width without a decoder, a bounded wait that gave up) stores NaN in place of its
// sums, so the call's output shows the failure as well as the status word.
__device__ __forceinline__ f4v nan4() {
    const float n = __builtin_nanf("");
    return f4v{n, n, n, n};
}

// A raw buffer resource over `bytes` bytes at `base` (gfx9 word 3: 32-bit data, no format conversion). `base` must
// be wave-uniform.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buffer_rsrc(const void* base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, 0x00020000);
}

// Dispatch a runtime K2 to wave_tiles<..., K2, ...> for K2 in [LO, HI]; false when outside.
#define EA_K2_SWITCH(k2, LO, HI, CALL)                                        \
    [&]() -> bool {                                                           \
        switch (k2) {                                                         \
            EA_K2_CASE(2, LO, HI, CALL) EA_K2_CASE(3, LO, HI, CALL)           \
            EA_K2_CASE(4, LO, HI, CALL) EA_K2_CASE(5, LO, HI, CALL)           \
            EA_K2_CASE(6, LO, HI, CALL) EA_K2_CASE(7, LO, HI, CALL)           \
            EA_K2_CASE(8, LO, HI, CALL) EA_K2_CASE(9, LO, HI, CALL)           \
            EA_K2_CASE(10, LO, HI, CALL) EA_K2_CASE(11, LO, HI, CALL)         \
            EA_K2_CASE(12, LO, HI, CALL) EA_K2_CASE(13, LO, HI, CALL)         \
            EA_K2_CASE(14, LO, HI, CALL) EA_K2_CASE(15, LO, HI, CALL)         \
            EA_K2_CASE(16, LO, HI, CALL)                                      \
            default: return false;                                            \
        }                                                                     \
    }()
#define EA_K2_CASE(K2_, LO, HI, CALL)                    \
    case K2_:                                            \
        if constexpr (K2_ >= LO && K2_ <= HI) {          \
            constexpr int K2V = K2_;                     \
            CALL;                                        \
            return true;                                 \
        } else {                                         \
            return false;                                \
        }

// ---- trellis staging through LDS (the decode layer and the prefill GEMM) ------------------------------------

constexpr int STAGE_MAXK2 = 10;  // widest trellis (K2) the staged paths decode: two words a lane a tile

// Where an item's tiles are: a buffer over the whole matrix, the byte offset of tile (0, 0) and the byte stride between
// k tiles; tile (t, j) sits at off + t * kstride + j * 16 K2 bytes (j: the wave's two column tiles, adjacent).
struct TileSpan {
    __amdgpu_buffer_rsrc_t r;
    int off, kstride;
};

// The two words of a tile this lane's four values come from and their bit offset, for a width in 2..10 (zeros for
// any other: the loads stay inside the buffer and the product then reports the width).
struct LaneQuad {
    int w0, w1, sh;
};
__device__ __forceinline__ LaneQuad lane_quad(int k2, int lane) {
    LaneQuad r{0, 0, 0};
    EA_K2_SWITCH(k2, 2, 10, ([&] {
                     const Quad q = quad_of<K2V>(mfma_lane_p0(lane));
                     r = LaneQuad{q.wa, q.wb, q.sh};
                 }()));
    return r;
}

// A wave's trellis of an item: the NKT rows of its two column tiles (2 * 16 K2 contiguous bytes a row) read with
// 16-byte loads, ceil(NKT * K2 / 32) a wave; lane l of load i carries chunk 64 i + l (row c / (2 K2), 16-byte column
// c % (2 K2)). Wide loads keep fewer requests in flight for the same bytes than a word a lane a tile.
template <int NKT>
constexpr int stage_loads() {
    return (NKT * 2 * STAGE_MAXK2 + 63) / 64;
}

template <int NKT>
__device__ __forceinline__ void stage_issue(const TileSpan& sp, int k2, int lane, u4v (&v)[stage_loads<NKT>()]) {
    // a width outside 2..10 stages nothing (its product reports the width): the region holds STAGE_MAXK2 rows
    const bool fits = k2 >= 2 && k2 <= STAGE_MAXK2;
    const int cpr = fits ? 2 * k2 : 1, chunks = fits ? NKT * cpr : 0;
    const int inv = (65536 + cpr - 1) / cpr;  // c / cpr == (c * inv) >> 16 for every chunk c < 16 * 20
    // every load is issued (a lane past the last chunk reads the last one again), so no branch hides from the
    // compiler how many loads are in flight
    const int last = chunks > 0 ? chunks - 1 : 0;
#pragma unroll
    for (int i = 0; i < stage_loads<NKT>(); ++i) {
        const int c = min(64 * i + lane, last);
        const int t = (c * inv) >> 16, col = c - t * cpr;
        v[i] = __builtin_bit_cast(u4v, __builtin_amdgcn_raw_buffer_load_b128(sp.r, t * sp.kstride + col * 16, sp.off,
                                                                               0));
    }
}

// Issue order: a compiler barrier after a batch of loads, then hold() on each earlier load's value. The values can
// only be used after the holds, which follow every load of the batch; without them the scheduler may consume an
// earlier load (and wait for it) before issuing the rest.
__device__ __forceinline__ void issued() { asm volatile("" ::: "memory"); }
template <typename T>
__device__ __forceinline__ void hold(T& v) {
    asm volatile("" : "+v"(v));
}

// The chunks into the wave's LDS region in order: tile (t, j) then starts at word (2 t + j) * 4 K2. Only the wave
// itself reads its region, and a wave's LDS accesses complete in order, so no barrier follows.
template <int NKT>
__device__ __forceinline__ void stage_store(uint32_t* st, int k2, int lane, const u4v (&v)[stage_loads<NKT>()]) {
    const int chunks = (k2 >= 2 && k2 <= STAGE_MAXK2) ? NKT * 2 * k2 : 0;
#pragma unroll
    for (int i = 0; i < stage_loads<NKT>(); ++i) {
        const int c = 64 * i + lane;
        if (c < chunks) *reinterpret_cast<u4v*>(st + 4 * c) = v[i];
    }
}

// The same for a width known at compile time: the loads a wave issues are exactly ceil(NKT * K2 / 32), and the
// chunk -> (row, column) split is a multiply by a constant.
template <int NKT, int K2>
constexpr int stage_loads_k() {
    return (NKT * 2 * K2 + 63) / 64;
}
template <int NKT, int K2>
__device__ __forceinline__ void stage_issue_k(const TileSpan& sp, int lane, u4v (&v)[stage_loads_k<NKT, K2>()]) {
    constexpr int cpr = 2 * K2, last = NKT * cpr - 1;
#pragma unroll
    for (int i = 0; i < stage_loads_k<NKT, K2>(); ++i) {
        const int c = 64 * i + lane < last ? 64 * i + lane : last;
        const int t = c / cpr, col = c - t * cpr;
        v[i] = __builtin_bit_cast(u4v, __builtin_amdgcn_raw_buffer_load_b128(sp.r, t * sp.kstride + col * 16, sp.off,
                                                                               0));
    }
}
template <int NKT, int K2>
__device__ __forceinline__ void stage_store_k(uint32_t* st, int lane, const u4v (&v)[stage_loads_k<NKT, K2>()]) {
#pragma unroll
    for (int i = 0; i < stage_loads_k<NKT, K2>(); ++i) {
        const int c = 64 * i + lane;
        if ((NKT * 2 * K2) % 64 == 0 || c < NKT * 2 * K2) *reinterpret_cast<u4v*>(st + 4 * c) = v[i];
    }
}
template <int K2>
__device__ __forceinline__ LaneQuad lane_quad_k(int lane) {
    const Quad q = quad_of<K2>(mfma_lane_p0(lane));
    return LaneQuad{q.wa, q.wb, q.sh};
}

}  // namespace ea
