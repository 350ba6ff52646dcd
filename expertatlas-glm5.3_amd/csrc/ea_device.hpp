// Device helpers shared by the gfx950 kernels: number formats, the path's exp, EXL3 trellis decode into
// MFMA operand registers, and the 128-point Walsh-Hadamard transform on a 64-lane wavefront.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace ea {

typedef _Float16 h2v __attribute__((ext_vector_type(2)));
typedef _Float16 h4v __attribute__((ext_vector_type(4)));
typedef _Float16 h8v __attribute__((ext_vector_type(8)));
// Decoded B operands travel as packed words (two fp16 values a word, the first in the low half) and become h4v / h8v
// only as whole registers: hipcc has mis-compiled fp16 element reads of a bit-cast vector (every element read as
// element 0), so no code here reads single fp16 elements of a decoded pair.
typedef uint32_t u2v __attribute__((ext_vector_type(2)));
typedef uint32_t u4v __attribute__((ext_vector_type(4)));
typedef float f4v __attribute__((ext_vector_type(4)));

constexpr float HAD_SCALE = 0.08838834764831845f;  // 1 / sqrt(128) as fp32 (decode.cuh:163)

enum Codebook : int { CB_3INST = 0, CB_MCG = 1, CB_MUL1 = 2 };
enum DType : int { F16 = 0, BF16 = 1, F32 = 2 };

// ---- number formats -------------------------------------------------------------------------------------------

// An fp32 value the compiler must materialise as it stands: stops it fusing the multiply that made the value into
// a following fp16 conversion (v_fma_mixlo_f16 rounds the exact product once, not the fp32 product).
__device__ __forceinline__ float materialise(float x) {
    asm volatile("" : "+v"(x));
    return x;
}

__device__ __forceinline__ float h2f(uint16_t h) { return (float)__builtin_bit_cast(_Float16, h); }
// fp32 -> fp16, round to nearest even, from the fp32 value itself.
__device__ __forceinline__ uint16_t f2h(float f) { return __builtin_bit_cast(uint16_t, (_Float16)materialise(f)); }
// Two fp32 values -> a packed fp16 pair (the first in the low half), each rounded to nearest even from the fp32 value
// itself: one v_cvt_pk_f16_f32.
__device__ __forceinline__ uint32_t f2h2(float a, float b) {
    typedef float f2v __attribute__((ext_vector_type(2)));
    return __builtin_bit_cast(uint32_t, __builtin_convertvector((f2v){materialise(a), materialise(b)}, h2v));
}
__device__ __forceinline__ float bf2f(uint16_t b) { return __builtin_bit_cast(float, (uint32_t)b << 16); }
__device__ __forceinline__ uint16_t f2bf(float f) {
    uint32_t u = __builtin_bit_cast(uint32_t, f);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40);
    u += 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}
__device__ __forceinline__ float bf16r(float x) { return bf2f(f2bf(x)); }

// One element of an activation array of dtype dt as fp32.
__device__ __forceinline__ float load_act(const void* p, int dt, size_t i) {
    if (dt == F32) return static_cast<const float*>(p)[i];
    const uint16_t v = static_cast<const uint16_t*>(p)[i];
    return dt == BF16 ? bf2f(v) : h2f(v);
}
__device__ __forceinline__ void store_act(void* p, int dt, size_t i, float v) {
    if (dt == F32) static_cast<float*>(p)[i] = v;
    else static_cast<uint16_t*>(p)[i] = dt == BF16 ? f2bf(v) : f2h(v);
}

// The path's exp: Cody & Waite reduction x = n ln2 + r, a degree-7 Taylor polynomial by Horner with fma, 2^n by
// exponent scaling. Only IEEE fma / add / multiply / ldexp, so the CPU checker computes the same bits.
// Straight-line code (the special cases are selects), so loads around a call are not serialized by its branches.
__device__ __forceinline__ float expf_path(float x) {
    const float xc = __builtin_fminf(__builtin_fmaxf(x, -104.0f), 89.0f);  // keeps n in range; NaN -> -104
    const float n = __builtin_rintf(xc * 1.44269502162933349609f);
    float r = __builtin_fmaf(-n, 0.693145751953125f, xc);
    r = __builtin_fmaf(-n, 1.42860682030941723212e-06f, r);
    float p = 1.98412698412698412e-04f;
    p = __builtin_fmaf(p, r, 1.38888888888888889e-03f);
    p = __builtin_fmaf(p, r, 8.33333333333333333e-03f);
    p = __builtin_fmaf(p, r, 4.16666666666666667e-02f);
    p = __builtin_fmaf(p, r, 1.66666666666666667e-01f);
    p = __builtin_fmaf(p, r, 0.5f);
    p = __builtin_fmaf(p, r, 1.0f);
    p = __builtin_fmaf(p, r, 1.0f);
    const int ni = (int)n;
    const float lo = __builtin_ldexpf(__builtin_ldexpf(p, ni + 64), -64);  // results below 2^-125: two steps
    float v = ni < -125 ? lo : __builtin_ldexpf(p, ni);
    v = x < -103.972084045410156f ? 0.0f : v;
    v = x > 88.72283935546875f ? __builtin_inff() : v;
    return x != x ? x : v;
}

// The router top-8's ranking key of a choice: order-preserving over numbers (a larger float has a larger key, +0 and -0
// share one), NaN just above 0, the key of a taken expert. A NaN choice so ranks below every number (-inf included),
// NaNs among themselves by the lower id, and a taken expert is never picked again. Both top-8 paths rank by it.
__device__ __forceinline__ uint32_t order_key(float f) {
    const uint32_t b = __builtin_bit_cast(uint32_t, f + 0.0f);
    const uint32_t k = (b & 0x80000000u) ? ~b : (b | 0x80000000u);
    return f != f ? 1u : k;
}

// ---- EXL3 trellis -------------------------------------------------------------------------------------------
// A 16x16 tile is a circular big-endian bit stream of 128 * K2 bits in 4 * K2 words; value p's 16-bit state is
// stream bits [E(p) - 16, E(p)); value p = 8 L + j sits at row 2 (L & 3) + (j & 1) + 8 ((j >> 1) & 1), column
// (L >> 2) + 8 (j >> 2) of the tile (decode.cuh:16-136).

template <int K2>
__host__ __device__ constexpr int stream_end(int p) {
    return (K2 & 1) ? ((p + 1) * K2 - ((p + 1) & 1)) / 2 : (p + 1) * (K2 / 2);
}

// Codebook value of one 16-bit state as fp16 (decode.cuh:86-120). The state's bits above 15 are ignored.
template <int CB>
__device__ __forceinline__ _Float16 cb_value(uint32_t s) {
    s &= 0xffffu;
    if constexpr (CB == CB_MUL1) {
        const uint32_t x = s * 0x83DCD12Du;
        const uint32_t h = __builtin_amdgcn_udot4(x, 0x01010101u, 0x6400u, false);  // 1024 + byte sum, fp16 bits
        return __builtin_fmaf16(__builtin_bit_cast(_Float16, (uint16_t)h), __builtin_bit_cast(_Float16, (uint16_t)0x1eee),
                                __builtin_bit_cast(_Float16, (uint16_t)0xc931));
    } else {
        uint32_t x = (CB == CB_MCG) ? s * 0xCBAC1FEDu : s * 89226354u + 64248484u;
        x = (x & 0x8FFF8FFFu) ^ 0x3B603B60u;
        return __builtin_bit_cast(_Float16, (uint16_t)(x & 0xffffu)) + __builtin_bit_cast(_Float16, (uint16_t)(x >> 16));
    }
}

// Two codebook values of two clean 16-bit states as a packed fp16 pair (the first in the low half): the same bits
// as cb_value in 3 VALU instructions a value. mcg / 3inst: one multiply (and add) a state, one v_bitop3 a state for
// (x & 0x8FFF8FFF) ^ 0x3B603B60 (truth table 0x6A over (x, mask, pattern)), one fp16 add of its two halves written
// into its half of the result. mul1: multiply, byte sum by v_dot4, one packed fp16 fma.
template <int CB>
__device__ __forceinline__ uint32_t cb_pair(uint32_t s0, uint32_t s1) {
    if constexpr (CB == CB_MUL1) {
        const uint32_t h0 = __builtin_amdgcn_udot4(s0 * 0x83DCD12Du, 0x01010101u, 0x6400u, false);
        const uint32_t h1 = __builtin_amdgcn_udot4(s1 * 0x83DCD12Du, 0x01010101u, 0x6400u, false);
        const h2v hh = __builtin_bit_cast(h2v, h0 | (h1 << 16));
        const h2v c1 = {__builtin_bit_cast(_Float16, (uint16_t)0x1eee), __builtin_bit_cast(_Float16, (uint16_t)0x1eee)};
        const h2v c0 = {__builtin_bit_cast(_Float16, (uint16_t)0xc931), __builtin_bit_cast(_Float16, (uint16_t)0xc931)};
        return __builtin_bit_cast(uint32_t, __builtin_elementwise_fma(hh, c1, c0));
    } else {
        const uint32_t x0 = (CB == CB_MCG) ? s0 * 0xCBAC1FEDu : s0 * 89226354u + 64248484u;
        const uint32_t x1 = (CB == CB_MCG) ? s1 * 0xCBAC1FEDu : s1 * 89226354u + 64248484u;
        // the mask and xor are the same in both halves: one bitop3 ((x & m) ^ c, table 0x6A) a state, then one fp16
        // add of a word's two halves a value (SDWA selects the halves and the destination half)
        const uint32_t a = __builtin_amdgcn_bitop3_b32(x0, 0x8FFF8FFFu, 0x3B603B60u, 0x6A);
        const uint32_t b = __builtin_amdgcn_bitop3_b32(x1, 0x8FFF8FFFu, 0x3B603B60u, 0x6A);
        // Both adds write half a register (SDWA dst_sel WORD_0 / WORD_1), and on gfx950 a half-register write needs
        // wait states before anything reads that register: the second add reads the first's (it keeps the low half),
        // and the MFMA or VALU that takes the pair reads the second's. The compiler inserts such wait states for code
        // it generates but cannot see them inside an asm string, so they are part of the sequence itself: two after
        // each add. Without them the result depended on how far the scheduler happened to place the readers: the
        // register-streaming item GEMM built for 3 row tiles summed wrong at widths 12-16 while the 7-tile build
        // passed. (The compiler's own form of these adds writes both halves padded and merges them with a v_or:
        // one VALU more a pair, measured 1-3.5 % slower on the decode-bound kernels.)
        uint32_t r;
        asm("v_add_f16_sdwa %0, %1, %1 dst_sel:WORD_0 dst_unused:UNUSED_PAD src0_sel:WORD_0 src1_sel:WORD_1\n\t"
            "s_nop 1\n\t"
            "v_add_f16_sdwa %0, %2, %2 dst_sel:WORD_1 dst_unused:UNUSED_PRESERVE src0_sel:WORD_0 src1_sel:WORD_1\n\t"
            "s_nop 1"
            : "=&v"(r)
            : "v"(a), "v"(b));
        return r;
    }
}

// A lane's view of four consecutive stream values p0 .. p0 + 3 (p0 even) of a tile, for K2 <= 10: their four
// windows lie inside the 32 stream bits that start at the first window, so one funnel shift of two words gives
// all four. Lane constants: the two word indices and the shift.
struct Quad {
    int wa, wb, sh;
};

template <int K2>
__host__ __device__ constexpr Quad quad_of(int p0) {
    constexpr int TW = 4 * K2, NB = 128 * K2;
    const int b0 = stream_end<K2>(p0) - 16 + NB;  // first window start, made positive
    const int a = (b0 - 1) >> 5;                  // word pair (a, a + 1) holds bits [32a, 32a + 64) with b0 - 32a in 1..32
    return Quad{a % TW, (a + 1) % TW, 32 - (b0 - 32 * a)};
}

// The four values from the lane's two words: one funnel shift, then a bit-field extract a state.
template <int K2, int CB>
__device__ __forceinline__ u2v decode_quad(uint32_t wa, uint32_t wb, int sh) {
    static_assert(K2 >= 2 && K2 <= 10, "the four windows must fit in 32 stream bits");
    const uint32_t seg = __builtin_amdgcn_alignbit(wa, wb, (uint32_t)sh);
    constexpr int e0 = stream_end<K2>(0);
    const uint32_t s0 = seg >> 16;
    const uint32_t s1 = __builtin_amdgcn_ubfe(seg, 16 - (stream_end<K2>(1) - e0), 16);
    const uint32_t s2 = __builtin_amdgcn_ubfe(seg, 16 - (stream_end<K2>(2) - e0), 16);
    const uint32_t s3 = __builtin_amdgcn_ubfe(seg, 16 - (stream_end<K2>(3) - e0), 16);
    return u2v{cb_pair<CB>(s0, s1), cb_pair<CB>(s2, s3)};
}

// Wider widths (K2 11..16): the four windows span up to 40 stream bits, so the lane reads three words and makes a
// 64-bit segment from two funnel shifts.
struct Quad3 {
    int w0, w1, w2, sh;
};

template <int K2>
__host__ __device__ constexpr Quad3 quad3_of(int p0) {
    constexpr int TW = 4 * K2, NB = 128 * K2;
    const int b0 = stream_end<K2>(p0) - 16 + NB;
    const int a = (b0 - 1) >> 5;
    return Quad3{a % TW, (a + 1) % TW, (a + 2) % TW, 32 - (b0 - 32 * a)};
}

template <int K2, int CB>
__device__ __forceinline__ u2v decode_quad3(uint32_t w0, uint32_t w1, uint32_t w2, int sh) {
    static_assert(K2 >= 11 && K2 <= 16, "three-word form");
    const uint32_t hi = __builtin_amdgcn_alignbit(w0, w1, (uint32_t)sh);
    const uint32_t lo = __builtin_amdgcn_alignbit(w1, w2, (uint32_t)sh);
    constexpr int e0 = stream_end<K2>(0);
    uint32_t s[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int d = (i == 0) ? 0 : (i == 1 ? stream_end<K2>(1) - e0 : (i == 2 ? stream_end<K2>(2) - e0 : stream_end<K2>(3) - e0));
        s[i] = d <= 16 ? __builtin_amdgcn_ubfe(hi, 16 - d, 16)
                       : (__builtin_amdgcn_alignbit(hi, lo, (uint32_t)(48 - d)) & 0xffffu);
    }
    return u2v{cb_pair<CB>(s[0], s[1]), cb_pair<CB>(s[2], s[3])};
}

// MFMA 16x16x16 f16 B-operand layout for one tile: lane l holds B[k'][n] for n = l & 15 and k' = 4 (l >> 4) + i.
// With g = l >> 4 and tile lane L = 4 (n & 7) + g, h = n >> 3, the stream values p0 = 8 L + 4 h + i sit at rows
// k = 2 g + (i & 1) + 8 (i >> 1) of column n. So the lane decodes four consecutive values, and the A operand
// (activations) must use the same k permutation: lane l of A holds rows 2g, 2g + 1, 2g + 8, 2g + 9.
__host__ __device__ constexpr int mfma_lane_p0(int lane) {
    const int n = lane & 15, g = (lane >> 4) & 3;
    return 8 * (4 * (n & 7) + g) + 4 * (n >> 3);
}

// ---- Walsh-Hadamard over 128 values on a wavefront ------------------------------------------------------------
// Lane j holds values 2j and 2j + 1. Levels run over index bits 0, 1, .., 6 in that order, each pair becoming
// (lower + upper, lower - upper) in fp32: the reference's butterflies (decode.cuh:146-161), so the same bits.
// The value of lane (l ^ M) in lane l, without the LDS crossbar: DPP within a row of 16 (xor 1 and 2 are quad
// permutes, xor 4 = half-row mirror after quad reverse, xor 8 = row rotation by 8) and gfx950's
// permlane swaps across rows (xor 16) and halves (xor 32).
template <int M>
__device__ __forceinline__ float lane_xor(float v) {
    const int x = __builtin_bit_cast(int, v);
    if constexpr (M == 1) {
        return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(x, 0xB1, 0xf, 0xf, false));  // quad_perm 1,0,3,2
    } else if constexpr (M == 2) {
        return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(x, 0x4E, 0xf, 0xf, false));  // quad_perm 2,3,0,1
    } else if constexpr (M == 4) {
        const int r = __builtin_amdgcn_mov_dpp(x, 0x1B, 0xf, 0xf, false);                    // lane ^ 3
        return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(r, 0x141, 0xf, 0xf, false));  // then ^ 7
    } else if constexpr (M == 8) {
        return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(x, 0x128, 0xf, 0xf, false));  // row_ror:8
    } else if constexpr (M == 16) {
        // swapping the odd rows of one copy with the even rows of another leaves row r's partner in the copy that
        // did not keep row r
        const auto p = __builtin_amdgcn_permlane16_swap((unsigned)x, (unsigned)x, false, false);
        const bool odd_row = (__builtin_amdgcn_mbcnt_hi(~0u, __builtin_amdgcn_mbcnt_lo(~0u, 0u)) >> 4) & 1;
        return __builtin_bit_cast(float, odd_row ? p[0] : p[1]);
    } else {
        static_assert(M == 32, "lane_xor: 1, 2, 4, 8, 16 or 32");
        const auto p = __builtin_amdgcn_permlane32_swap((unsigned)x, (unsigned)x, false, false);
        const bool upper = __builtin_amdgcn_mbcnt_hi(~0u, __builtin_amdgcn_mbcnt_lo(~0u, 0u)) >= 32;
        return __builtin_bit_cast(float, upper ? p[0] : p[1]);
    }
}

template <int M>
__device__ __forceinline__ void fwht_level(float& v0, float& v1, int lane) {
    const float o0 = lane_xor<M>(v0), o1 = lane_xor<M>(v1);
    const bool up = lane & M;
    v0 = up ? o0 - v0 : v0 + o0;
    v1 = up ? o1 - v1 : v1 + o1;
}

__device__ __forceinline__ void fwht128_w64(float& v0, float& v1, int lane) {
    const float a = v0 + v1, b = v0 - v1;
    v0 = a;
    v1 = b;
    fwht_level<1>(v0, v1, lane);
    fwht_level<2>(v0, v1, lane);
    fwht_level<4>(v0, v1, lane);
    fwht_level<8>(v0, v1, lane);
    fwht_level<16>(v0, v1, lane);
    fwht_level<32>(v0, v1, lane);
}

// ---- Walsh-Hadamard over 128 values held eight a lane by 16 lanes ---------------------------------------------
// Lane l of a 16-lane group holds values 8 h8_group(l) .. + 7. The butterflies run over value-index bits 0..6 in that
// order: bits 0..2 inside the lane, bits 3..6 across lanes at distances 1, 2, 7 and 8 (h8_group places the groups so
// that each of those distances is one DPP pattern: the two quad permutes, the half-row mirror, the row rotation by 8).
// A cross-lane step is one v_fmac_f32 with the partner's value as its DPP operand: v + s * partner, s = -1 in the lane
// holding the butterfly's upper element, whose result is then (lower - upper) negated, exactly (s = +-1, one
// rounding); the partner of every later step holds a value of the same sign, so after the four steps each lane's true
// values are its values times the returned sign, (-1)^popcount(group). Nonzero results are the plain butterflies'
// bits; a caller that scales by the sign with an fma adding +0 also returns every zero as +0.
__device__ __forceinline__ int h8_group(int lane) {
    const int l = lane & 15;
    return l ^ (((l >> 2) & 1) * 3);
}

// The four cross-lane steps of eight values in one statement, so their order is fixed: every DPP read comes eight
// instructions after the write of its register, the leading s_nop covers the first read, and the trailing one a DPP
// read of the last results by the code that follows (a VALU write followed by a DPP read of the same register needs
// two wait states, which the compiler's hazard pass does not see across an asm statement).
#define EA_FMAC_DPP8(ctl, s)                                                                                      \
    "v_fmac_f32_dpp %0, %0, " s " " ctl " row_mask:0xf bank_mask:0xf\n\t"                                           \
    "v_fmac_f32_dpp %1, %1, " s " " ctl " row_mask:0xf bank_mask:0xf\n\t"                                           \
    "v_fmac_f32_dpp %2, %2, " s " " ctl " row_mask:0xf bank_mask:0xf\n\t"                                           \
    "v_fmac_f32_dpp %3, %3, " s " " ctl " row_mask:0xf bank_mask:0xf\n\t"                                           \
    "v_fmac_f32_dpp %4, %4, " s " " ctl " row_mask:0xf bank_mask:0xf\n\t"                                           \
    "v_fmac_f32_dpp %5, %5, " s " " ctl " row_mask:0xf bank_mask:0xf\n\t"                                           \
    "v_fmac_f32_dpp %6, %6, " s " " ctl " row_mask:0xf bank_mask:0xf\n\t"                                           \
    "v_fmac_f32_dpp %7, %7, " s " " ctl " row_mask:0xf bank_mask:0xf\n\t"

__device__ __forceinline__ float fwht128_x8(float (&v)[8], int lane) {
#pragma unroll
    for (int b = 1; b < 8; b <<= 1)
#pragma unroll
        for (int j = 0; j < 8; ++j)
            if (!(j & b)) {
                const float lo = v[j], hi = v[j | b];
                v[j] = lo + hi;
                v[j | b] = lo - hi;
            }
    const int g = h8_group(lane);
    const float s3 = g & 1 ? -1.f : 1.f, s4 = g & 2 ? -1.f : 1.f, s5 = g & 4 ? -1.f : 1.f, s6 = g & 8 ? -1.f : 1.f;
    asm volatile("s_nop 1\n\t" EA_FMAC_DPP8("quad_perm:[1,0,3,2]", "%8") EA_FMAC_DPP8("quad_perm:[2,3,0,1]", "%9")
                     EA_FMAC_DPP8("row_half_mirror", "%10") EA_FMAC_DPP8("row_ror:8", "%11") "s_nop 1"
                 : "+v"(v[0]), "+v"(v[1]), "+v"(v[2]), "+v"(v[3]), "+v"(v[4]), "+v"(v[5]), "+v"(v[6]), "+v"(v[7])
                 : "v"(s3), "v"(s4), "v"(s5), "v"(s6));
    return __builtin_popcount((unsigned)g) & 1 ? -1.f : 1.f;
}
#undef EA_FMAC_DPP8

// 32-lane half-wave variant: lane j (0..31 within its half) holds values 4j .. 4j + 3.
__device__ __forceinline__ void fwht128_h32(float (&v)[4], int lane) {
    const float a = v[0] + v[1], b = v[0] - v[1], c = v[2] + v[3], d = v[2] - v[3];
    v[0] = a + c;
    v[1] = b + d;
    v[2] = a - c;
    v[3] = b - d;
#pragma unroll
    for (int m = 1; m < 32; m <<= 1) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const float o = __shfl_xor(v[j], m, 32);
            v[j] = (lane & m) ? o - v[j] : v[j] + o;
        }
    }
}

}  // namespace ea
