/* CPU oracle for the EXL3 routed-expert path: TEST INFRASTRUCTURE ONLY (see exl3_oracle.h).
 *
 * Every function restates the arithmetic of the reference (fiore-labo/ExpertAtlas-GLM5.3) at the file:line
 * cited beside it, in plain C, one value at a time (matrix products decode each matrix once through a per-codebook
 * table built from or_cb_value).
 * Build: oracle/Makefile (gcc -O2 -ffp-contract=off: no product is fused unless the reference fuses it).
 *
 * Pinning (what checks each part; tests/test_oracle_*.py):
 *   bitstream      three independent formulations agree on random tiles for every K2 in 2..16
 *   codebooks      exhaustive over all 65,536 states against a second (integer-only) formulation; mcg halves
 *                  lie in +-[2^-3, 2); mul1 against exact rational arithmetic
 *   placement      bijection on 16x16, equal to the reference's dequant (g, t, q) indexing
 *   fwht           equal to H.v with H[i][j] = (-1)^popcount(i & j) in fp64 (tolerance) and H.H = 128 I
 *   group / route  integer brute force and invariants
 *   layer math     the dense fp64 identity out = sum_k wts * svh_d * (H/sqrt128) W_d^T ... (tolerance)
 *   topk           exact brute-force sort with the documented tie rule
 */
#include "exl3_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

const float OR_HAD_SCALE = 0.08838834764831845f; /* 1 / sqrt(128) as fp32 (decode.cuh:163) */

/* ------------------------------------------------------------------------------------------------ */
/* number formats                                                                                   */
/* ------------------------------------------------------------------------------------------------ */

float or_h2f(uint16_t h) {
    const int s = h >> 15, e = (h >> 10) & 31, m = h & 1023;
    float v;
    if (e == 0) v = ldexpf((float)m, -24);
    else if (e == 31) v = m ? NAN : INFINITY;
    else v = ldexpf((float)(m | 1024), e - 25);
    return s ? -v : v;
}

/* One rounding from an exact double to fp16, ties to even. */
uint16_t or_d2h(double d) {
    uint16_t sign = 0;
    if (isnan(d)) return 0x7e00;
    if (signbit(d)) { sign = 0x8000; d = -d; }
    if (d == 0.0) return sign;
    int e;
    frexp(d, &e); /* d = f * 2^e, f in [0.5, 1) */
    /* quantum: 2^(e - 11) for normals (11 significant bits), 2^-24 below 2^-14 */
    int qe = e - 11;
    if (qe < -24) qe = -24;
    double q = nearbyint(ldexp(d, -qe)); /* round half to even in the default mode */
    double r = ldexp(q, qe);
    if (r >= 65520.0 || r > 65504.0) return sign | 0x7c00;
    if (r < ldexp(1.0, -14)) return sign | (uint16_t)(uint32_t)ldexp(r, 24); /* subnormal */
    int re;
    double f = frexp(r, &re);                       /* r = f * 2^re */
    uint32_t mant = (uint32_t)ldexp(f, 11) - 1024;  /* 10 stored bits */
    return sign | (uint16_t)(((re - 1 + 15) << 10) | mant);
}

uint16_t or_f2h(float f) { return or_d2h((double)f); }

float or_bf2f(uint16_t b) {
    uint32_t u = (uint32_t)b << 16;
    float f;
    memcpy(&f, &u, 4);
    return f;
}

uint16_t or_f2bf(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40);
    u += 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

/* exp for the sigmoid and SwiGLU of this path: Cody & Waite reduction x = n ln2 + r (|r| <= ln2/2), a
 * degree-7 Taylor polynomial in r by Horner with fma, then 2^n by exponent scaling. Only IEEE fma, add,
 * multiply and ldexp, so the HIP build computes the same bits. */
float or_expf(float x) {
    if (x != x) return x;
    if (x > 88.72283935546875f) return INFINITY;
    if (x < -103.972084045410156f) return 0.0f;
    const float n = nearbyintf(x * 1.44269502162933349609f);
    float r = fmaf(-n, 0.693145751953125f, x);          /* ln2 high part (15 significant bits) */
    r = fmaf(-n, 1.42860682030941723212e-06f, r);       /* ln2 - high part */
    float p = 1.98412698412698412e-04f;                 /* 1/7! */
    p = fmaf(p, r, 1.38888888888888889e-03f);           /* 1/6! */
    p = fmaf(p, r, 8.33333333333333333e-03f);           /* 1/5! */
    p = fmaf(p, r, 4.16666666666666667e-02f);           /* 1/4! */
    p = fmaf(p, r, 1.66666666666666667e-01f);           /* 1/3! */
    p = fmaf(p, r, 0.5f);
    p = fmaf(p, r, 1.0f);
    p = fmaf(p, r, 1.0f);
    const int ni = (int)n;
    if (ni < -125) return ldexpf(ldexpf(p, ni + 64), -64);
    return ldexpf(p, ni);
}

/* ------------------------------------------------------------------------------------------------ */
/* trellis bitstream: decode.cuh:16-84, experts_grouped.cuh:55-85                                   */
/* ------------------------------------------------------------------------------------------------ */

int or_tile_words(int k2) { return 4 * k2; } /* decode.cuh:16-19 */

/* decode.cuh:22-25: E(p), one past the last stream bit of value p's 16-bit window. */
int or_stream_end(int k2, int p) {
    return (k2 & 1) ? ((p + 1) * k2 - ((p + 1) & 1)) / 2 : (p + 1) * (k2 / 2);
}

/* The stream is big-endian and circular: 32-bit word w holds stream bits [32w, 32w + 32), stream bit 32w is
 * the word's bit 31. Value p's state is the 16 bits [E(p) - 16, E(p)) modulo the tile's 128 * K2 bits, the
 * first bit most significant (decode.cuh:65-84 reads the same bits through funnel shifts). */
static int stream_bit(const uint32_t* tile, int k2, int q) {
    const int nbits = 128 * k2;
    q %= nbits;
    if (q < 0) q += nbits;
    return (tile[q >> 5] >> (31 - (q & 31))) & 1;
}

uint32_t or_state(const uint32_t* tile, int k2, int p) {
    const int e = or_stream_end(k2, p);
    uint32_t s = 0;
    for (int q = e - 16; q < e; ++q) s = (s << 1) | (uint32_t)stream_bit(tile, k2, q);
    return s;
}

void or_tile_states(const uint32_t* tile, int k2, uint16_t* states) {
    for (int p = 0; p < 256; ++p) states[p] = (uint16_t)or_state(tile, k2, p);
}

/* ------------------------------------------------------------------------------------------------ */
/* codebooks: decode.cuh:86-120, experts_grouped.cuh:27-53                                          */
/* ------------------------------------------------------------------------------------------------ */

static uint16_t half_of(uint32_t x) { /* (x & 0x8fff) ^ 0x3b60 on one 16-bit half */
    return (uint16_t)((x & 0x8fffu) ^ 0x3b60u);
}

uint16_t or_cb_value(int cb, uint32_t s) {
    s &= 0xffffu;
    if (cb == 2) {
        /* mul1: x = s * 0x83DCD12D; h = fp16 bits 0x6400 + (sum of x's four bytes) = 1024 + sum;
         * v = fma(h, fp16 0x1eee, fp16 0xc931) in fp16, one rounding (decode.cuh:89-96). */
        const uint32_t x = s * 0x83DCD12Du;
        const uint32_t sum = (x & 255u) + ((x >> 8) & 255u) + ((x >> 16) & 255u) + (x >> 24);
        const uint16_t h = (uint16_t)(0x6400u + sum);
        const double exact = (double)or_h2f(h) * (double)or_h2f(0x1eee) + (double)or_h2f(0xc931);
        return or_d2h(exact); /* the product (22 bits) and the sum are exact in double */
    }
    /* mcg (cb 1): x = s * 0xCBAC1FED; 3inst (cb 0): x = s * 89226354 + 64248484. Then each 16-bit half of
     * (x & 0x8FFF8FFF) ^ 0x3B603B60 is an fp16; the value is their fp16 sum (decode.cuh:98-111). Both halves
     * are normal numbers in +-[2^-3, 2), so their fp32 sum is exact and one fp16 rounding follows. */
    const uint32_t x = (cb == 1) ? s * 0xCBAC1FEDu : s * 89226354u + 64248484u;
    const float a = or_h2f(half_of(x)), b = or_h2f(half_of(x >> 16));
    return or_f2h(a + b);
}

void or_codebook_lut(int cb, uint16_t* lut) {
    for (uint32_t s = 0; s < 65536u; ++s) lut[s] = or_cb_value(cb, s);
}

/* ------------------------------------------------------------------------------------------------ */
/* placement: decode.cuh:134-136 (value p = 8 lane + j)                                             */
/* ------------------------------------------------------------------------------------------------ */

int or_value_row(int p) {
    const int lane = p >> 3, j = p & 7;
    return 2 * (lane & 3) + (j & 1) + 8 * ((j >> 1) & 1);
}

int or_value_col(int p) {
    const int lane = p >> 3, j = p & 7;
    return (lane >> 2) + 8 * (j >> 2);
}

void or_decode_tile(const uint32_t* tile, int k2, int cb, uint16_t* w) {
    for (int p = 0; p < 256; ++p) w[or_value_row(p) * 16 + or_value_col(p)] = or_cb_value(cb, or_state(tile, k2, p));
}

/* The same values through a per-codebook table (built once from or_cb_value) and a word-level window read;
 * used by the matrix products below, where or_decode_tile's bit-by-bit reads would be slow. */
static uint16_t* lut_of(int cb) {
    static uint16_t* luts[3];
    if (!luts[cb]) {
        uint16_t* l = (uint16_t*)malloc(65536 * 2);
        or_codebook_lut(cb, l);
        luts[cb] = l;
    }
    return luts[cb];
}

static void decode_tile_f32(const uint32_t* tile, int k2, int cb, float* w) {
    const uint16_t* lut = lut_of(cb);
    const int nbits = 128 * k2, TW = 4 * k2;
    for (int p = 0; p < 256; ++p) {
        int b = or_stream_end(k2, p) - 16;
        if (b < 0) b += nbits;
        const uint64_t hi = tile[(b >> 5) % TW], lo = tile[((b >> 5) + 1) % TW];
        const uint32_t s = (uint32_t)((((hi << 32) | lo) >> (48 - (b & 31))) & 0xffffu);
        w[or_value_row(p) * 16 + or_value_col(p)] = or_h2f(lut[s]);
    }
}

/* experts_grouped.cuh:317-336: tile (kt, nt) at ((kt * N/16) + nt) * TW words. */
void or_dequant_expert(const uint32_t* T, int K, int N, int k2, int cb, uint16_t* W) {
    const int TW = 4 * k2, NT = N / 16;
    uint16_t w[256];
    for (int kt = 0; kt < K / 16; ++kt)
        for (int nt = 0; nt < NT; ++nt) {
            or_decode_tile(T + ((size_t)kt * NT + nt) * TW, k2, cb, w);
            for (int r = 0; r < 16; ++r)
                for (int c = 0; c < 16; ++c) W[(size_t)(kt * 16 + r) * N + nt * 16 + c] = w[r * 16 + c];
        }
}

/* exl3_linear.cu:489-503: tile (kt, nt) at kt * stride_k + (nt / 8) * stride_nb + (nt % 8) * TW. */
void or_unpack(const uint32_t* T, int K, int N, int k2, int cb, int64_t stride_k, int64_t stride_nb, uint16_t* W) {
    const int TW = 4 * k2;
    uint16_t w[256];
    for (int kt = 0; kt < K / 16; ++kt)
        for (int nt = 0; nt < N / 16; ++nt) {
            or_decode_tile(T + kt * stride_k + (nt / 8) * stride_nb + (nt % 8) * TW, k2, cb, w);
            for (int r = 0; r < 16; ++r)
                for (int c = 0; c < 16; ++c) W[(size_t)(kt * 16 + r) * N + nt * 16 + c] = w[r * 16 + c];
        }
}

/* linear.zig:99-107 (load): [K/16, N/16, TW] viewed [kt, nt/8, 8, TW] -> [nt/8, kt, 8, TW]. */
void or_expert_to_strips(const uint32_t* T, int K, int N, int k2, uint32_t* S) {
    const int TW = 4 * k2, KT = K / 16, NT = N / 16;
    for (int b = 0; b < NT / 8; ++b)
        for (int i = 0; i < KT; ++i)
            memcpy(S + ((size_t)b * KT + i) * 8 * TW, T + ((size_t)i * NT + b * 8) * TW, (size_t)8 * TW * 4);
}

/* ------------------------------------------------------------------------------------------------ */
/* Hadamard: decode.cuh:146-163                                                                     */
/* ------------------------------------------------------------------------------------------------ */

/* The reference butterflies: levels over index bits 0, 1 (in registers), then 2..6 (across lanes), each
 * pair becoming (lower + upper, lower - upper) in fp32. */
void or_fwht128(float* v) {
    for (int h = 1; h < 128; h <<= 1)
        for (int i = 0; i < 128; ++i)
            if (!(i & h)) {
                const float a = v[i], b = v[i + h];
                v[i] = a + b;
                v[i + h] = a - b;
            }
}

/* ------------------------------------------------------------------------------------------------ */
/* routed experts, decode path                                                                      */
/* ------------------------------------------------------------------------------------------------ */

static float load_x(const void* x, int dt, size_t i) {
    if (dt == 2) return ((const float*)x)[i];
    if (dt == 1) return or_bf2f(((const uint16_t*)x)[i]);
    return or_h2f(((const uint16_t*)x)[i]);
}

/* exl3_experts.cu:36-90: distinct experts < E in id order; members[u][m] = row * 32 + slot in row order
 * (at most maxm), -1 after the last; ucount = the number of distinct experts. */
void or_group(const int* pick, int R, int slots, int E, int maxm, int* uids, int* ucount, int* members) {
    const int n = R * slots;
    int place = 0;
    for (int e = 0; e < E; ++e) {
        int c = 0;
        for (int i = 0; i < n; ++i) c += pick[i] == e;
        if (!c) continue;
        uids[place] = e;
        int j = 0;
        for (int i = 0; i < n && j < maxm; ++i)
            if (pick[i] == e) members[place * maxm + j++] = (i / slots) * 32 + (i % slots);
        for (; j < maxm; ++j) members[place * maxm + j] = -1;
        ++place;
    }
    *ucount = place;
}

/* exl3_experts.cu:116-134: out{0,1}[p] = fp16((x[row] * suh{0,1}[e]) @ H * HAD_SCALE) for every routed slot. */
void or_rot_in(const void* x, int x_dtype, int x_stride, const int* pick, const uint16_t* suh0, const uint16_t* suh1,
               uint16_t* out0, uint16_t* out1, int rows, int K, int slots, int E) {
    float v[128];
    for (int p = 0; p < rows * slots; ++p) {
        const int e = pick[p], row = p / slots;
        if (e < 0 || e >= E) continue;
        for (int mat = 0; mat < 2; ++mat) {
            const uint16_t* suh = (mat ? suh1 : suh0) + (size_t)e * K;
            uint16_t* o = (mat ? out1 : out0) + (size_t)p * K;
            for (int blk = 0; blk < K / 128; ++blk) {
                for (int j = 0; j < 128; ++j)
                    v[j] = load_x(x, x_dtype, (size_t)row * x_stride + blk * 128 + j) * or_h2f(suh[blk * 128 + j]);
                or_fwht128(v);
                for (int j = 0; j < 128; ++j) o[blk * 128 + j] = or_f2h(v[j] * OR_HAD_SCALE);
            }
        }
    }
}

/* W_q [K, N] fp32 of an expert-layout matrix whose trellis rows are ns tiles apart. */
static float* dequant_f32(const uint32_t* T, int ns, int K, int N, int k2, int cb) {
    float* W = (float*)malloc(sizeof(float) * (size_t)K * N);
    (void)lut_of(cb); /* built before the threads start */
#pragma omp parallel for schedule(static)
    for (int kt = 0; kt < K / 16; ++kt) {
        float w[256];
        for (int nt = 0; nt < N / 16; ++nt) {
            decode_tile_f32(T + ((size_t)kt * ns + nt) * (4 * k2), k2, cb, w);
            for (int r = 0; r < 16; ++r)
                for (int c = 0; c < 16; ++c) W[(size_t)(kt * 16 + r) * N + nt * 16 + c] = w[r * 16 + c];
        }
    }
    return W;
}

/* experts_grouped.cuh:214-313: Z[mat][split][p][n] = sum over the split's k of x[p][k] * W_q[e][k][n]; within a
 * split each of `warps` consecutive k ranges is summed on its own (ascending k, fp32) and the warps are added in
 * order. Rows without an expert are left as they are. */
void or_grouped(const or_grouped_args* a) {
    const int KT = a->K >> 4, NS = a->ns > 0 ? a->ns : a->N >> 4;
    const int per_split = KT / a->SK, W = a->warps > 0 ? a->warps : 1, per_warp = per_split / W;
    const int N = a->N;
    for (int u = 0; u < *a->ucount && u < a->nexp_max; ++u) {
        const int e = a->uids[u];
        for (int mat = 0; mat < a->mats; ++mat) {
            const uint16_t* X = mat ? a->x1 : a->x0;
            float* Wq = dequant_f32(mat ? a->tp1[e] : a->tp0[e], NS, a->K, N, mat ? a->k2_1[e] : a->k2_0[e], a->cb);
            int nm = 0;
            while (nm < a->maxm && a->members[u * a->maxm + nm] >= 0) ++nm;
#pragma omp parallel for schedule(dynamic)
            for (int m = 0; m < nm; ++m) {
                const int code = a->members[u * a->maxm + m];
                const int r = (code >> 5) * a->slots + (code & 31);
                float* acc = (float*)malloc(sizeof(float) * (size_t)W * N);
                for (int split = 0; split < a->SK; ++split) {
                    memset(acc, 0, sizeof(float) * (size_t)W * N);
                    for (int w = 0; w < W; ++w) {
                        const int k0 = (split * per_split + w * per_warp) * 16;
                        float* aw = acc + (size_t)w * N;
                        for (int k = k0; k < k0 + per_warp * 16; ++k) {
                            const float xv = or_h2f(X[(size_t)r * a->K + k]);
                            const float* wr = Wq + (size_t)k * N;
                            for (int n = 0; n < N; ++n) aw[n] += xv * wr[n];
                        }
                    }
                    float* z = a->z + (((size_t)mat * a->SK + split) * a->P + r) * N;
                    for (int n = 0; n < N; ++n) {
                        float s = acc[n];
                        for (int w = 1; w < W; ++w) s += acc[(size_t)w * N + n];
                        z[n] = s;
                    }
                }
                free(acc);
            }
            free(Wq);
        }
    }
}

/* exl3_experts.cu:142-184 */
void or_gateup_epilogue(const float* Z, const int* pick, const uint16_t* svh_g, const uint16_t* svh_u,
                        const uint16_t* suh_d, uint16_t* xd, int rows, int P, int N, int SK, int slots, int E,
                        float limit, int act_mode) {
    float gv[128], uv[128], v[128];
    for (int p = 0; p < rows * slots; ++p) {
        const int e = pick[p];
        if (e < 0 || e >= E) continue;
        for (int blk = 0; blk < N / 128; ++blk) {
            for (int j = 0; j < 128; ++j) {
                const int n = blk * 128 + j;
                float sg = 0.f, su = 0.f;
                for (int s = 0; s < SK; ++s) {
                    sg += Z[((size_t)(0 * SK + s) * P + p) * N + n];
                    su += Z[((size_t)(1 * SK + s) * P + p) * N + n];
                }
                gv[j] = sg;
                uv[j] = su;
            }
            or_fwht128(gv);
            or_fwht128(uv);
            for (int j = 0; j < 128; ++j) {
                const size_t at = (size_t)e * N + blk * 128 + j;
                float act;
                if (act_mode == 0) {
                    const float gg = fminf(or_bf2f(or_f2bf(gv[j] * OR_HAD_SCALE * or_h2f(svh_g[at]))), limit);
                    const float uu = fminf(fmaxf(or_bf2f(or_f2bf(uv[j] * OR_HAD_SCALE * or_h2f(svh_u[at]))), -limit), limit);
                    act = or_bf2f(or_f2bf(or_bf2f(or_f2bf(gg / (1.f + or_expf(-gg)))) * uu));
                } else {
                    const float gg = fminf(gv[j] * OR_HAD_SCALE * or_h2f(svh_g[at]), limit);
                    const float uu = fminf(fmaxf(uv[j] * OR_HAD_SCALE * or_h2f(svh_u[at]), -limit), limit);
                    act = gg / (1.f + or_expf(-gg)) * uu;
                }
                v[j] = act * or_h2f(suh_d[at]);
            }
            or_fwht128(v);
            for (int j = 0; j < 128; ++j) xd[(size_t)p * N + blk * 128 + j] = or_f2h(v[j] * OR_HAD_SCALE);
        }
    }
}

/* exl3_experts.cu:223-268 */
void or_down_combine(const float* Z, const int* pick, const uint16_t* svh_d, float* y, const float* wts, float* out,
                     int rows, int P, int D, int SK, int slots, int E) {
    float v[128];
    for (int r = 0; r < rows; ++r) {
        for (int k = 0; k < slots; ++k) {
            const int p = r * slots + k, e = pick[p];
            if (e < 0 || e >= E) continue;
            for (int blk = 0; blk < D / 128; ++blk) {
                for (int j = 0; j < 128; ++j) {
                    float s = 0.f;
                    for (int q = 0; q < SK; ++q) s += Z[((size_t)q * P + p) * D + blk * 128 + j];
                    v[j] = s;
                }
                or_fwht128(v);
                for (int j = 0; j < 128; ++j)
                    y[(size_t)p * D + blk * 128 + j] = v[j] * OR_HAD_SCALE * or_h2f(svh_d[(size_t)e * D + blk * 128 + j]);
            }
        }
        for (int d = 0; d < D; ++d) {
            float acc = 0.f;
            for (int k = 0; k < slots; ++k) acc = fmaf(wts[r * slots + k], y[((size_t)r * slots + k) * D + d], acc);
            out[(size_t)r * D + d] = acc;
        }
    }
}

/* moe.zig:279-293 with the tile settings of moe.zig:16-17 (gate/up SK 4, down SK 1, 4 warps). */
void or_moe_routed(const void* x, int x_dtype, int x_stride, const int* pick, const float* wts, const or_routed* ex,
                   int R, int slots, float* y, float* out) {
    const int D = ex->dims, I = ex->width, E = ex->count, P = R * slots;
    const int maxu = P < E ? P : E;
    int* uids = (int*)malloc(sizeof(int) * (size_t)maxu);
    int* members = (int*)malloc(sizeof(int) * (size_t)maxu * R);
    int ucount = 0;
    uint16_t* xg = (uint16_t*)calloc((size_t)P * D, 2);
    uint16_t* xu = (uint16_t*)calloc((size_t)P * D, 2);
    uint16_t* xd = (uint16_t*)calloc((size_t)P * I, 2);
    const size_t zn = (size_t)(2 * 4 * I > D ? 2 * 4 * I : D) * P;
    float* z = (float*)calloc(zn, 4);
    or_group(pick, R, slots, E, R, uids, &ucount, members);
    or_rot_in(x, x_dtype, x_stride, pick, ex->suh_g, ex->suh_u, xg, xu, R, D, slots, E);
    or_grouped_args g = {xg, xu, ex->ptr[0], ex->ptr[1], ex->k2[0], ex->k2[1], uids, &ucount, members, z,
                         D, I, P, 4, R, slots, maxu, 2, ex->cb, 4, 0};
    or_grouped(&g);
    or_gateup_epilogue(z, pick, ex->svh_g, ex->svh_u, ex->suh_d, xd, R, P, I, 4, slots, E, INFINITY, 1);
    or_grouped_args d = {xd, xd, ex->ptr[2], ex->ptr[2], ex->k2[2], ex->k2[2], uids, &ucount, members, z,
                         I, D, P, 1, R, slots, maxu, 1, ex->cb, 4, 0};
    or_grouped(&d);
    or_down_combine(z, pick, ex->svh_d, y, wts, out, R, P, D, 1, slots, E);
    free(uids); free(members); free(xg); free(xu); free(xd); free(z);
}

/* ------------------------------------------------------------------------------------------------ */
/* prefill path                                                                                     */
/* ------------------------------------------------------------------------------------------------ */

/* prompt_experts.cu:162-244 with by_count off: per-expert counts, items (e, first, cnt <= ipm) in expert order,
 * sorted[] = pair ids grouped by expert. The reference orders an expert's pairs by atomic arrival; this
 * restatement uses ascending pair id, one of the orders the reference can produce. */
int or_route(const int* pick, int n, int E, int ipm, int max_items, int* sorted, int* items, int* item_count) {
    int* cnt = (int*)calloc((size_t)E, sizeof(int));
    for (int i = 0; i < n; ++i)
        if (pick[i] >= 0 && pick[i] < E) cnt[pick[i]]++;
    int off = 0, it = 0, total_items = 0;
    for (int e = 0; e < E; ++e) total_items += (cnt[e] + ipm - 1) / ipm;
    for (int e = 0; e < E; ++e) {
        for (int f = 0; f < cnt[e]; f += ipm, ++it)
            if (it < max_items) {
                items[3 * it] = e;
                items[3 * it + 1] = off + f;
                items[3 * it + 2] = cnt[e] - f < ipm ? cnt[e] - f : ipm;
            }
        int w = off;
        for (int i = 0; i < n; ++i)
            if (pick[i] == e) sorted[w++] = i;
        off += cnt[e];
    }
    *item_count = total_items < max_items ? total_items : max_items;
    free(cnt);
    return off;
}

/* prompt_experts.cu / prompt_experts.zig:146-248: the same function of x as the decode path (gate | up with the
 * input rotation, SwiGLU in fp32, the down input's rotation, down, FWHT, svh_d), each pair's result times its
 * routing weight summed into out [R, D]. The reference adds the pairs with atomics (an unspecified order); this
 * restatement adds them in slot order. */
void or_prompt_experts(const void* x, int x_dtype, int x_stride, const int* pick, const float* wts,
                       const or_routed* ex, int R, int slots, int do_round, float* out) {
    const int D = ex->dims;
    const int P = R * slots;
    float* y = (float*)calloc((size_t)P * D, 4);
    float* part = (float*)calloc((size_t)R * D, 4);
    /* per-pair y through the decode path's kernels with unit weights, then the weighted slot-order sum */
    float* ones = (float*)malloc(sizeof(float) * (size_t)P);
    for (int i = 0; i < P; ++i) ones[i] = 1.f;
    or_moe_routed(x, x_dtype, x_stride, pick, ones, ex, R, slots, y, part);
    for (int r = 0; r < R; ++r)
        for (int d = 0; d < D; ++d) {
            float acc = 0.f;
            for (int k = 0; k < slots; ++k) {
                const int p = r * slots + k;
                if (pick[p] < 0 || pick[p] >= ex->count) continue;
                acc += y[(size_t)p * D + d] * wts[p];
            }
            out[(size_t)r * D + d] = do_round ? or_bf2f(or_f2bf(acc)) : acc;
        }
    free(y); free(part); free(ones);
}

/* ------------------------------------------------------------------------------------------------ */
/* EXL3 linear                                                                                      */
/* ------------------------------------------------------------------------------------------------ */

/* linear.zig:61-79 plan */
void or_linear_plan(int k, int n, int* sk_out, int* wk_out) {
    const int kt = k / 16, nb = n / 128;
    int sk = 1, wk = nb >= 64 ? 8 : 4;
    if (nb < 64)
        while (nb * sk < 192 && sk < 64) sk *= 2;
    while ((wk > 4 || sk > 1) && (kt % (sk * wk) != 0 || kt / (sk * wk) < 8)) {
        if (wk > 4) wk = 4;
        else if (sk > 1) sk /= 2;
        else break;
    }
    *sk_out = sk;
    *wk_out = wk;
}

/* exl3_linear.cu:152-173 */
void or_exl3_rot_in(const void* x, int x_dtype, const uint16_t* suh, uint16_t* xh, int M, int K) {
    float v[128];
    for (int r = 0; r < M; ++r)
        for (int blk = 0; blk < K / 128; ++blk) {
            for (int j = 0; j < 128; ++j) v[j] = load_x(x, x_dtype, (size_t)r * K + blk * 128 + j) * or_h2f(suh[blk * 128 + j]);
            or_fwht128(v);
            for (int j = 0; j < 128; ++j) xh[(size_t)r * K + blk * 128 + j] = or_f2h(v[j] * OR_HAD_SCALE);
        }
}

static void store_y(void* y, int dt, size_t i, float v) {
    if (dt == 2) ((float*)y)[i] = v;
    else if (dt == 1) ((uint16_t*)y)[i] = or_f2bf(v);
    else ((uint16_t*)y)[i] = or_f2h(v);
}

/* exl3_linear.cu:231-484: per column block of 128, split s's warps w sum their k tiles in ascending order (fp32),
 * warps added in order, splits added in order; then FWHT, * HAD_SCALE * svh (+ bias) (finish, :69-81). */
void or_exl3_linear(const uint16_t* xh, const uint32_t* T, int64_t stride_k, int64_t stride_nb, const uint16_t* svh,
                    const uint16_t* bias, void* y, int y_dtype, int M, int K, int N, int k2, int cb, int SK, int WK) {
    const int KT = K / 16, per_warp = KT / SK / WK, TW = 4 * k2;
    float* W = (float*)malloc(sizeof(float) * (size_t)K * N);
    (void)lut_of(cb);
#pragma omp parallel for schedule(static)
    for (int kt = 0; kt < KT; ++kt) {
        float w[256];
        for (int nt = 0; nt < N / 16; ++nt) {
            decode_tile_f32(T + kt * stride_k + (nt / 8) * stride_nb + (nt % 8) * TW, k2, cb, w);
            for (int r = 0; r < 16; ++r)
                for (int c = 0; c < 16; ++c) W[(size_t)(kt * 16 + r) * N + nt * 16 + c] = w[r * 16 + c];
        }
    }
#pragma omp parallel for schedule(dynamic)
    for (int r = 0; r < M; ++r) {
        float* acc = (float*)malloc(sizeof(float) * (size_t)SK * WK * N);
        float v[128];
        memset(acc, 0, sizeof(float) * (size_t)SK * WK * N);
        for (int s = 0; s < SK; ++s)
            for (int wk = 0; wk < WK; ++wk) {
                float* a = acc + ((size_t)s * WK + wk) * N;
                const int k0 = (s * per_warp * WK + wk * per_warp) * 16;
                for (int k = k0; k < k0 + per_warp * 16; ++k) {
                    const float xv = or_h2f(xh[(size_t)r * K + k]);
                    const float* wr = W + (size_t)k * N;
                    for (int n = 0; n < N; ++n) a[n] += xv * wr[n];
                }
            }
        for (int nb = 0; nb < N / 128; ++nb) {
            for (int c = 0; c < 128; ++c) {
                const int n = nb * 128 + c;
                float tot = 0.f;
                for (int s = 0; s < SK; ++s) {
                    float ws = acc[((size_t)s * WK) * N + n];
                    for (int wk = 1; wk < WK; ++wk) ws += acc[((size_t)s * WK + wk) * N + n];
                    tot = s ? tot + ws : ws;
                }
                v[c] = tot;
            }
            or_fwht128(v);
            for (int c = 0; c < 128; ++c) {
                float o = v[c] * OR_HAD_SCALE * or_h2f(svh[nb * 128 + c]);
                if (bias) o += or_h2f(bias[nb * 128 + c]);
                store_y(y, y_dtype, (size_t)r * N + nb * 128 + c, o);
            }
        }
        free(acc);
    }
    free(W);
}

/* ------------------------------------------------------------------------------------------------ */
/* router top-8: native_ops.cu:998-1068                                                             */
/* ------------------------------------------------------------------------------------------------ */

/* The top-8's ranking key of a choice: order-preserving over numbers (+0 and -0 share one), NaN just above 0, the key
 * of a taken expert. So a NaN choice ranks below every number, -inf included, and NaNs among themselves by id; a
 * taken expert is never picked again. (The reference compares floats in a lane-order butterfly, where a NaN's fate
 * depends on its lane: native_ops.cu:1021-1027; this build fixes one rule for its two top-8 paths.) */
static uint32_t or_order_key(float f) {
    if (f != f) return 1u;
    const float g = f + 0.0f;
    uint32_t b;
    memcpy(&b, &g, 4);
    return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}

/* native_ops.cu:1015-1068: choice = sigmoid(l) + bias; 8 rounds of the largest key, the lower id on a tie;
 * wts = sigmoid / (sum of the picks' sigmoids in pick order + 1e-20) * scale. */
void or_topk8(const float* logits, const float* bias, int rows, int E, float scale, int* pick, float* wts) {
    float* score = (float*)malloc(sizeof(float) * (size_t)E);
    uint32_t* key = (uint32_t*)malloc(sizeof(uint32_t) * (size_t)E);
    for (int r = 0; r < rows; ++r) {
        for (int e = 0; e < E; ++e) {
            score[e] = 1.0f / (or_expf(0.0f - logits[(size_t)r * E + e]) + 1.0f);
            key[e] = or_order_key(score[e] + bias[e]);
        }
        float sw[8];
        int sp[8];
        for (int k = 0; k < 8; ++k) {
            int bi = 0;
            for (int e = 1; e < E; ++e)
                if (key[e] > key[bi]) bi = e;
            sp[k] = bi;
            sw[k] = score[bi];
            key[bi] = 0u;
        }
        float total = 0.f;
        for (int k = 0; k < 8; ++k) total = total + sw[k];
        for (int k = 0; k < 8; ++k) {
            pick[(size_t)r * 8 + k] = sp[k];
            wts[(size_t)r * 8 + k] = sw[k] / (total + 1e-20f) * scale;
        }
    }
    free(score);
    free(key);
}

/* ops.zig:131-136 (router_part native_ops.cu:1405-1460, router_sum :335-362): out [m, ne] = x [m, d] @ w^T, the
 * reduction in eight slices of kw = d / 8 added in slice order (part [8, m, ne] holds the slice sums when given).
 * Inside a slice, the order of this build's kernel (the reference's is inside tensor-core MMAs): 64 lane sums, lane l
 * taking the 4-value chunks c = l, l + 64, .. (c < kw / 4) in order by fp32 fma, then a butterfly: at distance
 * 32, 16, 8, 4, 2, 1 each lane sum becomes itself + the sum of lane (l ^ distance). x_dtype 0 fp16, 1 bf16. */
void or_router(const uint16_t* x, int x_dtype, int x_stride, const uint16_t* w, int m, int d, int ne, float* part,
               float* out) {
    const int kw = d / 8, nc = kw / 4;
#pragma omp parallel for schedule(static)
    for (int r = 0; r < m; ++r) {
        for (int e = 0; e < ne; ++e) {
            float tot = 0.f;
            for (int s = 0; s < 8; ++s) {
                float lane[64], nxt[64];
                for (int l = 0; l < 64; ++l) lane[l] = 0.f;
                for (int c = 0; c < nc; ++c) {
                    const size_t k = (size_t)s * kw + 4 * (size_t)c;
                    for (int i = 0; i < 4; ++i) {
                        const uint16_t xv = x[(size_t)r * x_stride + k + i];
                        const float xf = x_dtype == 1 ? or_bf2f(xv) : or_h2f(xv);
                        lane[c % 64] = fmaf(xf, or_bf2f(w[(size_t)e * d + k + i]), lane[c % 64]);
                    }
                }
                for (int dist = 32; dist >= 1; dist >>= 1) {
                    for (int l = 0; l < 64; ++l) nxt[l] = lane[l] + lane[l ^ dist];
                    memcpy(lane, nxt, sizeof(lane));
                }
                if (part) part[((size_t)s * m + r) * ne + e] = lane[0];
                tot = s ? tot + lane[0] : lane[0];
            }
            out[(size_t)r * ne + e] = tot;
        }
    }
}

/* native_ops.cu:429-441: out = bf16(bf16(silu(g)) * u), silu(g) = g / (exp(-g) + 1). */
void or_swiglu2(const uint16_t* g, const uint16_t* u, uint16_t* out, int n) {
    for (int i = 0; i < n; ++i) {
        const float gv = or_bf2f(g[i]);
        const float s = or_bf2f(or_f2bf(gv / (or_expf(0.0f - gv) + 1.0f)));
        out[i] = or_f2bf(s * or_bf2f(u[i]));
    }
}

/* ------------------------------------------------------------------------------------------------ */
/* deterministic data                                                                               */
/* ------------------------------------------------------------------------------------------------ */

/* SplitMix64's finaliser (Steele, Lea & Flood 2014). */
uint64_t or_mix64(uint64_t x) {
    x += 0x9E3779B97F4A7C15ull;
    x = (x ^ (x >> 30)) * 0xBF58476D1CE4E5B9ull;
    x = (x ^ (x >> 27)) * 0x94D049BB133111EBull;
    return x ^ (x >> 31);
}

/* word i = half (i & 1) of mix64(mix64(seed) + i / 2), the low half first */
void or_fill_words(uint64_t seed, uint32_t* w, size_t n) {
    const uint64_t base = or_mix64(seed);
    for (size_t i = 0; i < n; ++i) w[i] = (uint32_t)(or_mix64(base + (uint64_t)(i >> 1)) >> (32 * (i & 1)));
}
