/* The CPU baselines of the routed-expert decode layer and of one EXL3 linear: test infrastructure, timed by bench.py's
 * cpu_baseline leg and checked against the oracle by tests/test_cpu_layer.py. Never loaded by the product path.
 *
 * The same function as the oracle's moe.routed (moe.zig:279-293: rotate-in, gate / up GEMV, SwiGLU epilogue, down
 * GEMV, slot-ordered combine; exl3_experts.cu:116-268), organised for host cores: no matrix is dequantised into
 * memory; each task decodes its tiles (a 64-bit window read and a codebook table a value) straight into the sums of
 * every row that picked the expert, and OpenMP spreads every product over its column tiles (the gate / up of all
 * units at once, then the down of all units), so one row keeps every core busy. Sums run over k in ascending order in
 * fp32, so the results differ from the oracle's only by summation order (the oracle follows the kernels' K splits). */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#include "exl3_oracle.h"

static const float HS = 0.08838834764831845f; /* 1 / sqrt(128) */

/* value p's (row, col) in its tile and its window's first stream bit, per width (decode.cuh:21-25, 134-136) */
static int ROW[256], COL[256];
static int WSTART[17][256];
static float* LUTF[3];

static void tables(int cb) {
#pragma omp critical(cpu_layer_tables)
    {
        if (!LUTF[cb]) {
            for (int p = 0; p < 256; ++p) {
                ROW[p] = or_value_row(p);
                COL[p] = or_value_col(p);
                for (int k2 = 2; k2 <= 16; ++k2) {
                    int b = or_stream_end(k2, p) - 16;
                    if (b < 0) b += 128 * k2;
                    WSTART[k2][p] = b;
                }
            }
            float* l = (float*)malloc(sizeof(float) * 65536);
            for (uint32_t s = 0; s < 65536u; ++s) l[s] = or_h2f(or_cb_value(cb, s));
            LUTF[cb] = l;
        }
    }
}

/* w[16][16] fp32 of one tile */
static inline void decode(const uint32_t* tile, int k2, const float* lut, float* w) {
    const int TW = 4 * k2;
    const int* ws = WSTART[k2];
    for (int p = 0; p < 256; ++p) {
        const int b = ws[p], i = b >> 5;
        const uint64_t v = ((uint64_t)tile[i] << 32) | tile[i + 1 < TW ? i + 1 : 0];
        w[ROW[p] * 16 + COL[p]] = lut[(uint32_t)(v >> (48 - (b & 31))) & 0xffffu];
    }
}

static void fwht(float* v) {
    for (int h = 1; h < 128; h <<= 1)
        for (int i = 0; i < 128; i += 2 * h)
            for (int j = i; j < i + h; ++j) {
                const float a = v[j], b = v[j + h];
                v[j] = a + b;
                v[j + h] = a - b;
            }
}

/* out [R, D] = sum over slots of wts * expert(x row), x fp16 (x_dtype 0) or bf16 (1) [R, D]; the same arguments as
 * or_moe_routed. */
void cpu_moe_routed(const void* x, int x_dtype, int x_stride, const int* pick, const float* wts, const or_routed* ex,
                    int R, int slots, float* out) {
    const int D = ex->dims, I = ex->width, E = ex->count, P = R * slots, cb = ex->cb;
    tables(cb);
    const float* lut = LUTF[cb];
    const int KT = D / 16, NTI = I / 16, KTD = I / 16, NTD = D / 16;
    /* rotated inputs xh[mat][p][D] (fp16 values as float) */
    float* xh = (float*)malloc(sizeof(float) * 2 * (size_t)P * D);
    float* z = (float*)calloc((size_t)2 * P * I, sizeof(float));
    float* xd = (float*)malloc(sizeof(float) * (size_t)P * I);
    float* y = (float*)calloc((size_t)P * D, sizeof(float));
#pragma omp parallel for schedule(static)
    for (int t = 0; t < 2 * P * (D / 128); ++t) {
        const int mat = t / (P * (D / 128)), rem = t % (P * (D / 128)), p = rem / (D / 128), blk = rem % (D / 128);
        const int e = pick[p], r = p / slots;
        float* o = xh + ((size_t)mat * P + p) * D + blk * 128;
        if (e < 0 || e >= E) {
            memset(o, 0, 128 * sizeof(float));
            continue;
        }
        const uint16_t* suh = (mat ? ex->suh_u : ex->suh_g) + (size_t)e * D + blk * 128;
        float v[128];
        for (int j = 0; j < 128; ++j) {
            const uint16_t xv = ((const uint16_t*)x)[(size_t)r * x_stride + blk * 128 + j];
            v[j] = (x_dtype == 1 ? or_bf2f(xv) : or_h2f(xv)) * or_h2f(suh[j]);
        }
        fwht(v);
        for (int j = 0; j < 128; ++j) o[j] = or_h2f(or_f2h(v[j] * HS));
    }
    /* the distinct picked experts and their pairs (units), so each tile is decoded once for all of its rows */
    int* unit_e = (int*)malloc(sizeof(int) * (size_t)P);
    int* unit_first = (int*)malloc(sizeof(int) * ((size_t)P + 1));
    int* unit_pairs = (int*)malloc(sizeof(int) * (size_t)P);
    int U = 0, np = 0;
    for (int e = 0; e < E; ++e) {
        int first = np;
        for (int p = 0; p < P; ++p)
            if (pick[p] == e) unit_pairs[np++] = p;
        if (np > first) {
            unit_e[U] = e;
            unit_first[U++] = first;
        }
    }
    unit_first[U] = np;
    /* gate / up: a task a (matrix, unit, column tile); its k tiles in order, every member row at once */
#pragma omp parallel for schedule(dynamic, 4)
    for (int t = 0; t < 2 * U * NTI; ++t) {
        const int mat = t / (U * NTI), rem = t % (U * NTI), u = rem / NTI, nt = rem % NTI;
        const int e = unit_e[u], m0 = unit_first[u], nm = unit_first[u + 1] - m0;
        const int k2 = (mat ? ex->k2[1] : ex->k2[0])[e], TW = 4 * k2;
        const uint32_t* T = (mat ? ex->ptr[1] : ex->ptr[0])[e];
        float w[256];
        for (int m = 0; m < nm; ++m) memset(z + ((size_t)mat * P + unit_pairs[m0 + m]) * I + nt * 16, 0, 64);
        for (int kt = 0; kt < KT; ++kt) {
            decode(T + ((size_t)kt * NTI + nt) * TW, k2, lut, w);
            for (int m = 0; m < nm; ++m) {
                const int p = unit_pairs[m0 + m];
                const float* xr = xh + ((size_t)mat * P + p) * D + kt * 16;
                float* acc = z + ((size_t)mat * P + p) * I + nt * 16;
                for (int rr = 0; rr < 16; ++rr)
                    for (int c = 0; c < 16; ++c) acc[c] += xr[rr] * w[rr * 16 + c];
            }
        }
    }
    /* SwiGLU epilogue (act_mode 1, no limit) */
#pragma omp parallel for schedule(static)
    for (int t = 0; t < P * (I / 128); ++t) {
        const int p = t / (I / 128), blk = t % (I / 128), e = pick[p];
        if (e < 0 || e >= E) continue;
        float g[128], u[128], v[128];
        memcpy(g, z + (size_t)p * I + blk * 128, sizeof(g));
        memcpy(u, z + ((size_t)P + p) * I + blk * 128, sizeof(u));
        fwht(g);
        fwht(u);
        for (int j = 0; j < 128; ++j) {
            const size_t at = (size_t)e * I + blk * 128 + j;
            const float gg = g[j] * HS * or_h2f(ex->svh_g[at]), uu = u[j] * HS * or_h2f(ex->svh_u[at]);
            v[j] = gg / (1.f + expf(-gg)) * uu * or_h2f(ex->suh_d[at]);
        }
        fwht(v);
        for (int j = 0; j < 128; ++j) xd[(size_t)p * I + blk * 128 + j] = or_h2f(or_f2h(v[j] * HS));
    }
    /* down: a task a (unit, column tile), every member row at once */
#pragma omp parallel for schedule(dynamic, 8)
    for (int t = 0; t < U * NTD; ++t) {
        const int u = t / NTD, nt = t % NTD;
        const int e = unit_e[u], m0 = unit_first[u], nm = unit_first[u + 1] - m0;
        const int k2 = ex->k2[2][e], TW = 4 * k2;
        const uint32_t* T = ex->ptr[2][e];
        float w[256];
        for (int kt = 0; kt < KTD; ++kt) {
            decode(T + ((size_t)kt * NTD + nt) * TW, k2, lut, w);
            for (int m = 0; m < nm; ++m) {
                const int p = unit_pairs[m0 + m];
                const float* xr = xd + (size_t)p * I + kt * 16;
                float* acc = y + (size_t)p * D + nt * 16;
                for (int rr = 0; rr < 16; ++rr)
                    for (int c = 0; c < 16; ++c) acc[c] += xr[rr] * w[rr * 16 + c];
            }
        }
    }
    /* down rotation, svh_d, and the slot-ordered combine */
#pragma omp parallel for schedule(static)
    for (int t = 0; t < R * (D / 128); ++t) {
        const int r = t / (D / 128), blk = t % (D / 128);
        float acc[128] = {0}, v[128];
        for (int k = 0; k < slots; ++k) {
            const int p = r * slots + k, e = pick[p];
            if (e < 0 || e >= E) continue;
            memcpy(v, y + (size_t)p * D + blk * 128, sizeof(v));
            fwht(v);
            for (int j = 0; j < 128; ++j)
                acc[j] = fmaf(wts[p], v[j] * HS * or_h2f(ex->svh_d[(size_t)e * D + blk * 128 + j]), acc[j]);
        }
        memcpy(out + (size_t)r * D + blk * 128, acc, sizeof(acc));
    }
    free(unit_e);
    free(unit_first);
    free(unit_pairs);
    free(xh);
    free(z);
    free(xd);
    free(y);
}

/* One EXL3 linear, y [M, N] fp32 = FWHT(rot_in(x) . W) * HS * svh: the oracle's or_exl3_rot_in then or_exl3_linear
 * (exl3_linear.cu:150-173 rotation, :231-484 product, finish :69-81), with W in linear.zig's strips layout (tile
 * (kt, nt) at (nt / 8) stride_nb + kt stride_k + (nt % 8) TW words, linear.zig:99-107). For host cores: the rows are
 * rotated in parallel, then each task (a column tile) decodes its k tiles in ascending order straight into the sums of
 * every row, so one row keeps every core busy; then the output rotation a (row, column block). The sums run over k in
 * order in fp32, so the result differs from the oracle's only by summation order (the oracle follows the kernel's
 * K splits). */
void cpu_exl3_linear(const void* x, int x_dtype, const uint16_t* suh, const uint32_t* T, int64_t stride_k,
                     int64_t stride_nb, const uint16_t* svh, float* y, int M, int K, int N, int k2, int cb) {
    tables(cb);
    const float* lut = LUTF[cb];
    const int KT = K / 16, NT = N / 16, TW = 4 * k2;
    float* xh = (float*)malloc(sizeof(float) * (size_t)M * K);
    float* acc = (float*)calloc((size_t)M * N, sizeof(float));
#pragma omp parallel for schedule(static)
    for (int t = 0; t < M * (K / 128); ++t) {
        const int r = t / (K / 128), blk = t % (K / 128);
        float v[128];
        for (int j = 0; j < 128; ++j) {
            const uint16_t xv = ((const uint16_t*)x)[(size_t)r * K + blk * 128 + j];
            v[j] = (x_dtype == 1 ? or_bf2f(xv) : or_h2f(xv)) * or_h2f(suh[blk * 128 + j]);
        }
        fwht(v);
        for (int j = 0; j < 128; ++j) xh[(size_t)r * K + blk * 128 + j] = or_h2f(or_f2h(v[j] * HS));
    }
#pragma omp parallel for schedule(dynamic, 2)
    for (int nt = 0; nt < NT; ++nt) {
        float w[256];
        const uint32_t* strip = T + (size_t)(nt / 8) * stride_nb + (size_t)(nt % 8) * TW;
        for (int kt = 0; kt < KT; ++kt) {
            decode(strip + (size_t)kt * stride_k, k2, lut, w);
            for (int m = 0; m < M; ++m) {
                const float* xr = xh + (size_t)m * K + kt * 16;
                float* a = acc + (size_t)m * N + nt * 16;
                for (int rr = 0; rr < 16; ++rr)
                    for (int c = 0; c < 16; ++c) a[c] += xr[rr] * w[rr * 16 + c];
            }
        }
    }
#pragma omp parallel for schedule(static)
    for (int t = 0; t < M * (N / 128); ++t) {
        const int r = t / (N / 128), nb = t % (N / 128);
        float v[128];
        memcpy(v, acc + (size_t)r * N + nb * 128, sizeof(v));
        fwht(v);
        for (int c = 0; c < 128; ++c) y[(size_t)r * N + nb * 128 + c] = v[c] * HS * or_h2f(svh[nb * 128 + c]);
    }
    free(xh);
    free(acc);
}
