/* CPU oracle for the EXL3 routed-expert path: TEST INFRASTRUCTURE ONLY.
 *
 * A plain-C restatement of the reference kernels' arithmetic (fiore-labo/ExpertAtlas-GLM5.3,
 * zig/kernels/cuda/glm53/ (.cu and .cuh files) and the Zig launchers that fix their shapes). Only tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg may load it, and only as the checker or the
 * CPU baseline; the product path never links it.
 *
 * Numbers: fp16 / bf16 travel as uint16_t bit patterns; every rounding point of the reference is
 * reproduced explicitly (fp32 products, fp32 butterflies, round-to-nearest-even to fp16).
 * Matrix products over k are accumulated in fp32 in ascending k order inside each reference split;
 * the reference's tensor-core accumulation order is unspecified, so those results are compared with a
 * tolerance, never bit for bit.
 */
#ifndef EXL3_ORACLE_H
#define EXL3_ORACLE_H
#include <stdint.h>
#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- scalar number formats ---- */
float or_h2f(uint16_t h);
uint16_t or_f2h(float f);            /* round to nearest even, overflow to inf */
uint16_t or_d2h(double d);           /* round an exact double straight to fp16 (one rounding) */
float or_bf2f(uint16_t b);
uint16_t or_f2bf(float f);           /* round to nearest even */
float or_expf(float x);              /* the path's exp (Cody-Waite + Taylor, fma only) */

/* ---- trellis bitstream (decode.cuh:16-84) ---- */
int or_tile_words(int k2);                                /* 4 * K2 */
int or_stream_end(int k2, int p);                         /* E(p) */
uint32_t or_state(const uint32_t* tile, int k2, int p);   /* 16-bit state of value p (closed form) */
void or_tile_states(const uint32_t* tile, int k2, uint16_t* states);

/* ---- codebooks (decode.cuh:86-120) ---- */
uint16_t or_cb_value(int cb, uint32_t state);             /* fp16 bits; cb 0 3inst, 1 mcg, 2 mul1 */
void or_codebook_lut(int cb, uint16_t* lut);              /* 65536 entries */

/* ---- placement (decode.cuh:134-136) and dequantisation ---- */
int or_value_row(int p);                                  /* k within the tile of stream value p */
int or_value_col(int p);                                  /* n within the tile */
void or_decode_tile(const uint32_t* tile, int k2, int cb, uint16_t* w16x16);   /* [k][n] */
/* expert layout: tile (kt, nt) at ((kt * N/16) + nt) * TW words (experts_grouped.cuh:317-336) */
void or_dequant_expert(const uint32_t* T, int K, int N, int k2, int cb, uint16_t* W);
/* strided layout: tile (kt, nt) at kt*stride_k + (nt/8)*stride_nb + (nt%8)*TW (exl3_linear.cu:489-503) */
void or_unpack(const uint32_t* T, int K, int N, int k2, int cb, int64_t stride_k, int64_t stride_nb,
               uint16_t* W);
/* expert layout -> "strips" [N/128][K/16][8][TW] (linear.zig:99-107) */
void or_expert_to_strips(const uint32_t* T, int K, int N, int k2, uint32_t* S);

/* ---- Hadamard (decode.cuh:146-163) ---- */
void or_fwht128(float* v);                                /* unscaled, the reference butterfly order */
extern const float OR_HAD_SCALE;

/* ---- routed experts, decode path (exl3_experts.cu, experts.zig, moe.zig) ---- */
/* x_dtype: 0 fp16, 1 bf16, 2 fp32 */
void or_group(const int* pick, int R, int slots, int E, int maxm, int* uids, int* ucount, int* members);
void or_rot_in(const void* x, int x_dtype, int x_stride, const int* pick, const uint16_t* suh0,
               const uint16_t* suh1, uint16_t* out0, uint16_t* out1, int rows, int K, int slots, int E);
typedef struct {
    const uint16_t* x0;
    const uint16_t* x1;
    const uint32_t* const* tp0;  /* host pointers per expert */
    const uint32_t* const* tp1;
    const int* k2_0;
    const int* k2_1;
    const int* uids;
    const int* ucount;
    const int* members;
    float* z;
    int K, N, P, SK, maxm, slots, nexp_max, mats, cb, warps, ns;
} or_grouped_args;
void or_grouped(const or_grouped_args* a);
void or_gateup_epilogue(const float* Z, const int* pick, const uint16_t* svh_g, const uint16_t* svh_u,
                        const uint16_t* suh_d, uint16_t* xd, int rows, int P, int N, int SK, int slots, int E,
                        float limit, int act_mode);
void or_down_combine(const float* Z, const int* pick, const uint16_t* svh_d, float* y, const float* wts,
                     float* out, int rows, int P, int D, int SK, int slots, int E);

typedef struct {
    const uint32_t* const* ptr[3];   /* gate, up, down: host pointer per expert */
    const int* k2[3];
    const uint16_t* suh_g;
    const uint16_t* suh_u;
    const uint16_t* svh_g;
    const uint16_t* svh_u;
    const uint16_t* suh_d;
    const uint16_t* svh_d;
    int count, dims, width, cb;
} or_routed;
/* moe.routed (moe.zig:279-293): out f32 [R, D]; y is the caller's [R*slots, D] scratch (read for
 * slots whose pick is not an expert, exl3_experts.cu:250-253). */
void or_moe_routed(const void* x, int x_dtype, int x_stride, const int* pick, const float* wts,
                   const or_routed* ex, int R, int slots, float* y, float* out);

/* ---- prefill path (prompt_experts.cu, prompt_experts.zig) ---- */
int or_route(const int* pick, int n, int E, int ipm, int max_items, int* sorted, int* items, int* item_count);
/* out f32 [R, D] = sum over slots of wts * expert(x) (the fp32 sum before any bf16 rounding);
 * do_round rounds each output through bf16 (prompt_experts.zig:246). */
void or_prompt_experts(const void* x, int x_dtype, int x_stride, const int* pick, const float* wts,
                       const or_routed* ex, int R, int slots, int do_round, float* out);

/* ---- EXL3 linear (exl3_linear.cu, linear.zig) ---- */
void or_linear_plan(int k, int n, int* sk, int* wk);
void or_exl3_rot_in(const void* x, int x_dtype, const uint16_t* suh, uint16_t* xh, int M, int K);
/* y [M, N] (y_dtype 0 fp16, 1 bf16, 2 fp32) = FWHT(xh @ W_q) / sqrt(128) * svh (+ bias) */
void or_exl3_linear(const uint16_t* xh, const uint32_t* T, int64_t stride_k, int64_t stride_nb,
                    const uint16_t* svh, const uint16_t* bias, void* y, int y_dtype, int M, int K, int N,
                    int k2, int cb, int SK, int WK);

/* ---- router logits (ops.zig:131-136; native_ops.cu:335-362, 1405-1460) ---- */
void or_router(const uint16_t* x, int x_dtype, int x_stride, const uint16_t* w, int m, int d, int ne, float* part,
               float* out);

/* ---- router top-8 (native_ops.cu:998-1068) ---- */
void or_topk8(const float* logits, const float* bias, int rows, int E, float scale, int* pick, float* wts);

/* ---- the shared expert (forward.zig:2328-2341): gate/up -> bf16, SwiGLU -> bf16, down -> f32 ---- */
void or_swiglu2(const uint16_t* g, const uint16_t* u, uint16_t* out, int n);

/* ---- deterministic data (counter-based: the same bytes on every host) ---- */
uint64_t or_mix64(uint64_t x);
void or_fill_words(uint64_t seed, uint32_t* w, size_t n);

#ifdef __cplusplus
}
#endif
#endif
