// Launchers of the decode-path expert kernels (ea_experts.hip), shared with the layer orchestration.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "ea_exl3.h"

namespace ea {

int launch_group(hipStream_t s, const int* pick, int* uids, int* ucount, int* members, uint32_t rows, uint32_t slots,
                 uint32_t experts, uint32_t maxm);
int launch_rot_in(hipStream_t s, const void* x, int x_dtype, uint32_t x_stride, const int* pick, const uint16_t* suh0,
                  const uint16_t* suh1, uint16_t* out0, uint16_t* out1, uint32_t rows, uint32_t kdim, uint32_t slots,
                  uint32_t experts, void* zero = nullptr, int zero_half = 0);
int launch_grouped(hipStream_t s, const ea_grouped_args& a);
// The prefill path's scratch inside a moe scratch of more than 16 rows (ea_prompt.hip): its bytes, and its carve
// from `base` (the pair plane included; zeroed by ea_moe_scratch_init, which is all a prompt scratch needs).
size_t prompt_region_bytes(const ea_routed* ex, uint32_t rows, uint32_t slots);
int prompt_region_carve(const ea_routed* ex, uint32_t rows, uint32_t slots, uint64_t base, ea_prompt_scratch* s);
// With pclass: a pair with pclass[pair] != 0 sums z's split 0 and then zp's planes 1 .. skp - 1 ([skp - 1][2][p][n])
// instead of z's sk splits; only >= 0 (with pclass) takes just the pairs of that class (0 or 1).
int launch_gateup_epilogue(hipStream_t s, const float* z, const int* pick, const uint16_t* svh_g,
                           const uint16_t* svh_u, const uint16_t* suh_d, uint16_t* xd, uint32_t rows, uint32_t p,
                           uint32_t n, uint32_t sk, uint32_t slots, uint32_t experts, float limit, uint32_t act_mode,
                           const int* pclass = nullptr, const float* zp = nullptr, uint32_t skp = 1,
                           int only = -1);
int launch_down_combine(hipStream_t s, const float* z, const int* pick, const uint16_t* svh_d, float* y,
                        const float* wts, float* out, uint32_t rows, uint32_t p, uint32_t d, uint32_t sk,
                        uint32_t slots, uint32_t experts, bool skip_invalid = false);

// The most rows the decode layer's launches take; a moe scratch above it holds the prefill path's region instead.
constexpr uint32_t DL_REGION_ROWS = 16;
// The decode layer (ea_decode_layer.hip): the region a moe scratch of `rows` rows holds for it (zero when the shape
// has none), and its launches (EA_UNPORTED_GROUPED_VARIANT when not instantiated for the layer). router_w (bf16
// [256, D]) or null: when given, a router launch first writes the logits into `logits`.
size_t dl_region_bytes(uint32_t rows, uint32_t slots, uint32_t D, uint32_t I, uint32_t E);
int decode_layer(hipStream_t s, const void* x, int x_dtype, uint32_t x_stride, const float* logits,
                 const float* bias, float scale, int32_t* pick, float* wts, const ea_routed* ex,
                 const ea_linear* const* shared, const ea_moe_scratch* sc, float* out, uint32_t R,
                 const void* router_w = nullptr);

// The router's logits (ea_router.hip): out fp32 [m, ne] = x [m, d] @ w^T, eight slices added in order.
int launch_router(hipStream_t s, const void* x, int x_dtype, uint32_t x_stride, const void* w, float* part, float* out,
                  uint32_t m, uint32_t d, uint32_t ne);

}  // namespace ea
