// The router's logits: out fp32 [m, ne] = x [m, d] @ w^T with w bf16 [ne, d], the reduction over d cut into eight
// slices of kw = d / 8 that are summed in slice order (ops.zig:131-136: router_part native_ops.cu:1405-1460, then
// router_sum native_ops.cu:335-362).
//
// The summation order inside a slice is this build's own (the reference sums a slice inside tensor-core MMAs, an order
// no document fixes): a wave takes one slice of one (row, expert) dot product; lane l sums the 4-value chunks
// c = l, l + 64, l + 128, .. of the slice (c < kw / 4) in ascending order, each chunk's values in order, by fp32 fma;
// then the 64 lane sums are added by a butterfly over lane distances 32, 16, 8, 4, 2, 1. Products of 16-bit operands
// are exact in fp32, so an fma and a multiply-then-add give the same bits. A block holds the eight slices of its
// experts and rows (a wave a slice) and adds them in slice order, so the logits need no second launch.
#include <hip/hip_runtime.h>

#include "ea_device.hpp"
#include "ea_gemm.hpp"
#include "ea_host.hpp"

namespace ea {

constexpr int RT_SLICES = 8;  // ops.zig:133
constexpr int RT_ROWS = 16;   // rows a block

// The lane sums of a wave added by the butterfly; every lane ends with the total.
__device__ __forceinline__ float wave_sum_butterfly(float v) {
    v = v + lane_xor<32>(v);
    v = v + lane_xor<16>(v);
    v = v + lane_xor<8>(v);
    v = v + lane_xor<4>(v);
    v = v + lane_xor<2>(v);
    v = v + lane_xor<1>(v);
    return v;
}

__device__ __forceinline__ void act4(uint2 u, bool bf, float (&v)[4]) {
    const uint16_t h[4] = {(uint16_t)(u.x & 0xffffu), (uint16_t)(u.x >> 16), (uint16_t)(u.y & 0xffffu),
                           (uint16_t)(u.y >> 16)};
#pragma unroll
    for (int i = 0; i < 4; ++i) v[i] = bf ? bf2f(h[i]) : h2f(h[i]);
}

// Block (expert group of EB, row group of RT_ROWS): wave s computes slice s of every (row, expert) of the block.
// ONE (m = 1): the lane's chunks four at a time, every weight and activation load of the four issued before the
// first product (a chunk past the slice re-reads the slice's last chunk and is not added); the same sums in the same
// order as the general form, whose loads of a row under `r < rows` wait chunk by chunk.
template <int EB, bool ONE>
__global__ void __launch_bounds__(64 * RT_SLICES) router_kernel(const uint16_t* __restrict__ x, int x_bf16,
                                                                int x_stride, const uint16_t* __restrict__ w,
                                                                float* __restrict__ part, float* __restrict__ out,
                                                                int m, int d, int ne) {
    __shared__ float sums[RT_SLICES][RT_ROWS][EB];
    const int lane = threadIdx.x & 63, s = threadIdx.x >> 6;
    const int e0 = blockIdx.x * EB, m0 = blockIdx.y * RT_ROWS;
    const int rows = min(RT_ROWS, m - m0), kw = d / RT_SLICES, nc = kw / 4;
    const bool bf = x_bf16 != 0;
    float acc[RT_ROWS][EB];
#pragma unroll
    for (int r = 0; r < RT_ROWS; ++r)
#pragma unroll
        for (int j = 0; j < EB; ++j) acc[r][j] = 0.0f;
    const size_t k_lo = (size_t)s * kw;
    if constexpr (ONE) {
        static_assert(EB == 1, "one row: one expert a block");
        const uint16_t* wr = w + (size_t)e0 * d + k_lo;  // e0 < ne: a block per expert
        const uint16_t* xr = x + (size_t)m0 * x_stride + k_lo;
        for (int c0 = 0; c0 < nc; c0 += 4 * 64) {
            uint2 wu[4], xu[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int c = min(c0 + i * 64 + lane, nc - 1);
                wu[i] = *reinterpret_cast<const uint2*>(wr + 4 * (size_t)c);
                xu[i] = *reinterpret_cast<const uint2*>(xr + 4 * (size_t)c);
            }
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                float wv[4], xv[4];
                act4(wu[i], true, wv);
                act4(xu[i], bf, xv);
                if (c0 + i * 64 + lane < nc)
#pragma unroll
                    for (int q = 0; q < 4; ++q) acc[0][0] = __builtin_fmaf(xv[q], wv[q], acc[0][0]);
            }
        }
    } else {
#pragma unroll 3
        for (int c = lane; c < nc; c += 64) {
            const size_t k = k_lo + 4 * (size_t)c;
            uint2 wu[EB];
#pragma unroll
            for (int j = 0; j < EB; ++j)
                wu[j] = e0 + j < ne ? *reinterpret_cast<const uint2*>(w + (size_t)(e0 + j) * d + k) : uint2{0u, 0u};
            float wv[EB][4];
#pragma unroll
            for (int j = 0; j < EB; ++j) act4(wu[j], true, wv[j]);
#pragma unroll
            for (int r = 0; r < RT_ROWS; ++r) {
                if (r < rows) {
                    float xv[4];
                    act4(*reinterpret_cast<const uint2*>(x + (size_t)(m0 + r) * x_stride + k), bf, xv);
#pragma unroll
                    for (int j = 0; j < EB; ++j)
#pragma unroll
                        for (int i = 0; i < 4; ++i) acc[r][j] = __builtin_fmaf(xv[i], wv[j][i], acc[r][j]);
                }
            }
        }
    }
#pragma unroll
    for (int r = 0; r < RT_ROWS; ++r) {
        if (r < rows) {
#pragma unroll
            for (int j = 0; j < EB; ++j) {
                const float t = wave_sum_butterfly(acc[r][j]);
                if (lane == 0) sums[s][r][j] = t;
            }
        }
    }
    __syncthreads();
    const int t = threadIdx.x;
    if (t < rows * EB) {
        const int r = t / EB, j = t % EB, e = e0 + j;
        if (e < ne) {
            float tot = sums[0][r][j];
            if (part) part[(size_t)(m0 + r) * ne + e] = tot;
#pragma unroll
            for (int q = 1; q < RT_SLICES; ++q) {
                const float p = sums[q][r][j];
                if (part) part[((size_t)q * m + m0 + r) * ne + e] = p;
                tot = tot + p;
            }
            out[(size_t)(m0 + r) * ne + e] = tot;
        }
    }
}

int launch_router(hipStream_t s, const void* x, int x_dtype, uint32_t x_stride, const void* w, float* part, float* out,
                  uint32_t m, uint32_t d, uint32_t ne) {
    EA_REQUIRE_CTX(c);
    if (!x || !w || !out) return EA_BAD_ARGUMENT;
    if (x_dtype != F16 && x_dtype != BF16) return EA_BAD_ARGUMENT;
    // ops.zig:134: the reduction splits into eight slices of whole 64-value steps
    if (d == 0 || d % (RT_SLICES * 64) != 0) return EA_UNEVEN_SPLIT;
    if (x_stride < d || x_stride % 4 != 0) return EA_BAD_ROW_STRIDE;
    if ((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(w)) & 7) return EA_BAD_ARGUMENT;
    if (m == 0 || ne == 0) return EA_OK;
    const unsigned gy = (m + RT_ROWS - 1) / RT_ROWS;
    const auto* xs = static_cast<const uint16_t*>(x);
    const auto* ws = static_cast<const uint16_t*>(w);
    if (m == 1)
        router_kernel<1, true><<<dim3(ne, gy), 64 * RT_SLICES, 0, s>>>(xs, x_dtype == BF16, (int)x_stride, ws, part,
                                                                        out, (int)m, (int)d, (int)ne);
    else if (m <= RT_ROWS)
        router_kernel<1, false><<<dim3(ne, gy), 64 * RT_SLICES, 0, s>>>(xs, x_dtype == BF16, (int)x_stride, ws, part,
                                                                         out, (int)m, (int)d, (int)ne);
    else
        router_kernel<4, false><<<dim3((ne + 3) / 4, gy), 64 * RT_SLICES, 0, s>>>(xs, x_dtype == BF16, (int)x_stride,
                                                                                   ws, part, out, (int)m, (int)d,
                                                                                   (int)ne);
    return launched();
}

}  // namespace ea

extern "C" int ea_router(ea_stream_t stream, const void* x, int x_dtype, uint32_t x_stride, const void* w, float* part,
                         float* out, uint32_t m, uint32_t d, uint32_t ne) {
    return ea::launch_router(ea::as_stream(stream), x, x_dtype, x_stride, w, part, out, m, d, ne);
}
