// One decode window's MoE FFN in one persistent launch (R <= 16 rows): router top-8 (optional), grouping, the
// routed experts' gate|up with their input rotation, the gate/up epilogue, down with its epilogue, the shared
// expert as one more unit, and the slot-ordered combine (+ shared) into out.
//
// Reference semantics: moe.routed (moe.zig:279-293; exl3_experts.cu), the shared expert's mlp (forward.zig:2328-2341:
// exl3 linears with bf16 outputs, swiglu2, linear down) and ffnMain's add (forward.zig:2401-2403). The work
// decomposition is this build's own: blocks pull items from a device-wide queue in a fixed order -- routing, every
// unit's gate|up k-chunks, every unit's down column blocks -- and an item that needs earlier results waits on a
// flag those items raise; every item it waits on has a lower index, so the queue always drains. Split-k partial
// sums are added in chunk order and the slots in slot order, so the output bits do not depend on timing.
#include <hip/hip_runtime.h>

#include "ea_device.hpp"
#include "ea_gemm.hpp"
#include "ea_experts.hpp"
#include "ea_host.hpp"

namespace ea {

constexpr int DL_THREADS = 256;
constexpr int DL_WAVES = DL_THREADS / 64;
constexpr int DL_MAXR = 16;   // rows of a window (one MFMA row tile)
constexpr int DL_KT = 16;     // k tiles of a gate|up item: 256 k, two Hadamard blocks
constexpr int DL_MAXI = 256;  // widest rank-local intermediate (I) the LDS layout holds
constexpr int DL_RS = 264;    // LDS row stride of the staged activations, halves (padding spreads the banks)

// Scratch of the one-launch layer, carved on the host for the scratch's row capacity (any R up to it runs).
struct DLLayout {
    float* zp;          // [Q, NH, 2, KC, 128] gate|up partial sums, Q = pairs + rows (the shared expert's rows last)
    uint16_t* xd;       // [Q, I] down inputs
    float* sy;          // [rows, D] the shared expert's output
    int* uids;          // [U] unit -> expert (unit 0 is the shared expert when there is one)
    int* ucount;        // [1]
    int* members;       // [U, DL_MAXR] pair ids in row order
    int* mcount;        // [U]
    int* nvalid;        // [rows] slots of a row whose pick is an expert
    unsigned* sync;     // next item, blocks done, generation, routing flag
    unsigned* xd_flag;  // [U, NH] generation of the unit's finished down inputs
    unsigned* cnt_gu;   // [U, NH] gate|up chunks done (reset to zero by the last)
    unsigned* cnt_out;  // [rows, D / 128] contributions arrived (reset to zero by the combine)
};

struct DLArgs {
    const float* logits;  // [R, 256] or null: pick / wts are then inputs
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
    int has_shared, sh_k2;
    const uint32_t* sh_w[3];  // shared gate, up, down words (strips layout)
    const uint16_t* sh_suh[3];
    const uint16_t* sh_svh[3];
    float* out;
    float* yroute;  // [P, D] routed per-pair down outputs (read as they are for slots without an expert)
    DLLayout lay;
    int R, slots, D, I, U;
};

__device__ __forceinline__ unsigned ld_acquire(const unsigned* p) {
    return __hip_atomic_load(p, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_release(unsigned* p, unsigned v) {
    __hip_atomic_store(p, v, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_relaxed(unsigned* p, unsigned v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float ld_coherent(const float* p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Block-wide wait until *flag == v (one thread spins; the others see the data after the barrier and an acquire).
// Every wait here is on an item with a lower queue index, so it ends within microseconds; the spin is still
// bounded (about a second) so that misuse (overlapping calls on one scratch) drains the launch with an error
// instead of holding the GPU.
constexpr unsigned DL_SPIN_LIMIT = 1u << 20;
__device__ __forceinline__ void block_wait(const unsigned* flag, unsigned v, int* status) {
    if (threadIdx.x == 0) {
        unsigned n = 0;
        while (ld_acquire(flag) != v) {
            if (++n == DL_SPIN_LIMIT) {
                record_error(status, DEV_WAIT_TIMEOUT);
                break;
            }
            __builtin_amdgcn_s_sleep(2);
        }
    }
    __syncthreads();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
}

// acc[j] += A (16 staged rows from LDS, rows >= nm read as zero) @ tiles (t, j), t in [0, nkt), two tiles a step.
template <int CB, int K2, int NTW>
__device__ __forceinline__ void wave_tiles_lds(const uint32_t* __restrict__ base, size_t kstride, int nkt,
                                               const uint16_t* xs, int nm, int lane, f4v (&acc)[NTW]) {
    constexpr int TW = 4 * K2;
    using TL = TileLane<K2, CB>;
    constexpr int NWD = TL::NW;
    // an opaque copy of the lane id: keeps the compiler from hoisting every width's lane constants out of the
    // persistent loop (they would stay live across it and spill)
    int ln = lane;
    asm volatile("" : "+v"(ln));
    const TL tl(ln);
    const int m = ln & 15, g = (ln >> 4) & 3;
    const bool live = m < nm;
    const uint16_t* xr = xs + m * DL_RS + 2 * g;
    uint32_t wa[NTW][2][NWD], wb[NTW][2][NWD];
    auto fetch = [&](uint32_t (&w)[NTW][2][NWD], int t) {
        const uint32_t* t0 = base + (size_t)t * kstride;
#pragma unroll
        for (int j = 0; j < NTW; ++j) {
            tl.fetch(t0 + j * TW, w[j][0]);
            tl.fetch(t0 + kstride + j * TW, w[j][1]);
        }
    };
    auto compute = [&](uint32_t (&w)[NTW][2][NWD], int t) {
        h8v a = {0, 0, 0, 0, 0, 0, 0, 0};
        if (live) {
            const uint16_t* xk = xr + t * 16;
            const u4v au = {*reinterpret_cast<const uint32_t*>(xk), *reinterpret_cast<const uint32_t*>(xk + 8),
                            *reinterpret_cast<const uint32_t*>(xk + 16), *reinterpret_cast<const uint32_t*>(xk + 24)};
            a = __builtin_bit_cast(h8v, au);
        }
#pragma unroll
        for (int j = 0; j < NTW; ++j) {
            const u2v b0 = tl.decode(w[j][0]);
            const u2v b1 = tl.decode(w[j][1]);
            const h8v b = __builtin_bit_cast(h8v, (u4v{b0.x, b0.y, b1.x, b1.y}));
            acc[j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, acc[j], 0, 0, 0);
        }
    };
    const int steps = nkt >> 1;  // nkt is even on every call (16 tiles, or I / 16)
    fetch(wa, 0);
    int s = 0;
#pragma unroll 1
    for (; s + 2 <= steps; s += 2) {
        fetch(wb, 2 * s + 2);
        compute(wa, 2 * s);
        if (s + 2 < steps) fetch(wa, 2 * s + 4);
        compute(wb, 2 * s + 2);
    }
    if (s < steps) compute(wa, 2 * s);
}

// ---- routing ----------------------------------------------------------------------------------------------------

// One row's top-8 on one wave (E = 256: four experts a lane): choice = sigmoid + bias, the larger first, the lower
// id on a tie; wts = sigmoid / (sum of the picks' sigmoids in pick order + 1e-20) * scale (native_ops.cu:1015-1068).
__device__ void topk8_wave(const float* logits, const float* bias, float scale, int32_t* pick, float* wts, int lane) {
    float score[4], choice[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const int e = q * 64 + lane;
        score[q] = 1.0f / (expf_path(0.0f - logits[e]) + 1.0f);
        choice[q] = score[q] + bias[e];
    }
    float total = 0.0f;
    float my_w = 0.0f;
    int my_p = 0;
    for (int k = 0; k < 8; ++k) {
        float v = choice[0];
        int i = lane;
#pragma unroll
        for (int q = 1; q < 4; ++q)
            if (choice[q] > v) {  // q * 64 + lane > i: ties keep the lower id
                v = choice[q];
                i = q * 64 + lane;
            }
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) {
            const float ov = __shfl_xor(v, o, 64);
            const int oi = __shfl_xor(i, o, 64);
            if (ov > v || (ov == v && oi < i)) {
                v = ov;
                i = oi;
            }
        }
        const float s = __shfl(score[0], i & 63, 64);
        const float s1 = __shfl(score[1], i & 63, 64);
        const float s2 = __shfl(score[2], i & 63, 64);
        const float s3 = __shfl(score[3], i & 63, 64);
        const int qw = i >> 6;
        const float sw = qw == 0 ? s : (qw == 1 ? s1 : (qw == 2 ? s2 : s3));
        total = total + sw;
        if (lane == k) {
            my_w = sw;
            my_p = i;
        }
        if ((i & 63) == lane) choice[qw] = -__builtin_inff();
    }
    if (lane < 8) {
        pick[lane] = my_p;
        wts[lane] = my_w / (total + 1e-20f) * scale;
    }
}

__device__ void routing_item(const DLArgs& a, const DLLayout& l, unsigned gen, int* sh_pick) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int n = a.R * a.slots;
    if (a.logits) {
        for (int r = wave; r < a.R; r += DL_WAVES)
            topk8_wave(a.logits + (size_t)r * 256, a.bias, a.scale, a.pick + r * 8, a.wts + r * 8, lane);
        __threadfence_block();
        __syncthreads();
    }
    for (int i = threadIdx.x; i < n; i += DL_THREADS) sh_pick[i] = a.pick[i];
    __syncthreads();
    // distinct experts in id order, members in row order (exl3_experts.cu:36-90); E <= 1024: four a thread
    int cnt[4];
    int used = 0;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const int e = threadIdx.x * 4 + q;
        int c = 0;
        if (e < a.E)
            for (int i = 0; i < n; ++i) c += sh_pick[i] == e;
        cnt[q] = c;
        used += c > 0;
    }
    __shared__ int wsum[DL_WAVES];
    int inc = used;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const int v = __shfl_up(inc, o, 64);
        if (lane >= o) inc += v;
    }
    if (lane == 63) wsum[wave] = inc;
    __syncthreads();
    int before = 0;
    for (int w = 0; w < wave; ++w) before += wsum[w];
    int place = before + inc - used;
    const int hs = a.has_shared;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        if (!cnt[q]) continue;
        const int e = threadIdx.x * 4 + q;
        l.uids[hs + place] = e;
        int j = 0;
        for (int i = 0; i < n && j < DL_MAXR; ++i)
            if (sh_pick[i] == e) l.members[(hs + place) * DL_MAXR + j++] = i;
        l.mcount[hs + place] = j;
        ++place;
    }
    if (threadIdx.x == DL_THREADS - 1) {
        int tot = 0;
        for (int w = 0; w < DL_WAVES; ++w) tot += wsum[w];
        *l.ucount = hs + tot;
        if (hs) {
            l.mcount[0] = a.R;
            for (int r = 0; r < a.R; ++r) l.members[r] = r;
        }
    }
    for (int r = threadIdx.x; r < a.R; r += DL_THREADS) {
        int c = 0;
        for (int k = 0; k < a.slots; ++k) {
            const int e = sh_pick[r * a.slots + k];
            c += e >= 0 && e < a.E;
        }
        l.nvalid[r] = c;
    }
    __syncthreads();
    // a row nothing will arrive for (no routed slot, no shared expert): its combine reads y as it is
    if (!hs)
        for (int r = 0; r < a.R; ++r) {
            if (l.nvalid[r] != 0) continue;
            for (int d = threadIdx.x; d < a.D; d += DL_THREADS) {
                float acc = 0.f;
                for (int k = 0; k < a.slots; ++k)
                    acc = __builtin_fmaf(a.wts[r * a.slots + k], a.yroute[(size_t)(r * a.slots + k) * a.D + d], acc);
                a.out[(size_t)r * a.D + d] = acc;
            }
        }
    __threadfence();
    __syncthreads();
    if (threadIdx.x == 0) st_release(a.lay.sync + 3, gen);
}

// ---- gate | up ----------------------------------------------------------------------------------------------------

// The unit's member q-index (pair id, or P + row for the shared expert) and activation row.
__device__ __forceinline__ void member_of(const DLArgs& a, const DLLayout& l, int u, int m, int& q, int& row) {
    if (a.has_shared && u == 0) {
        q = a.R * a.slots + m;
        row = m;
    } else {
        const int p = l.members[u * DL_MAXR + m];
        q = p;
        row = p / a.slots;
    }
}

template <int CB, int SCB>
__device__ void gateup_item(const DLArgs& a, const DLLayout& l, unsigned gen, int u, int nh, int mat, int c,
                            uint16_t* xs, int* sh_last, int* status) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const bool shared = a.has_shared && u == 0;
    if (!shared) {
        block_wait(a.lay.sync + 3, gen, status);
        if (u >= *l.ucount) return;
    }
    const int nm = shared ? a.R : l.mcount[u];
    const int e = shared ? -1 : l.uids[u];
    const int KC = a.D / 256, NH = a.I / 128;
    // the rotated activations of this k range: xs[m][k] = fp16(((x * suh) @ H) * HAD_SCALE), a wave a (row, block)
    const uint16_t* suh = shared ? (mat ? a.sh_suh[1] : a.sh_suh[0]) : (mat ? a.suh_u : a.suh_g) + (size_t)e * a.D;
    for (int task = wave; task < nm * 2; task += DL_WAVES) {
        const int m = task >> 1, blk = task & 1;
        int q, row;
        member_of(a, l, u, m, q, row);
        const int k = c * 256 + blk * 128 + 2 * lane;
        const size_t xi = (size_t)row * a.x_stride + k;
        float v0 = load_act(a.x, a.x_dtype, xi) * h2f(suh[k]);
        float v1 = load_act(a.x, a.x_dtype, xi + 1) * h2f(suh[k + 1]);
        fwht128_w64(v0, v1, lane);
        *reinterpret_cast<uint32_t*>(xs + m * DL_RS + blk * 128 + 2 * lane) =
            (uint32_t)f2h(v0 * HAD_SCALE) | ((uint32_t)f2h(v1 * HAD_SCALE) << 16);
    }
    __syncthreads();
    // wave w: n tiles nh * 8 + 2w, +1 over the 16 k tiles of chunk c
    const int nt0 = nh * 8 + 2 * wave, kt0 = c * DL_KT;
    f4v acc[2] = {f4v{0.f, 0.f, 0.f, 0.f}, f4v{0.f, 0.f, 0.f, 0.f}};
    bool ok;
    if (shared) {
        const int TW = 4 * a.sh_k2;
        const uint32_t* base = (mat ? a.sh_w[1] : a.sh_w[0]) + (size_t)(nt0 >> 3) * (a.D / 16) * 8 * TW + (size_t)kt0 * 8 * TW + (nt0 & 7) * TW;
        ok = EA_K2_SWITCH(a.sh_k2, 2, 10, (wave_tiles_lds<SCB, K2V, 2>(base, (size_t)8 * 4 * K2V, DL_KT, xs, nm, lane, acc)));
    } else {
        const int k2 = (mat ? a.k2t[1] : a.k2t[0])[e];
        const uint32_t* T = reinterpret_cast<const uint32_t*>((mat ? a.ptr[1] : a.ptr[0])[e]);
        const int ns = a.I / 16;
        const uint32_t* base = T + ((size_t)kt0 * ns + nt0) * 4 * k2;
        ok = EA_K2_SWITCH(k2, 2, 10, (wave_tiles_lds<CB, K2V, 2>(base, (size_t)ns * 4 * K2V, DL_KT, xs, nm, lane, acc)));
    }
    if (!ok && lane == 0) record_error(status, DEV_UNSUPPORTED_WIDTH);
    // partial sums of this chunk: zp[q][nh][mat][c][128]
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int m = 4 * (lane >> 4) + i;
            if (m >= nm) continue;
            int q, row;
            member_of(a, l, u, m, q, row);
            const int col = (2 * wave + j) * 16 + (lane & 15);
            a.lay.zp[((((size_t)q * NH + nh) * 2 + mat) * KC + c) * 128 + col] = acc[j][i];
        }
    __threadfence();
    __syncthreads();
    if (threadIdx.x == 0) *sh_last = atomicAdd(l.cnt_gu + u * NH + nh, 1u) == (unsigned)(2 * KC - 1);
    __syncthreads();
    if (!*sh_last) return;
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
    // the last chunk of (unit, column block): chunks summed in order, FWHT, svh, SwiGLU, suh_d, FWHT -> xd
    for (int m = wave; m < nm; m += DL_WAVES) {
        int q, row;
        member_of(a, l, u, m, q, row);
        const float* zg = a.lay.zp + (((size_t)q * NH + nh) * 2 + 0) * KC * 128;
        const float* zu = a.lay.zp + (((size_t)q * NH + nh) * 2 + 1) * KC * 128;
        float g[2] = {0.f, 0.f}, uu[2] = {0.f, 0.f};
        for (int cc = 0; cc < KC; ++cc)
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                g[j] += ld_coherent(zg + cc * 128 + 2 * lane + j);
                uu[j] += ld_coherent(zu + cc * 128 + 2 * lane + j);
            }
        fwht128_w64(g[0], g[1], lane);
        fwht128_w64(uu[0], uu[1], lane);
        const int n = nh * 128 + 2 * lane;
        float v[2];
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            if (shared) {
                // the shared expert's gate / up linears write bf16 (forward.zig:2330), swiglu2 (native_ops.cu:429-441)
                // makes act in bf16, and the down linear's rot_in reads it (exl3_linear.cu:152-173)
                const float gq = bf16r(g[j] * HAD_SCALE * h2f(a.sh_svh[0][n + j]));
                const float uq = bf16r(uu[j] * HAD_SCALE * h2f(a.sh_svh[1][n + j]));
                const float s = bf16r(gq / (expf_path(0.0f - gq) + 1.0f));
                v[j] = bf16r(s * uq) * h2f(a.sh_suh[2][n + j]);
            } else {
                const size_t at = (size_t)e * a.I + n + j;
                const float gg = g[j] * HAD_SCALE * h2f(a.svh_g[at]);
                const float ug = uu[j] * HAD_SCALE * h2f(a.svh_u[at]);
                v[j] = gg / (1.f + expf_path(-gg)) * ug * h2f(a.suh_d[at]);
            }
        }
        fwht128_w64(v[0], v[1], lane);
        *reinterpret_cast<uint32_t*>(a.lay.xd + (size_t)q * a.I + n) =
            (uint32_t)f2h(v[0] * HAD_SCALE) | ((uint32_t)f2h(v[1] * HAD_SCALE) << 16);
    }
    __threadfence();
    __syncthreads();
    if (threadIdx.x == 0) {
        st_relaxed(l.cnt_gu + u * NH + nh, 0u);
        st_release(l.xd_flag + u * NH + nh, gen);
    }
}

// ---- down + combine -------------------------------------------------------------------------------------------------

template <int CB, int SCB>
__device__ void down_item(const DLArgs& a, const DLLayout& l, unsigned gen, int u, int cb, uint16_t* xs, float* ys,
                          int* last_rows, int* n_last, int* status) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const bool shared = a.has_shared && u == 0;
    const int NH = a.I / 128, DB = a.D / 128;
    // every down item needs the routing: the arrival count of a row (nvalid) and, in the combine, wts
    block_wait(a.lay.sync + 3, gen, status);
    if (!shared && u >= *l.ucount) return;
    for (int h = 0; h < NH; ++h) block_wait(l.xd_flag + u * NH + h, gen, status);
    const int nm = shared ? a.R : l.mcount[u];
    const int e = shared ? -1 : l.uids[u];
    // stage the unit's down inputs
    for (int idx = threadIdx.x; idx < nm * (a.I / 2); idx += DL_THREADS) {
        const int m = idx / (a.I / 2), k = 2 * (idx % (a.I / 2));
        int q, row;
        member_of(a, l, u, m, q, row);
        *reinterpret_cast<uint32_t*>(xs + m * DL_RS + k) = *reinterpret_cast<const uint32_t*>(a.lay.xd + (size_t)q * a.I + k);
    }
    __syncthreads();
    const int nt0 = cb * 8 + 2 * wave, KT = a.I / 16;
    f4v acc[2] = {f4v{0.f, 0.f, 0.f, 0.f}, f4v{0.f, 0.f, 0.f, 0.f}};
    bool ok;
    if (shared) {
        const int TW = 4 * a.sh_k2;
        const uint32_t* base = a.sh_w[2] + (size_t)(nt0 >> 3) * KT * 8 * TW + (nt0 & 7) * TW;
        ok = EA_K2_SWITCH(a.sh_k2, 2, 10, (wave_tiles_lds<SCB, K2V, 2>(base, (size_t)8 * 4 * K2V, KT, xs, nm, lane, acc)));
    } else {
        const int k2 = a.k2t[2][e];
        const uint32_t* T = reinterpret_cast<const uint32_t*>(a.ptr[2][e]);
        const int ns = a.D / 16;
        const uint32_t* base = T + (size_t)nt0 * 4 * k2;
        ok = EA_K2_SWITCH(k2, 2, 10, (wave_tiles_lds<CB, K2V, 2>(base, (size_t)ns * 4 * K2V, KT, xs, nm, lane, acc)));
    }
    if (!ok && lane == 0) record_error(status, DEV_UNSUPPORTED_WIDTH);
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int i = 0; i < 4; ++i) ys[(4 * (lane >> 4) + i) * 128 + (2 * wave + j) * 16 + (lane & 15)] = acc[j][i];
    __syncthreads();
    // FWHT of each member's 128 columns, * HAD_SCALE * svh_d: the pair's y (or the shared expert's sy)
    for (int m = wave; m < nm; m += DL_WAVES) {
        int q, row;
        member_of(a, l, u, m, q, row);
        float v0 = ys[m * 128 + 2 * lane], v1 = ys[m * 128 + 2 * lane + 1];
        fwht128_w64(v0, v1, lane);
        const int n = cb * 128 + 2 * lane;
        const uint16_t* svh = shared ? a.sh_svh[2] : a.svh_d + (size_t)e * a.D;
        float* dst = shared ? a.lay.sy + (size_t)row * a.D : a.yroute + (size_t)q * a.D;
        dst[n] = v0 * HAD_SCALE * h2f(svh[n]);
        dst[n + 1] = v1 * HAD_SCALE * h2f(svh[n + 1]);
    }
    __threadfence();
    __syncthreads();
    if (threadIdx.x == 0) *n_last = 0;
    __syncthreads();
    if (threadIdx.x < nm) {
        int q, row;
        member_of(a, l, u, threadIdx.x, q, row);
        const unsigned expect = (unsigned)(l.nvalid[row] + a.has_shared);
        if (atomicAdd(l.cnt_out + row * DB + cb, 1u) == expect - 1) last_rows[atomicAdd(n_last, 1)] = row;
    }
    __syncthreads();
    const int nl = *n_last;
    if (nl == 0) return;
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
    // every contribution to (row, column block) has arrived: the slots in order from 0 (exl3_experts.cu:256-267),
    // then + the shared expert (forward.zig:2403)
    for (int t = wave; t < nl; t += DL_WAVES) {
        const int r = last_rows[t];
        const int n = cb * 128 + 2 * lane;
        float a0 = 0.f, a1 = 0.f;
        for (int k = 0; k < a.slots; ++k) {
            const float w = a.wts[r * a.slots + k];
            const float* y = a.yroute + (size_t)(r * a.slots + k) * a.D + n;
            a0 = __builtin_fmaf(w, ld_coherent(y), a0);
            a1 = __builtin_fmaf(w, ld_coherent(y + 1), a1);
        }
        if (a.has_shared) {
            a0 = a0 + ld_coherent(a.lay.sy + (size_t)r * a.D + n);
            a1 = a1 + ld_coherent(a.lay.sy + (size_t)r * a.D + n + 1);
        }
        a.out[(size_t)r * a.D + n] = a0;
        a.out[(size_t)r * a.D + n + 1] = a1;
        if (lane == 0) st_relaxed(l.cnt_out + r * DB + cb, 0u);
    }
}

// ---- the persistent kernel ---------------------------------------------------------------------------------------

template <int CB, int SCB>
__global__ void __launch_bounds__(DL_THREADS) __attribute__((amdgpu_waves_per_eu(4))) decode_layer_kernel(DLArgs a, int* status) {
    __shared__ __attribute__((aligned(16))) uint16_t xs[DL_MAXR * DL_RS];
    __shared__ __attribute__((aligned(16))) float ys[DL_MAXR * 128];
    __shared__ int sh_item, sh_last, n_last;
    __shared__ int last_rows[DL_MAXR];
    __shared__ int sh_pick[DL_MAXR * 32];
    const DLLayout& l = a.lay;
    const unsigned gen = __hip_atomic_load(a.lay.sync + 2, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) + 1;
    const int NH = a.I / 128, KC = a.D / 256, DB = a.D / 128;
    const int n_gu = a.U * NH * 2 * KC, n_dn = a.U * DB;
    const int total = 1 + n_gu + n_dn;
    for (;;) {
        if (threadIdx.x == 0) sh_item = (int)atomicAdd(a.lay.sync + 0, 1u);
        __syncthreads();
        const int item = sh_item;
        __syncthreads();
        if (item >= total) break;
        if (item == 0) {
            routing_item(a, l, gen, sh_pick);
        } else if (item <= n_gu) {
            const int it = item - 1;
            const int u = it / (NH * 2 * KC), rem = it % (NH * 2 * KC);
            gateup_item<CB, SCB>(a, l, gen, u, rem / (2 * KC), (rem / KC) & 1, rem % KC, xs, &sh_last, status);
        } else {
            const int it = item - 1 - n_gu;
            down_item<CB, SCB>(a, l, gen, it / DB, it % DB, xs, ys, last_rows, &n_last, status);
        }
        __syncthreads();
    }
    // the last block out resets the queue and moves the generation on for the next launch
    if (threadIdx.x == 0) {
        __threadfence();
        if (atomicAdd(a.lay.sync + 1, 1u) == gridDim.x - 1) {
            st_relaxed(a.lay.sync + 0, 0u);
            st_relaxed(a.lay.sync + 1, 0u);
            st_release(a.lay.sync + 2, gen);
        }
    }
}

// ---- host side ----------------------------------------------------------------------------------------------------

static size_t align256(size_t n) { return (n + 255) & ~(size_t)255; }

// Region sizes for a scratch of `rows` rows (capacity); offsets in bytes from the region's base.
struct DLCarve {
    size_t zp, xd, sy, ws, sync, total;
    size_t U, NH, DB;
};

static DLCarve dl_carve(uint32_t rows, uint32_t slots, uint32_t D, uint32_t I, uint32_t E) {
    DLCarve c{};
    const size_t P = (size_t)rows * slots, Q = P + rows;
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
    c.zp = take(Q * c.NH * 2 * KC * 128 * 4);
    c.xd = take(Q * I * 2);
    c.sy = take((size_t)rows * D * 4);
    c.ws = take((c.U + 1 + c.U * DL_MAXR + c.U + rows) * 4);
    c.sync = take((4 + 2 * c.U * c.NH + (size_t)rows * c.DB) * 4);
    c.total = off;
    return c;
}

static bool dl_shape_ok(uint32_t rows, uint32_t slots, uint32_t D, uint32_t I, uint32_t E) {
    return rows >= 1 && rows <= DL_MAXR && slots >= 1 && slots <= 32 && D >= 256 && D % 256 == 0 &&
           (I == 128 || I == DL_MAXI) && E >= 1 && E <= 1024;
}

// Bytes of the one-launch layer's region in a moe scratch of `rows` rows: zero when the shape has no such path.
size_t dl_region_bytes(uint32_t rows, uint32_t slots, uint32_t D, uint32_t I, uint32_t E) {
    return dl_shape_ok(rows, slots, D, I, E) ? dl_carve(rows, slots, D, I, E).total : 0;
}

static DLLayout dl_layout(uint64_t base, uint32_t rows, uint32_t slots, uint32_t D, uint32_t I, uint32_t E) {
    const DLCarve c = dl_carve(rows, slots, D, I, E);
    DLLayout l;
    l.zp = dptr<float>(base + c.zp);
    l.xd = dptr<uint16_t>(base + c.xd);
    l.sy = dptr<float>(base + c.sy);
    int* ws = dptr<int>(base + c.ws);
    l.uids = ws;
    l.ucount = ws + c.U;
    l.members = l.ucount + 1;
    l.mcount = l.members + c.U * DL_MAXR;
    l.nvalid = l.mcount + c.U;
    l.sync = dptr<unsigned>(base + c.sync);
    l.xd_flag = l.sync + 4;
    l.cnt_gu = l.xd_flag + c.U * c.NH;
    l.cnt_out = l.cnt_gu + c.U * c.NH;
    return l;
}

template <int CB, int SCB>
static int dl_launch(hipStream_t s, const DLArgs& a, int* status, int cus) {
    static int per_cu = 0;  // resident blocks a CU, once per instantiation
    if (per_cu == 0) {
        int n = 0;
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, decode_layer_kernel<CB, SCB>, DL_THREADS, 0) !=
                hipSuccess ||
            n < 1)
            n = 1;
        per_cu = n;
    }
    const int NH = a.I / 128, KC = a.D / 256, DB = a.D / 128;
    const int total = 1 + a.U * NH * 2 * KC + a.U * DB;
    int grid = per_cu * cus;
    if (grid > total) grid = total;
    decode_layer_kernel<CB, SCB><<<grid, DL_THREADS, 0, s>>>(a, status);
    return launched();
}

// The one-launch layer: routing from logits (when given), the routed experts of `ex`, the shared expert (when
// given) and their sum into out [R, D]. EA_UNPORTED_GROUPED_VARIANT when the shape, widths or codebooks are not
// instantiated here; the caller then runs the launch sequence.
int decode_layer(hipStream_t s, const void* x, int x_dtype, uint32_t x_stride, const float* logits,
                 const float* bias, float scale, int32_t* pick, float* wts, const ea_routed* ex,
                 const ea_linear* const* shared, const ea_moe_scratch* sc, float* out, uint32_t R) {
    EA_REQUIRE_CTX(c);
    const uint32_t D = ex->dims, I = ex->width, E = ex->count, slots = sc->slots;
    if (!sc->fused || R > sc->rows || !dl_shape_ok(sc->rows, slots, D, I, E)) return EA_UNPORTED_GROUPED_VARIANT;
    if (ex->k2_gu[0] < 2 || ex->k2_gu[1] > 10 || ex->k2_d[0] < 2 || ex->k2_d[1] > 10) return EA_UNPORTED_GROUPED_VARIANT;
    if (logits && (E != 256 || slots != 8)) return EA_UNPORTED_GROUPED_VARIANT;
    if (x_dtype != EA_F16 && x_dtype != EA_BF16) return EA_BAD_ARGUMENT;
    int scb = (int)ex->cb;
    DLArgs a{};
    if (shared) {
        const ea_linear *g = shared[0], *u = shared[1], *d = shared[2];
        if (!g || !u || !d) return EA_BAD_ARGUMENT;
        if (g->k != D || u->k != D || g->n != I || u->n != I || d->k != I || d->n != D) return EA_BAD_WIDTH;
        if (g->k2 != u->k2 || g->k2 != d->k2 || g->cb != u->cb || g->cb != d->cb) return EA_UNPORTED_GROUPED_VARIANT;
        if (g->k2 < 2 || g->k2 > 10) return EA_UNPORTED_GROUPED_VARIANT;
        scb = (int)g->cb;
        a.has_shared = 1;
        a.sh_k2 = (int)g->k2;
        for (int m = 0; m < 3; ++m) {
            a.sh_w[m] = dptr<const uint32_t>(shared[m]->words);
            a.sh_suh[m] = dptr<const uint16_t>(shared[m]->suh);
            a.sh_svh[m] = dptr<const uint16_t>(shared[m]->svh);
        }
    }
    a.logits = logits;
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
    a.lay = dl_layout(sc->fused, sc->rows, slots, D, I, E);
    a.R = (int)R;
    a.slots = (int)slots;
    a.D = (int)D;
    a.I = (int)I;
    const uint32_t P = R * slots;
    a.U = a.has_shared + (int)(P < E ? P : E);
    const int rcb = (int)ex->cb;
    if (rcb == 1 && scb == 1) return dl_launch<1, 1>(s, a, c->status, c->cus);
    if (rcb == 1 && scb == 2) return dl_launch<1, 2>(s, a, c->status, c->cus);
    if (rcb == 2 && scb == 2) return dl_launch<2, 2>(s, a, c->status, c->cus);
    if (rcb == 2 && scb == 1) return dl_launch<2, 1>(s, a, c->status, c->cus);
    return EA_UNPORTED_GROUPED_VARIANT;
}

}  // namespace ea

using namespace ea;

extern "C" {

int ea_ffn_moe_decode(ea_stream_t stream, const void* x, int x_dtype, uint32_t x_stride, const float* logits,
                      const float* bias, float scale, int32_t* pick, float* wts, const ea_routed* ex,
                      const ea_linear* const* shared, const ea_moe_scratch* sc, float* out, uint32_t R) {
    EA_REQUIRE_CTX(c);
    if (!x || !logits || !bias || !pick || !wts || !ex || !sc || !out) return EA_BAD_ARGUMENT;
    if (R > sc->rows) return EA_SCRATCH_TOO_SMALL;
    if (R == 0) return EA_OK;
    return decode_layer(as_stream(stream), x, x_dtype, x_stride, logits, bias, scale, pick, wts, ex, shared, sc, out,
                        R);
}

}  // extern "C"
