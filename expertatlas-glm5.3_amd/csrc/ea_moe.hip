// One MoE layer's routed experts on the decode path (moe.zig): the scratch layout and the launch sequence
// group -> rot_in -> grouped gate|up -> gate/up epilogue -> grouped down -> down epilogue + combine.
#include <hip/hip_runtime.h>

#include "ea_experts.hpp"
#include "ea_host.hpp"

namespace ea {

// moe.zig:16-17: (nt, warps, K splits, prefetch) of the gate/up and down launches.
constexpr uint32_t GATEUP_CFG[4] = {8, 4, 4, 1};
constexpr uint32_t DOWN_CFG[4] = {8, 4, 1, 1};

static size_t align256(size_t n) { return (n + 255) & ~(size_t)255; }

// Windows the decode layer does not hold (more than 16 rows) up to the reference's widest decode window
// (forward.zig:21 MAX_LIN_ROWS = 128) take the prefill path's item GEMMs instead of the six-launch sequence; the
// scratch holds a prompt scratch for them after the sequence's buffers (which the experts.* calls may still use).
constexpr uint32_t WINDOW_ROWS = 128;

struct MoeLayout {
    size_t xg, xu, xd, z, y, ids, count, members, sync, fused, fused_bytes, total;
};

static MoeLayout moe_layout(const ea_routed* ex, uint32_t rows, uint32_t slots) {
    const size_t P = (size_t)rows * slots, D = ex->dims, I = ex->width;
    const size_t maxu = P < ex->count ? P : ex->count;
    const size_t zn = (2 * GATEUP_CFG[2] * I > DOWN_CFG[2] * D ? 2 * GATEUP_CFG[2] * I : DOWN_CFG[2] * D) * P;
    MoeLayout l{};
    size_t off = 0;
    auto take = [&](size_t bytes) {
        const size_t at = off;
        off += align256(bytes);
        return at;
    };
    l.xg = take(P * D * 2);
    l.xu = take(P * D * 2);
    l.xd = take(P * I * 2);
    l.z = take(zn * 4);
    l.y = take(P * D * 4);
    l.ids = take(maxu * 4);
    l.count = take(16);
    l.members = take(maxu * rows * 4);
    l.sync = take(4096);
    l.fused_bytes = dl_region_bytes(rows, slots, (uint32_t)D, (uint32_t)I, ex->count);
    if (l.fused_bytes == 0 && rows > DL_REGION_ROWS && rows <= WINDOW_ROWS && D % 128 == 0 && I % 128 == 0)
        l.fused_bytes = prompt_region_bytes(ex, rows, slots);
    l.fused = take(l.fused_bytes);
    l.total = off;
    return l;
}

__global__ void fill_u32_kernel(uint32_t* p, uint32_t v, size_t n) {
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x) p[i] = v;
}

// Fills n 32-bit words with v by a kernel (not hipMemsetAsync: the call may be captured into a graph).
int fill_words(hipStream_t s, void* p, uint32_t v, size_t n) {
    if (n == 0) return EA_OK;
    size_t blocks = (n + 255) / 256;
    if (blocks > 4096) blocks = 4096;
    fill_u32_kernel<<<(unsigned)blocks, 256, 0, s>>>(static_cast<uint32_t*>(p), v, n);
    return launched();
}

}  // namespace ea

using namespace ea;

extern "C" {

size_t ea_moe_scratch_bytes(const ea_routed* ex, uint32_t rows, uint32_t slots) {
    if (!ex) return 0;
    return moe_layout(ex, rows, slots).total;
}

int ea_moe_scratch_init(ea_stream_t stream, ea_moe_scratch* s, void* base, size_t bytes, const ea_routed* ex,
                        uint32_t rows, uint32_t slots) {
    EA_REQUIRE_CTX(c);
    if (!s || !base || !ex || rows == 0 || slots == 0 || slots > 32) return EA_BAD_ARGUMENT;
    if (reinterpret_cast<uintptr_t>(base) & 255) return EA_BAD_ARGUMENT;
    const MoeLayout l = moe_layout(ex, rows, slots);
    if (bytes < l.total) return EA_SCRATCH_TOO_SMALL;
    const uint64_t b = reinterpret_cast<uintptr_t>(base);
    s->xg = b + l.xg;
    s->xu = b + l.xu;
    s->xd = b + l.xd;
    s->z = b + l.z;
    s->y = b + l.y;
    s->ids = b + l.ids;
    s->count = b + l.count;
    s->members = b + l.members;
    s->sync = b + l.sync;
    s->fused = l.fused_bytes ? b + l.fused : 0;
    s->rows = rows;
    s->slots = slots;
    // moe.zig:271-272: everything zero, members -1
    hipStream_t st = as_stream(stream);
    int r = fill_words(st, base, 0u, l.members / 4);
    if (r) return r;
    r = fill_words(st, dptr<void>(s->members), 0xffffffffu, (l.sync - l.members) / 4);
    if (r) return r;
    return fill_words(st, dptr<void>(s->sync), 0u, (l.total - l.sync) / 4);
}

int ea_moe_routed(ea_stream_t stream, const void* x, int x_dtype, uint32_t x_stride, const int32_t* pick,
                  const float* wts, const ea_routed* ex, const ea_moe_scratch* sc, float* out, uint32_t R) {
    EA_REQUIRE_CTX(c);
    if (!ex || !sc || !x || !pick || !wts || !out) return EA_BAD_ARGUMENT;
    if (R > sc->rows) return EA_SCRATCH_TOO_SMALL;
    if (R == 0) return EA_OK;
    hipStream_t s = as_stream(stream);
    const int f = decode_layer(s, x, x_dtype, x_stride, nullptr, nullptr, 0.f, const_cast<int32_t*>(pick),
                               const_cast<float*>(wts), ex, nullptr, sc, out, R);
    if (f != EA_UNPORTED_GROUPED_VARIANT) return f;
    // more than 16 rows: the prefill path in the scratch's prompt region, when the scratch was made for this shape
    // (its region sits where this layer's layout puts it) and the widths are ones the item GEMMs decode
    if (sc->rows > DL_REGION_ROWS && sc->fused && ex->k2_gu[0] >= 2 && ex->k2_gu[1] <= 16 && ex->k2_d[0] >= 2 &&
        ex->k2_d[1] <= 16 && ex->cb <= 2) {
        const MoeLayout l = moe_layout(ex, sc->rows, sc->slots);
        if (l.fused_bytes && sc->fused == sc->xg + l.fused) {
            ea_prompt_scratch ps{};
            prompt_region_carve(ex, sc->rows, sc->slots, sc->fused, &ps);
            return ea_prompt_experts_run(stream, x, x_dtype, x_stride, pick, wts, ex, &ps, out, R, 0, 0);
        }
    }
    const uint32_t D = ex->dims, I = ex->width, E = ex->count, slots = sc->slots, P = R * slots;
    const uint32_t maxu = P < E ? P : E;
    int r = launch_group(s, pick, dptr<int>(sc->ids), dptr<int>(sc->count), dptr<int>(sc->members), R, slots, E, R);
    if (r) return r;
    r = launch_rot_in(s, x, x_dtype, x_stride, pick, dptr<const uint16_t>(ex->suh_g), dptr<const uint16_t>(ex->suh_u),
                      dptr<uint16_t>(sc->xg), dptr<uint16_t>(sc->xu), R, D, slots, E);
    if (r) return r;
    ea_grouped_args g{};
    g.x0 = sc->xg;
    g.x1 = sc->xu;
    g.tp0 = ex->ptr[0];
    g.tp1 = ex->ptr[1];
    g.k2_0 = ex->k2[0];
    g.k2_1 = ex->k2[1];
    g.uids = sc->ids;
    g.ucount = sc->count;
    g.members = sc->members;
    g.z = sc->z;
    g.K = D;
    g.N = I;
    g.P = P;
    g.SK = GATEUP_CFG[2];
    g.maxm = R;
    g.slots = slots;
    g.nexp_max = maxu;
    g.mats = 2;
    g.cb = ex->cb;
    g.nt = GATEUP_CFG[0];
    g.warps = GATEUP_CFG[1];
    g.pf = GATEUP_CFG[3];
    g.lo = ex->k2_gu[0];
    g.hi = ex->k2_gu[1];
    r = launch_grouped(s, g);
    if (r) return r;
    r = launch_gateup_epilogue(s, dptr<const float>(sc->z), pick, dptr<const uint16_t>(ex->svh_g),
                               dptr<const uint16_t>(ex->svh_u), dptr<const uint16_t>(ex->suh_d),
                               dptr<uint16_t>(sc->xd), R, P, I, GATEUP_CFG[2], slots, E, __builtin_inff(), 1);
    if (r) return r;
    ea_grouped_args d = g;
    d.x0 = d.x1 = sc->xd;
    d.tp0 = d.tp1 = ex->ptr[2];
    d.k2_0 = d.k2_1 = ex->k2[2];
    d.K = I;
    d.N = D;
    d.SK = DOWN_CFG[2];
    d.mats = 1;
    d.nt = DOWN_CFG[0];
    d.warps = DOWN_CFG[1];
    d.pf = DOWN_CFG[3];
    d.lo = ex->k2_d[0];
    d.hi = ex->k2_d[1];
    r = launch_grouped(s, d);
    if (r) return r;
    return launch_down_combine(s, dptr<const float>(sc->z), pick, dptr<const uint16_t>(ex->svh_d),
                               dptr<float>(sc->y), wts, out, R, P, D, DOWN_CFG[2], slots, E);
}

}  // extern "C"
