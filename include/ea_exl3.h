/* ea_exl3.h: the C ABI of the MI355X (gfx950) EXL3 routed-expert path.
 *
 * Drop-in boundary for fiore-labo/ExpertAtlas-GLM5.3's expert dispatch and quantized-linear calls. Each entry
 * point names the reference interface it replaces (paths relative to the reference repository). Conventions,
 * as in the reference:
 *   - every tensor is a raw device address; the caller owns every buffer (weights, tables, scratch);
 *   - no entry point allocates, frees, synchronises or reads device data on the host, except the documented
 *     set-up calls (ea_init, ea_*_scratch_init, ea_prompt_experts_supported);
 *   - every call is asynchronous on `stream` (a hipStream_t; 0 = the null stream), capturable in a HIP graph,
 *     and returns an ea_status checked before any launch;
 *   - fp16 / bf16 arrays are 16-bit patterns; dtype codes follow exl3.zig:8 (0 fp16, 1 bf16, 2 fp32);
 *   - codebooks: 0 3inst, 1 mcg, 2 mul1 (decode.cuh:13). K2 = 2 * bits a weight.
 */
#ifndef EA_EXL3_H
#define EA_EXL3_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef void* ea_stream_t;

/* Status codes map one to one onto the reference's Zig error names. */
typedef enum ea_status {
    EA_OK = 0,
    EA_BAD_ROT_IN = 1,                /* exl3.zig:79 error.BadRotIn */
    EA_UNPORTED_LINEAR_WALK = 2,      /* exl3.zig:98 error.UnportedLinearWalk */
    EA_UNEVEN_K_SPLIT = 3,            /* exl3.zig:102 error.UnevenKSplit */
    EA_UNPORTED_LINEAR_VARIANT = 4,   /* exl3.zig:109,128 error.UnportedLinearVariant */
    EA_TOO_MANY_EXPERTS = 5,          /* experts.zig:99 error.TooManyExperts */
    EA_TOO_MANY_SLOTS = 6,            /* experts.zig:100,196 error.TooManySlots */
    EA_GROUP_SHARED_MEMORY = 7,       /* experts.zig:105 error.GroupSharedMemory */
    EA_UNEVEN_SPLIT = 8,              /* experts.zig:141 error.UnevenSplit */
    EA_BAD_ROW_STRIDE = 9,            /* experts.zig:142 error.BadRowStride */
    EA_UNPORTED_GROUPED_VARIANT = 10, /* experts.zig:148 error.UnportedGroupedVariant */
    EA_BAD_WIDTH = 11,                /* experts.zig:175,197 error.BadWidth */
    EA_SCRATCH_TOO_SMALL = 12,        /* moe.zig:285 error.ScratchTooSmall */
    EA_INVALID = 13,                  /* prompt_experts.zig:147,150 error.Invalid */
    EA_NOT_GROUPABLE = 14,            /* linear.zig:165,181 error.NotGroupable */
    EA_HIP_FAILED = 15,               /* driver.zig:38-47 error.CudaFailed */
    EA_OUT_OF_DEVICE_MEMORY = 16,     /* driver.zig error.OutOfDeviceMemory */
    EA_NOT_INITIALIZED = 17,          /* a call before ea_init on this device */
    EA_BAD_ARGUMENT = 18,             /* a null pointer or a size outside the documented range */
    EA_UNSUPPORTED_WIDTH = 19,        /* a K2 / codebook this build has no decoder for */
    EA_SYNC_TIMEOUT = 20,             /* a kernel's bounded wait on its block's LDS counters gave up */
    /* expert banks (weights.zig, split.zig, moe.zig, expert_swap.zig) */
    EA_BANK_IO = 21,                  /* a file could not be opened or mapped (std.fs errors) */
    EA_BAD_SAFETENSORS = 22,          /* core/safetensors.zig error.BadSafetensors / UnsupportedDType / RankTooHigh */
    EA_BAD_INDEX = 23,                /* weights.zig:48 error.BadIndex */
    EA_MISSING_TENSOR = 24,           /* weights.zig:170-171 error.MissingTensor */
    EA_NO_SPLIT_RULE = 25,            /* split.zig:59 error.NoSplitRule */
    EA_STRADDLES_HADAMARD = 26,       /* split.zig:69,71 error.StraddlesHadamard (UnevenSplit is EA_UNEVEN_SPLIT) */
    EA_STORED_WORLD_NOT_MULTIPLE = 27,/* weights.zig:41,59 error.StoredWorldNotMultiple */
    EA_TOO_MANY_STORED_RANKS = 28,    /* weights.zig:142,203 error.TooManyStoredRanks */
    EA_STORED_SHARES_DIFFER = 29,     /* weights.zig:148,246 error.StoredSharesDiffer */
    EA_BAD_TRELLIS = 30,              /* moe.zig:109,180 error.BadTrellis */
    EA_PACKED_SCALES = 31,            /* moe.zig:88,163 error.PackedScalesUnsupported */
    EA_MIXED_CODEBOOKS = 32,          /* moe.zig:132,212 error.MixedCodebooks */
    EA_SWAP_CODEBOOK_DIFFERS = 33,    /* expert_swap.zig:335,364 error.SwapCodebookDiffers */
    EA_SWAP_BAD_TRELLIS = 34,         /* expert_swap.zig:382 error.SwapBadTrellis */
    EA_SWAP_BAD_SCALES = 35,          /* expert_swap.zig:383 error.SwapBadScales */
    EA_SWAP_WIDTH_UNSUPPORTED = 36,   /* expert_swap.zig:98 error.SwapWidthUnsupported */
    EA_SWAP_NO_BANK = 37,             /* expert_swap.zig:99 error.SwapNoBank */
    EA_OUT_OF_HOST_MEMORY = 38        /* a host allocation of the bank reader failed (Zig's error.OutOfMemory) */
} ea_status;

enum { EA_F16 = 0, EA_BF16 = 1, EA_F32 = 2 };
enum { EA_CB_3INST = 0, EA_CB_MCG = 1, EA_CB_MUL1 = 2 };

const char* ea_strerror(int status);
/* Set-up for the current device (the reference's Kernels.load: experts.zig:84, exl3.zig:63,
 * prompt_experts.zig:72). Idempotent per device. */
int ea_init(int device);
int ea_fini(void);
/* Device-side status word: kernels record an expert width they have no decoder for, or a bounded in-kernel wait that
 * gave up, here instead of trapping (experts_grouped.cuh:265-287 traps); the affected sums are stored as NaN, so the
 * call's output carries the failure too. Reads and clears it; synchronous (tests and health checks only). */
int ea_device_status(int* code);
/* The device address of the current device's status word (one int32, 0 = no error; the first error's ea_status code
 * otherwise), for a host that checks it without a synchronizing call: copy it asynchronously on its own stream (or
 * inside its own graph) after a window's launches and read the copy later. Clearing it is the caller's (a 4-byte
 * write of 0). No counterpart in the reference, whose kernels trap. */
int ea_device_status_address(void** addr);

/* ---- trellis decode --------------------------------------------------------------------------------------- */

/* W [K, N] fp16 from one expert-layout matrix (tile (kt, nt) at ((kt * N/16) + nt) * 4 * K2 words).
 * Replaces tf_exl3x::dequant_kernel (experts_grouped.cuh:317-336). K2 in 2..16. */
int ea_dequant(ea_stream_t stream, const void* trellis, void* w, uint32_t K, uint32_t N, uint32_t k2, uint32_t cb);

/* W [K, N] fp16 from a strided layout (tile (kt, nt) at kt * stride_k + (nt / 8) * stride_nb + (nt % 8) * TW).
 * Replaces exl3.Kernels.unpackW (exl3.zig:125-136; exl3_linear.cu:489-503). */
int ea_exl3_unpack(ea_stream_t stream, const void* t, void* w, uint32_t kdim, uint32_t n, uint32_t k2, uint32_t cb,
                   int64_t stride_k, int64_t stride_nb);

/* ---- routed experts, decode path (experts.zig, moe.zig) ---------------------------------------------------- */

/* uids [maxu], ucount [1], members [maxu, maxm] (row * 32 + slot; -1 padded) of R rows' picks [R, slots].
 * Replaces experts.Kernels.group (experts.zig:98-118; exl3_experts.cu:36-90). */
int ea_experts_group(ea_stream_t stream, const int32_t* pick, int32_t* uids, int32_t* ucount, int32_t* members,
                     uint32_t rows, uint32_t slots, uint32_t experts, uint32_t maxm);

/* out0 / out1 [rows * slots, kdim] fp16 = fp16(((x * suh) @ H) / sqrt(128)) of each routed slot's gate and up.
 * Replaces experts.Kernels.rotIn (experts.zig:122-136; exl3_experts.cu:116-134); x_dtype adds fp16 and fp32
 * inputs to the reference's bf16. */
int ea_experts_rot_in(ea_stream_t stream, const void* x, int x_dtype, uint32_t x_stride, const int32_t* pick,
                      const void* suh0, const void* suh1, void* out0, void* out1, uint32_t rows, uint32_t kdim,
                      uint32_t slots, uint32_t experts);

/* experts.zig:41-67 GroupedArgs (host side only). */
typedef struct ea_grouped_args {
    uint64_t x0, x1;       /* fp16 [P, K] rotated inputs of matrix 0 / 1 */
    uint64_t tp0, tp1;     /* int64 [E] trellis pointers */
    uint64_t k2_0, k2_1;   /* int32 [E] widths */
    uint64_t uids, ucount, members;
    uint64_t z;            /* fp32 [mats, SK, P, N] */
    uint32_t K, N, P, SK, maxm, slots, nexp_max, mats, cb, nt, warps, pf, lo, hi, ns;
} ea_grouped_args;

/* One grouped launch. Replaces experts.Kernels.grouped (experts.zig:140-169; experts_grouped.cuh:214-313). */
int ea_experts_grouped(ea_stream_t stream, const ea_grouped_args* a);

/* xd [P, n] fp16 = rotate(SwiGLU(svh * rotate(sum of gate / up splits)) * suh_d).
 * Replaces experts.Kernels.gateupEpilogue (experts.zig:174-190; exl3_experts.cu:142-184). */
int ea_experts_gateup_epilogue(ea_stream_t stream, const float* z, const int32_t* pick, const void* svh_g,
                               const void* svh_u, const void* suh_d, void* xd, uint32_t rows, uint32_t p, uint32_t n,
                               uint32_t sk, uint32_t slots, uint32_t experts, float limit, uint32_t act_mode);

/* y [P, d] = rotate(sum of down splits) * svh_d; out [rows, d] fp32 = fma chain over slots of wts * y.
 * Replaces experts.Kernels.downCombine (experts.zig:195-211; exl3_experts.cu:223-268). */
int ea_experts_down_combine(ea_stream_t stream, const float* z, const int32_t* pick, const void* svh_d, float* y,
                            const float* wts, float* out, uint32_t rows, uint32_t p, uint32_t d, uint32_t sk,
                            uint32_t slots, uint32_t experts);

/* moe.zig:19-37 Routed: one layer's routed experts on the device. */
typedef struct ea_routed {
    uint64_t ptr[3];       /* gate, up, down: int64 [E] device tables of trellis addresses */
    uint64_t k2[3];        /* int32 [E] device tables of widths */
    uint64_t suh_g, suh_u, svh_g, svh_u, suh_d, svh_d;  /* fp16, stacked [E, D] / [E, I] */
    uint32_t count, dims, width, cb;
    uint32_t k2_gu[2];     /* (min, max) over gate and up */
    uint32_t k2_d[2];
} ea_routed;

/* moe.zig:242-275 Scratch, carved from one caller-owned device buffer. */
typedef struct ea_moe_scratch {
    uint64_t xg, xu, xd, z, y, ids, count, members;
    uint64_t sync;         /* reserved counters (zeroed by ea_moe_scratch_init) */
    uint64_t fused;        /* the decode layer's region (rows <= 16), the prefill path's (17..128 rows), else 0;
                              zeroed by init */
    uint32_t rows, slots;
} ea_moe_scratch;

size_t ea_moe_scratch_bytes(const ea_routed* ex, uint32_t rows, uint32_t slots);
/* Carves `base` (ea_moe_scratch_bytes long, 256-byte aligned) and fills it as moe.zig:271-272 does
 * (zeros; members -1), asynchronously on `stream`. */
int ea_moe_scratch_init(ea_stream_t stream, ea_moe_scratch* s, void* base, size_t bytes, const ea_routed* ex,
                        uint32_t rows, uint32_t slots);

/* out fp32 [R, D] = the R rows' routed experts weighted by wts. Replaces moe.routed (moe.zig:279-293).
 * x: [R, D] rows x_stride apart; pick int32 / wts fp32 [R, slots]. With a scratch of at most 16 rows, widths
 * 2..10, fp16 or bf16 x and I of 128 or 256, the decode layer's launches (one at one row, five above); with a scratch
 * of 17..128 rows (the reference's decode windows, forward.zig:21), the prefill path's item GEMMs in the scratch's
 * prompt region, the slots added in order (the same bits every run; every pair of a window computed); otherwise the
 * six-launch sequence of moe.zig:279-293. On the decode layer and the sequence, as the reference groups pairs
 * (maxm = R), an expert computes its first R pairs in pair order; a slot past them (picks naming one expert more than
 * R times) reads y as it is, as a slot without an expert does. */
int ea_moe_routed(ea_stream_t stream, const void* x, int x_dtype, uint32_t x_stride, const int32_t* pick,
                  const float* wts, const ea_routed* ex, const ea_moe_scratch* s, float* out, uint32_t R);


/* ---- routed experts, prefill path (prompt_experts.zig) ----------------------------------------------------- */

typedef struct ea_prompt_scratch {
    uint64_t sorted, items, count, xd, plane;  /* plane 0: no deterministic pair plane */
    uint64_t xg, xu, z;                        /* this build's rotated inputs and partial sums */
    uint64_t zp, pclass;                       /* this build's K-split sums of large items, each pair's item list */
    uint32_t rows, slots, max_items;
} ea_prompt_scratch;

/* Whether the prefill kernels cover `ex` (prompt_experts.zig:46-61); reads the width tables (synchronous). */
int ea_prompt_experts_supported(const ea_routed* ex, int* ok);
/* prompt_experts.zig:105-122 Scratch.planeBytes / init. planes 0 (the reference's default): no pair plane, the down
 * items add the slots into out with atomics in arrival order (modes 0 and 1); planes 1: the fp32 pair plane [min(rows,
 * 4096) * slots, D] and a slot-ordered combine, the same bits every run (mode 2). A shard the atomic down epilogue does
 * not take (I above 256, or D % 256 != 0) keeps the plane whatever planes says; the byte count follows. */
size_t ea_prompt_scratch_bytes(const ea_routed* ex, uint32_t rows, uint32_t slots, int planes);
int ea_prompt_scratch_init(ea_stream_t stream, ea_prompt_scratch* s, void* base, size_t bytes, const ea_routed* ex,
                           uint32_t rows, uint32_t slots, int planes);

/* out [R, D] fp32 (fp16 with half_sums) = sum over slots of wts * expert(x), rounded through bf16 when do_round.
 * Replaces prompt_experts.run (prompt_experts.zig:146-248). Without a pair plane (s->plane 0) the pass clears its rows
 * of out and its down items add each slot with fp32 atomics (half_sums: packed fp16 atomics; out 4-byte aligned);
 * half_sums with a plane is EA_INVALID (prompt_experts.zig:155), as is half_sums with do_round (:147). The two item
 * lists run side by side: the call forks one
 * per-device side stream off `stream` with events and joins it back before returning, so the call stays capturable;
 * calls on one device therefore must not run or be captured concurrently from several host threads (the side stream
 * and its events are shared; a mutex orders the forks, not the streams' work). */
int ea_prompt_experts_run(ea_stream_t stream, const void* x, int x_dtype, uint32_t xstride, const int32_t* pick,
                          const float* wts, const ea_routed* ex, const ea_prompt_scratch* s, void* out, uint32_t R,
                          int do_round, int half_sums);

/* ---- EXL3 linear (exl3.zig, linear.zig) -------------------------------------------------------------------- */

#define EA_MAX_JOBS 3
/* exl3.zig:12-28, byte for byte (88 / 272 / 48 bytes). */
typedef struct ea_job {
    uint64_t xh, T;
    int64_t stride_k, stride_nb;
    uint64_t svh, bias, y, Z, counters;
    int32_t y_dtype, N, SK, start;
} ea_job;
typedef struct ea_jobs {
    ea_job j[EA_MAX_JOBS];
    int32_t n;
} ea_jobs;
typedef struct ea_rot_jobs {
    uint64_t suh[EA_MAX_JOBS], xh[EA_MAX_JOBS];
} ea_rot_jobs;

/* xh_j [m, kdim] fp16 = fp16(((x * suh_j) @ H) / sqrt(128)) for 1..3 jobs. Replaces exl3.Kernels.rotIn
 * (exl3.zig:78-91; exl3_linear.cu:152-173). */
int ea_exl3_rot_in(ea_stream_t stream, const void* x, int x_dtype, const ea_rot_jobs* jobs, uint32_t njobs,
                   uint32_t m, uint32_t kdim);
/* One launch over `jobs`. Replaces exl3.Kernels.linear (exl3.zig:95-121; exl3_linear.cu:231-484). */
int ea_exl3_linear(ea_stream_t stream, const ea_jobs* jobs, uint32_t m, uint32_t kdim, uint32_t k2, uint32_t cb,
                   uint32_t wk, uint32_t loads);

/* linear.zig:10-33 Linear (words in the strips layout [N/128][K/16][8][TW]). */
typedef struct ea_linear {
    uint64_t words, suh, svh, counters;  /* counters: int32 [8 * N / 128], zero; left zero by the kernel */
    uint32_t k, n, k2, cb, sk, wk;
} ea_linear;
/* linear.zig:142-154 Scratch: xh fp16 [M, K] and z fp32 [SK, M, N] a layer. z must not hold the small-row kernel's
 * tag when first used (zero it once at allocation, as the counters are): calls of up to about 8 rows, and of 17 to 128
 * rows (in passes of 8), with an even split count hand their partial sums over in z as tagged 8-byte slots and leave
 * every slot they used zero. Two calls
 * that run at once on one z race, as in the reference. A call whose status word then reads EA_SYNC_TIMEOUT (a
 * split's block never stored its slot) leaves its slots as they are: zero z again before the next call on it. */
typedef struct ea_linear_scratch {
    uint64_t xh[EA_MAX_JOBS], z[EA_MAX_JOBS];
} ea_linear_scratch;

/* linear.zig:61-79 plan */
void ea_linear_plan(uint32_t k, uint32_t n, uint32_t* sk, uint32_t* wk);
/* linear.zig:164-188 call / callRotated: outs[j] = x @ W_j for 1..3 groupable layers, m <= 128 rows (rot_in + one linear launch). */
int ea_linear_call(ea_stream_t stream, const ea_linear_scratch* s, const ea_linear* const* ls, uint32_t nls,
                   const void* x, int x_dtype, uint32_t m, const uint64_t* outs, const int* out_dtypes);
int ea_linear_call_rotated(ea_stream_t stream, const ea_linear_scratch* s, const ea_linear* const* ls, uint32_t nls,
                           uint32_t m, const uint64_t* outs, const int* out_dtypes);

/* ---- routing input and the shared expert's activation ------------------------------------------------------ */

/* pick int32 / wts fp32 [rows, 8] from logits fp32 [rows, 256] and bias fp32 [256]: sigmoid + bias, top 8 (the
 * lower id on a tie), wts = sigmoid / (their sum + 1e-20) * scale; log: 0 or a byte per pick.
 * Replaces ops.topk (ops.zig:189-191; native_ops.cu:998-1068). */
int ea_topk8(ea_stream_t stream, const float* logits, const float* bias, int32_t* pick, float* wts, uint32_t rows,
             float scale, uint8_t* log);

/* The router's logits: out fp32 [m, ne] = x [m, d] @ w^T, w bf16 [ne, d] (rows of d), x fp16 or bf16 (x_dtype 0 / 1;
 * the reference takes bf16) with rows x_stride elements apart. The reduction over d is cut into eight slices of d / 8
 * that are added in slice order; when part is not NULL the slice sums are also written to part fp32 [8, m, ne]. One
 * launch. Replaces ops.router (ops.zig:131-136): router_part (native_ops.cu:1405-1460) + router_sum (:335-362).
 * Within a slice the order is this build's (the reference's is inside tensor-core MMAs): lane l of a wave sums the
 * 4-value chunks l, l + 64, .. of the slice in order by fp32 fma, then a butterfly adds the 64 lane sums over lane
 * distances 32, 16, 8, 4, 2, 1. d % 512 != 0: EA_UNEVEN_SPLIT (ops.zig:134 unsupported); x_stride < d or not a
 * multiple of 4: EA_BAD_ROW_STRIDE; x or w not 8-byte aligned: EA_BAD_ARGUMENT. */
int ea_router(ea_stream_t stream, const void* x, int x_dtype, uint32_t x_stride, const void* w, float* part,
              float* out, uint32_t m, uint32_t d, uint32_t ne);

/* out = bf16(bf16(silu(g)) * u) over rows of `width` bf16. Replaces ops.swiglu2 (native_ops.cu:429-441). */
int ea_swiglu2(ea_stream_t stream, const void* g, const void* u, void* out, uint32_t rows, uint32_t width);

/* a[i] += b[i] for n fp32 values: the routed part plus the shared expert (forward.zig:2403 -> glue.addF32,
 * glue.cu:57). */
int ea_add_f32(ea_stream_t stream, float* a, const float* b, size_t n);

/* ---- the decode layer in one call --------------------------------------------------------------------------- */

/* ffnMain's expert part for a decode window in one call (one launch at one row, five above): pick / wts
 * [R, 8] = top-8 of logits [R, 256] (as
 * ea_topk8, written out), out [R, D] = moe.routed(x) + the shared expert's mlp(x) (gate and up EXL3 linears with
 * bf16 outputs, swiglu2, the down linear with fp32 output), or the routed part alone when shared is NULL.
 * Replaces the sequence ops.topk -> moe.routed -> forward.mlp -> glue.addF32 of forward.zig:2361-2403 (the
 * reference's decode graph issues those as separate launches). shared: gate, up, down ea_linear (k, n = D, I / I, D;
 * one width in 2..10 and one codebook, mcg or mul1: the codebooks the reference's linear takes). Needs s from
 * ea_moe_scratch_init with rows <= 16, R <= rows, E = 256, slots = 8, I of 128 or 256, routed widths 2..10, routed
 * codebook 3inst, mcg or mul1; EA_UNPORTED_GROUPED_VARIANT otherwise. Concurrent calls sharing one scratch race. */
int ea_ffn_moe_decode(ea_stream_t stream, const void* x, int x_dtype, uint32_t x_stride, const float* logits,
                      const float* bias, float scale, int32_t* pick, float* wts, const ea_routed* ex,
                      const ea_linear* const* shared, const ea_moe_scratch* s, float* out, uint32_t R);

/* ffnMain's routing and expert part from the normed activations: logits fp32 [R, 256] = x @ router_w^T (router_w bf16
 * [256, D]; ea_router's launch and summation order), written to `logits` (caller-owned, as the reference's mlog), then
 * ea_ffn_moe_decode on them. Replaces ops.router -> ops.topk -> moe.routed -> forward.mlp -> glue.addF32
 * (forward.zig:2350-2403; ops.zig:131-136). Beyond ea_ffn_moe_decode's conditions: D % 512 == 0 (EA_UNEVEN_SPLIT),
 * x_stride >= D and a multiple of 4 (EA_BAD_ROW_STRIDE), x and router_w 8-byte aligned (EA_BAD_ARGUMENT); all are
 * checked before the first launch. */
int ea_ffn_moe_decode_router(ea_stream_t stream, const void* x, int x_dtype, uint32_t x_stride, const void* router_w,
                             float* logits, const float* bias, float scale, int32_t* pick, float* wts,
                             const ea_routed* ex, const ea_linear* const* shared, const ea_moe_scratch* s, float* out,
                             uint32_t R);

/* ea_ffn_moe_decode without a scratch argument: it allocates nothing and takes no workspace. No counterpart in the
 * reference: it is for callers that cannot allocate device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc). The scratch is a file-scope device array of 12 MiB that the library holds on each
 * device it runs on until the process ends (resolved and cleared by ea_init), carved for 16 rows of the call's layer
 * shape. R above 16, or a layer shape whose carve exceeds the array, returns EA_SCRATCH_TOO_SMALL before any launch;
 * shapes the decode layer does not take return EA_UNPORTED_GROUPED_VARIANT (there is no sequence fallback). Every call
 * on a device shares that device's array: calls that overlap in time on one device (several streams, or concurrent
 * host threads) race and must not be issued. */
int ea_ffn_moe_decode_static(ea_stream_t stream, const void* x, int x_dtype, uint32_t x_stride, const float* logits,
                             const float* bias, float scale, int32_t* pick, float* wts, const ea_routed* ex,
                             const ea_linear* const* shared, float* out, uint32_t R);

/* ---- expert banks: a rank's shard of a checkpoint, loading a layer, changing experts' widths ------------------ */

/* weights.Reader (weights.zig:20-240): a checkpoint or bank directory read for tensor-parallel rank `rank` of `world`.
 * Whole tensors are cut to the rank's share by the split rules (split.zig:18-81: output-split projections cut the
 * trellis' second axis and svh, input-split ones the trellis' first axis and suh; markers and the other scale whole;
 * shares never straddle a 128-value Hadamard block); pre-sharded tensors ("...P_proj.rank{s}.S", assemble.py:173-237)
 * from stored_world ranks are joined stored_world / world at a time. Host-side only (no GPU). */
typedef struct ea_bank ea_bank;
/* weights.zig:41-51 Reader.open: dir/model.safetensors.index.json ("weight_map": name -> file). */
int ea_bank_open(const char* dir, uint32_t rank, uint32_t world, uint32_t stored_world, ea_bank** out);
/* weights.zig:52-61 Reader.openFile: one safetensors file of dir, every tensor it holds. */
int ea_bank_open_file(const char* dir, const char* fname, uint32_t rank, uint32_t world, uint32_t stored_world,
                      ea_bank** out);
void ea_bank_close(ea_bank* b);
/* weights.zig:196-202 Reader.has: the tensor is there, whole or as stored ranks (1 / 0). */
int ea_bank_has(const ea_bank* b, const char* name);
/* A share's dtype (0 BOOL 1 U8 2 I8 3 U16 4 I16 5 F16 6 BF16 7 U32 8 I32 9 F32 10 U64 11 I64 12 F64), rank, shape (1
 * past rank) and byte count. */
typedef struct ea_share_info {
    int32_t dtype;
    uint32_t rank;
    uint64_t shape[8];
    uint64_t bytes;
} ea_share_info;
/* weights.zig:204-225 Reader.get: this rank's share of `name` into host memory dst (cap bytes; dst NULL: info only). */
int ea_bank_share(ea_bank* b, const char* name, ea_share_info* info, void* dst, uint64_t cap);

/* One MoE layer's routed experts on the current device, loaded from banks: moe.loadFrom (moe.zig:65-151). Every
 * expert's gate / up / down trellis shares ("model.layers.L.mlp.experts.e.{gate,up,down}_proj.trellis", i16
 * [K/16, N/16, 8 K2]) back to back in one slab a projection, each 256-byte aligned; int64 pointer and int32 width
 * tables; fp16 suh / svh stacked [E, K] / [E, N]; the codebook from expert 0's gate marker (.mcg 1, .mul1 2, none 0).
 * readers: one per bank; pick (E bytes) names each expert's reader, or NULL for readers[0] (then nreaders >= 1);
 * with a pick, every expert's markers must agree (EA_MIXED_CODEBOOKS). The layer owns its device memory. Set-up call:
 * allocates and copies synchronously. */
typedef struct ea_layer ea_layer;
int ea_layer_load(ea_bank* const* readers, uint32_t nreaders, const uint8_t* pick, uint32_t layer, uint32_t experts,
                  ea_layer** out);
/* The layer's ea_routed (its device tables and scales), valid until ea_layer_free. */
const ea_routed* ea_layer_routed(const ea_layer* l);
void ea_layer_free(ea_layer* l);
/* Experts changed (expert_swap.zig swapLayer). */
typedef struct ea_swap_stats {
    uint32_t experts, up, down;
    uint64_t read_bytes;
} ea_swap_stats;
/* Change experts' widths between calls (expert_swap.zig:345-467): expert j goes from current[j] to target[j] bits,
 * read from banks[target[j]] (banks: 9 readers indexed by bits, NULL where none; the reference opens
 * "experts-layer-NNN.safetensors" of each width's bank dir: expert_swap.zig:301-308). New slabs are made (unchanged
 * experts copied on the device, changed ones uploaded), the changed experts' scales overwritten, and the ptr / k2 tables
 * rewritten in place: a captured graph holds the tables' addresses, so its replays run the new widths. The K2 ranges
 * of the ea_routed only widen. A failure before the device is written leaves the layer as it was. Synchronous; no
 * kernel may use the layer meanwhile. */
int ea_layer_swap(ea_layer* l, ea_bank* const* banks, uint32_t layer, const uint8_t* target, const uint8_t* current,
                  ea_swap_stats* st);

/* ---- benchmark instrumentation (no counterpart in the reference) ------------------------------------------- */

/* With on != 0, every call that runs the decode layer (ea_ffn_moe_decode, and ea_moe_routed when it takes that
 * path) records a HIP event on its stream before each of its four stages (gate|up, epilogue, down, combine) and after
 * the last; a stage run inside another launch (the epilogue and the combine with one row) is the time between two
 * back-to-back events. For benchmarks; not under graph capture. */
int ea_profile_enable(int on);
/* ms[0..3]: the four stages of the most recent recorded call, in milliseconds (waits for that call); n >= 4.
 * EA_INVALID when nothing was recorded since ea_profile_enable. */
int ea_profile_stages(float* ms, uint32_t n);

#ifdef __cplusplus
}
#endif
#endif
