/*
 * moe_mi355x.h — C ABI of the MI355X (gfx950) quantised MoE-layer library, libmoe_mi355x.so.
 *
 * The reference (Tigerly1/moe-lab) has no native FFI: its drop-in boundary is the Python "variant"
 * module contract (reference README.md:141-158, moelab/mlx_backend.py:3-8, moelab/torch_backend.py:3-5):
 *     prepare(w_gate, w_up, w_down) -> state;  run(state, x, idx, wts, act) -> y;  dequant(state)
 * plus run_slots (moelab/variants/mlx/metal_q4_moe.py:49-51) and the fused router tail topk_norm
 * (moelab/router.py:71-80). Each entry point below replaces the GPU work behind one of those calls;
 * the Python variant modules in moe-lab_amd/variants/ bind them with ctypes (moe-lab_amd/_lib.py).
 *
 * Conventions (all entry points):
 *   - every pointer is a device pointer (HBM), except the moe_experts_t descriptor itself, which
 *     lives in host memory and is read during the call only;
 *   - all work is enqueued on `stream` (a hipStream_t, passed as void*; NULL = default stream) and
 *     is asynchronous; nothing allocates device memory and nothing synchronises the host;
 *   - outputs and workspace are caller-allocated; sizes come from the *_workspace_bytes queries;
 *   - return 0 on success, a negative MOE_ERR_* code on invalid arguments (checked before any
 *     launch; mirrors the reference's shape asserts, e.g. metal_q4_moe.py:34) or launch failure;
 *   - reentrant; calls that share a workspace must be stream-ordered. The library's only mutable state is the table
 *     of moe_experts_run_static's array addresses, one per device, filled once under a lock (and that array).
 */
#ifndef MOE_MI355X_H
#define MOE_MI355X_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* return codes */
#define MOE_OK 0
#define MOE_ERR_ARG (-1)       /* shape, size or pointer argument invalid */
#define MOE_ERR_DTYPE (-2)     /* activation dtype or weight format not supported by this entry */
#define MOE_ERR_WORKSPACE (-3) /* workspace missing or smaller than *_workspace_bytes */
#define MOE_ERR_LAUNCH (-4)    /* the HIP runtime refused a launch */
#define MOE_ERR_ALIGN (-5)     /* a pointer is not 16-byte aligned */

/* activation / logits dtypes */
#define MOE_DTYPE_BF16 0
#define MOE_DTYPE_F16 1
#define MOE_DTYPE_F32 2

/*
 * Weight formats. The reference's state holds, per projection, codes u32 [E, N, K/8] (8 nibbles per word,
 * low nibble first) plus scales/biases bf16 [E, N, K/64] (int4 g64, metal_q4_decode_v4.py:161-169) or E8M0
 * bytes u8 [E, N, K/32] (MXFP4, metal_mxfp4_moe.py:448-455). This library takes the same numbers packed
 * row by row: each of the E*N rows is one record of moe_row_bytes(fmt, K) bytes, the row's K/2 code bytes
 * (the reference's words, unchanged) followed by its group metadata, zero-padded to a multiple of 16:
 *   MOE_FMT_INT4_G64: K/64 words, word g = scale_g (bf16, low half) | bias_g (bf16, high half) << 16
 *   MOE_FMT_MXFP4:    K/32 E8M0 bytes
 * so a row streams as one contiguous run. moelab_amd.formats converts in both directions.
 */
#define MOE_FMT_INT4_G64 0
#define MOE_FMT_MXFP4 1

/* GLU activations (reference metal_q4_decode_v4.py:36-41, metal_mxfp4_gptoss.py:36-43) */
#define MOE_ACT_SWIGLU 0      /* silu(g) * u */
#define MOE_ACT_GEGLU 1       /* tanh-GELU(g) * u (Gemma-4) */
#define MOE_ACT_GPTOSS 2      /* g = min(g,7), u = clip(u,-7,7), g * sigmoid(1.702 g) * (u + 1) */

/* expert-path selection for moe_experts_run */
#define MOE_PATH_AUTO 0       /* T == 1 -> per-slot GEMV (two launches); T > 1 -> grouped expert tiles */
#define MOE_PATH_SLOTS 1      /* per-slot GEMV over all T*k slots, no grouping, two launches (the stock-style
                                 gather of the reference's pre-tile kernels) */
#define MOE_PATH_GROUPED 2    /* grouped expert tiles: each selected expert's weights read once */

/* One projection of all E experts: N output rows of K inputs. */
typedef struct {
    const void* rows;    /* packed rows [E, N, moe_row_bytes(fmt, K)], 16-byte aligned */
    const float* bias;   /* optional additive row bias fp32 [E, N] (gpt-oss), NULL if none */
    const void* tiles;   /* optional: the same weights in the tile-major layout below (moe_tiles_pack of rows),
                            E * moe_tile_bytes(fmt, N, K) bytes, 16-byte aligned. The grouped path (T > 1)
                            streams these; NULL in any of gate/up/down: it reads rows (slower) */
} moe_proj_t;

/* Bytes of one packed row of K inputs in format fmt (0 for an invalid fmt or K). */
size_t moe_row_bytes(int fmt, int K);

/*
 * Tile-major layout (no counterpart in the reference, whose Metal kernels read its words row by row): the
 * grouped T > 1 path loads 16 rows x 128 inputs per MFMA step group, and HBM delivers such loads near its peak
 * only as contiguous bursts, so the same numbers are re-laid out once, at load time, on the device:
 *   tiles [E][N/16][S = ceil(K/128)][slice record], a slice record = 16 rows x 128 inputs:
 *     1024 bytes of code words: 16 bytes at offset 16 * (r + 16 g) (row r, lane group g = 0..3) hold the
 *     row's words (index within the row, s = slice)
 *         MOE_FMT_INT4_G64: 16s + 2g, 16s + 2g + 1, 16s + 8 + 2g, 16s + 9 + 2g
 *         MOE_FMT_MXFP4:    16s + g, 16s + 4 + g, 16s + 8 + g, 16s + 12 + g
 *     each with its nibbles (codes e0 .. e7, low nibble first) stored as e0 e2 e4 e6 e1 e3 e5 e7
 *     then the metadata of the slice's groups, per row r:
 *         MOE_FMT_INT4_G64: 8 bytes at 1024 + 8r = group words 2s, 2s + 1, each (scale, bias) times 2^-X
 *                           (bf16, exact), X the row's exponent below   (record: 1152 bytes)
 *         MOE_FMT_MXFP4:    4 bytes at 1024 + 4r = E8M0 bytes of groups 4s .. 4s + 3   (record: 1088 bytes)
 *     words and groups past K (K % 128 == 64) are zero.
 *   int4 only, after the records of all E experts: row exponents int8 [E][N]. X = (biased exponent of the row's
 *     largest bf16 |scale| or |bias|) - 137, i.e. floor(log2 of it) - 10, clamped to [-120, 120]; 0 for an
 *     all-zero row or one holding an inf or NaN. The scaled metadata puts every row's largest at [2^10, 2^11), so
 *     the kernels that dequantise to fp16 keep any absolute scale range (scales of 1e-8 or 1e30 alike); the tile
 *     kernels multiply each row's sums by 2^X.
 * moe_tile_bytes: bytes per expert of an N x K projection in this layout (int4: records + N exponent bytes;
 *                 0 if N % 16, K % 64 or fmt invalid).
 * moe_tiles_pack: rows [E, N, moe_row_bytes(fmt, K)] -> tiles [E * moe_tile_bytes(fmt, N, K)], on `stream`.
 */
size_t moe_tile_bytes(int fmt, int N, int K);
int moe_tiles_pack(int fmt, int E, int N, int K, const void* rows, void* tiles, void* stream);

/* Expert weights: gate/up [E, F, d], down [E, d, F]. */
typedef struct {
    int32_t fmt;         /* MOE_FMT_* */
    int32_t E, d, F;
    moe_proj_t gate, up, down;
} moe_experts_t;

/*
 * Fused router: gate GEMV + router tail.
 * Replaces the stock gate GEMV self.gate(x) (reference e2e.py:57-59) followed by router.topk_norm
 * (reference moelab/router.py:71-80; semantics router.py:1-12).
 *   x [T, d] bf16, wr [E, d] bf16, bias [E] fp32 or NULL
 *   logits [T, E] fp32 out: x . wr^T (+ bias), fp32, fixed reduction order (see the kernel source)
 *   idx [T, k] int32, wts [T, k] fp32 out; norm = 1: softmax over the top-k logits (= renormalised
 *   softmax), norm = 0: full-softmax probabilities (DeepSeek-V2 greedy); weights are multiplied by scale.
 *   Ties: lowest expert id. NaN logits count as -inf. Limits: E <= 1024, 1 <= k <= min(E, 32), d % 8 == 0.
 *   Two launches: the logits over many workgroups, then the tails, one wave per token. counters: unused (may be NULL; kept, with moe_router_counter_count, so existing callers link
 *   unchanged).
 */
int moe_router(const void* x, const void* wr, const float* bias, int T, int d, int E, int k, int norm, float scale,
               float* logits, int32_t* idx, float* wts, int32_t* counters, void* stream);
int moe_router_counter_count(int T);

/*
 * Fused router that also builds the slot grouping: moe_router's logits launch, then one launch that runs every token's
 * tail (one wave per token: the same ids and weights as moe_router), after which the last workgroup to finish sorts
 * the T*k slots p = t*k + j stably by expert, with the counts' offsets from a wave prefix sum. Replaces the stock gate
 * GEMV +
 * router.topk_norm (as moe_router) followed by the grouping prepass of the grouped kernels (reference
 * metal_q4_tiles_v2.py:362-373 MAP kernel order, closed form of reference triton_fused_moe.py:56-70 align()).
 *   x, wr, bias, T, d, E, k, norm, scale, logits, idx, wts: as moe_router;
 *   counts [E], offsets [E+1], sorted [T*k], active [E], meta [2] int32 out: as moe_group (meta[1] = 0).
 */
int moe_router_group(const void* x, const void* wr, const float* bias, int T, int d, int E, int k, int norm,
                     float scale, float* logits, int32_t* idx, float* wts, int32_t* counts, int32_t* offsets,
                     int32_t* sorted, int32_t* active, int32_t* meta, void* stream);

/*
 * Router tail on given logits: reference moelab/router.py:71-80 topk_norm(logits, k, norm).
 *   logits [T, E] of dtype MOE_DTYPE_*; idx [T, k] int32, wts [T, k] fp32 out.
 */
int moe_topk(const void* logits, int dtype, int T, int E, int k, int norm, float scale, int32_t* idx, float* wts,
             void* stream);

/*
 * Slot grouping: slots p = t*k + j sorted stably by expert (reference metal_q4_tiles_v2.py:362-373 MAP
 * kernel order; closed form of reference triton_fused_moe.py:56-70 align()).
 *   idx [n] int32 in; counts [E], offsets [E+1], sorted [n], active [E], meta [2] int32 out.
 *   meta[0] = number of experts with count > 0 (listed ascending in active[0..meta[0]) , rest -1);
 *   meta[1] = number of slots whose id is outside [0, E) (they join no group).
 */
int moe_group(const int32_t* idx, int n, int E, int32_t* counts, int32_t* offsets, int32_t* sorted, int32_t* active,
              int32_t* meta, void* stream);

/*
 * Expert part of the layer: reference variant run(state, x, idx, wts, act) (metal_q4_moe.py:54-64,
 * metal_mxfp4_moe.py:474-512, metal_mxfp4_gptoss.py:129-167):
 *   y[t] = residual[t] + sum_j wts[t,j] * ( down_e( act(gate_e x_t + bg_e, up_e x_t + bu_e) ) + bd_e ),
 *   e = idx[t,j]; residual optional (NULL = 0).
 *   x [T, d] of x_dtype (MOE_DTYPE_BF16, MOE_DTYPE_F16 or MOE_DTYPE_F32: fp16 and fp32 x enter the gate/up
 *   products exactly, as 2 or 3 bf16 planes whose sum is x; the reference's fp32 path is its exact scalar tiles,
 *   metal_q4_moe.py:62-64); y and residual [T, d] of y_dtype (any of the three; the reference returns x.dtype,
 *   MOE_DTYPE_F32 gives the unrounded result); idx [T, k] int32; wts [T, k] fp32.
 *   path: MOE_PATH_*; nored = 1 writes the unweighted per-slot outputs y[T*k, d] instead (reference
 *   run_slots / NORED, metal_q4_moe.py:49-51; per-slot path only, residual must be NULL).
 *   Accumulation in fp32; the GLU output h is kept between the two launches as an unevaluated sum of two
 *   bf16 planes (about 16 significant bits, where the reference kernels store it in x.dtype). Exception: int4
 *   grouped calls with more than 16 slots per expert on average (prefill-sized T, path MOE_PATH_GROUPED with
 *   the tile-major copies) run the down projection, and above 32 also the gate/up, on fp16 MFMA: weights
 *   rounded once to fp16 from the row-exponent-scaled metadata, x and h carried as fp16 with a power-of-two
 *   exponent per row (no overflow and no flush to zero whatever a row's absolute scale); within a row, weights
 *   more than 2^13 below the row's largest |16 s|, |b| fall into fp16's subnormal range (absolute step 2^-19 of
 *   the row's largest |s|, |b|); ~1e-3 of the outputs' RMS in the worst case measured, 1.4e-3 with one scale
 *   group per row at 256x the others' (numpy emulation).
 *   Requirements: d % 64 == 0, F % 64 == 0, F <= 16384; x, y, rows 16-byte aligned.
 *   workspace: moe_experts_workspace_bytes(...) bytes (any contents; every call writes what it reads). Calls
 *   sharing a workspace must be stream-ordered.
 */
int moe_experts_run(const moe_experts_t* w, const void* x, int x_dtype, const int32_t* idx, const float* wts, int T,
                    int k, int act, int path, int nored, void* y, int y_dtype, const void* residual, void* workspace,
                    size_t workspace_bytes, void* stream);
size_t moe_experts_workspace_bytes(const moe_experts_t* w, int T, int k, int path);

/*
 * moe_experts_run without a workspace argument: no counterpart in the reference. For callers that cannot
 * allocate (code under HIP graph capture, serving loops or harnesses that forbid allocation): the workspace is a
 * device array inside the library, MOE_STATIC_SCRATCH_BYTES on each GPU it runs on, held until the process ends.
 * Arguments, results and errors as moe_experts_run; calls whose workspace (moe_experts_workspace_bytes) exceeds
 * MOE_STATIC_SCRATCH_BYTES return MOE_ERR_WORKSPACE before any launch (the Qwen3-30B-A3B shape fits calls of up
 * to 110 tokens).
 * It allocates nothing. Every call on one GPU uses that GPU's one array, which keeps the last call's contents (no
 * call needs particular contents): calls that overlap on one GPU (other streams, other threads) race, and the
 * caller must order them. The first call on each device (the device of `stream`; the current device for the null
 * stream) looks up the array's address (hipGetSymbolAddress); make it outside graph capture: a call with T = 0 does
 * only that.
 */
#define MOE_STATIC_SCRATCH_BYTES ((size_t)32 << 20)
int moe_experts_run_static(const moe_experts_t* w, const void* x, int x_dtype, const int32_t* idx, const float* wts,
                           int T, int k, int act, int path, int nored, void* y, int y_dtype, const void* residual,
                           void* stream);

/*
 * The same call split at the one data dependency inside it, the GLU output h held in the workspace.
 * The reference dispatches these as separate kernels as well (metal_q4_decode_v4.py:177-184 _k1 gate_up,
 * _k2 down). stages = MOE_STAGE_GATE_UP: grouping (grouped path) + gate/up + GLU, h into the workspace;
 * MOE_STAGE_DOWN: down projection + combine from the h a previous GATE_UP call with the same arguments
 * left in the same workspace (stream-ordered); MOE_STAGE_ALL = both = moe_experts_run. Lets a caller
 * interleave other work between the two stages, or time each stage on its own stream.
 */
#define MOE_STAGE_GATE_UP 1
#define MOE_STAGE_DOWN 2
#define MOE_STAGE_ALL 3
int moe_experts_run_stages(const moe_experts_t* w, const void* x, int x_dtype, const int32_t* idx, const float* wts,
                           int T, int k, int act, int path, int nored, void* y, int y_dtype, const void* residual,
                           void* workspace, size_t workspace_bytes, int stages, void* stream);

/*
 * Router and experts in one call: moe_router's logits (same fixed order, so the same ids) and tail, then
 * moe_experts_run's default path. The reference calls them one after the other, the stock gate GEMV, router.topk_norm,
 * then the variant's run (reference e2e.py:57-64, moelab/router.py:71-80).
 *   T == 1: the router launch computes the logits only and every gate/up wave runs the tail over the 128..1024 logits
 *   itself for its own slot (no hand-off between workgroups inside a launch: measured at 1-2 us per round trip on this
 *   part); one wave writes idx / wts.
 *   T > 1: the router's two launches (as moe_router_group) compute the logits, run the tails and build the slot
 *   grouping and the expert kernels' pass lists, so the expert launches follow with no top-k or grouping launch of
 *   their own; where the gate/up wave tiles group the slots in-kernel (a few slots per expert) they do it there
 *   instead (one of their workgroups writes the lists for the down stage).
 *   x [T, d] bf16 (MOE_DTYPE_BF16 only: the gate GEMV reads bf16); wr [E, d] bf16, wr_bias [E] fp32 or NULL;
 *   norm, scale: as moe_router; idx [T, k] int32 and wts [T, k] fp32 out (as moe_router's); y, residual, act,
 *   y_dtype: as moe_experts_run. workspace: moe_layer_workspace_bytes(w, T, k) bytes (any contents).
 */
int moe_layer_run(const moe_experts_t* w, const void* x, int x_dtype, const void* wr, const float* wr_bias, int T,
                  int k, int norm, float scale, int act, int32_t* idx, float* wts, void* y, int y_dtype,
                  const void* residual, void* workspace, size_t workspace_bytes, void* stream);
size_t moe_layer_workspace_bytes(const moe_experts_t* w, int T, int k);

/*
 * moe_layer_run with S shared experts (the caller semantics of the reference's model patches, routed experts then the
 * shared module: e2e.py:57-68 Qwen-style gated shared expert, e2e.py:138-147 DeepSeek-V2): w holds E = E_r + S experts
 * as for moe_experts_run_shared (experts E_r .. E_r + S - 1 the shared ones), wr [E_r, d] routes over the first E_r.
 *   y[t] = residual[t] + sum_j wts[t,j] * expert_{idx[t,j]}(x_t) + g_t * sum_s expert_{E_r + s}(x_t),
 *   g_t = sigmoid(x_t . gate) (gate: bf16 [d], computed by the router launch as one more logit row, in the logits'
 *   fixed order) or 1 when gate is NULL. The router's launches write idx / wts [T, k] (the routed slots), the merged
 *   [T, k + S] slot lists and, at T > 1, their grouping; then the experts as moe_experts_run_shared.
 *   Limits: 1 <= S < E, E_r <= 1024, k <= min(E_r, 32), k + S <= 64.
 *   workspace: moe_layer_shared_workspace_bytes(w, S, T, k) bytes (any contents).
 */
int moe_layer_run_shared(const moe_experts_t* w, int S, const void* x, int x_dtype, const void* wr,
                         const float* wr_bias, const void* gate, int T, int k, int norm, float scale, int act,
                         int32_t* idx, float* wts, void* y, int y_dtype, const void* residual, void* workspace,
                         size_t workspace_bytes, void* stream);
size_t moe_layer_shared_workspace_bytes(const moe_experts_t* w, int S, int T, int k);

/*
 * Shared experts: S always-on experts added to every token, the caller semantics of the reference's model
 * patches (reference e2e.py:66-68 Qwen-style gated shared expert, sigmoid(x . w_gate) * shared_expert(x);
 * e2e.py:146-147 DeepSeek, + shared_experts(x)). The reference runs them as stock mlx-lm modules; here they go
 * through the same expert kernels as the routed experts:
 *   y[t] = residual[t] + g_t * sum_s ( down_s( act(gate_s x_t + bg_s, up_s x_t + bu_s) ) + bd_s ),
 *   g_t = sigmoid(x_t . gate) (gate: bf16 [d], fp32 dot in a fixed order) or 1 when gate is NULL.
 *   ws: the S shared experts as an expert set (E = S <= 32; same formats, packing and optional tile copies).
 *   x, y, residual, dtypes, act: as moe_experts_run (path auto: per-slot GEMV at T == 1, grouped tiles above).
 *   workspace: moe_shared_experts_workspace_bytes(ws, T) bytes (any contents), as for moe_experts_run.
 * A layer with routed and shared experts is moe_experts_run (routed, into y) followed by this call with
 * residual = y.
 */
int moe_shared_experts_run(const moe_experts_t* ws, const void* x, int x_dtype, int T, int act, const void* gate,
                           void* y, int y_dtype, const void* residual, void* workspace, size_t workspace_bytes,
                           void* stream);
size_t moe_shared_experts_workspace_bytes(const moe_experts_t* ws, int T);

/*
 * Routed and shared experts in one call (no counterpart in the reference, whose model patches run the shared
 * experts as a separate module after the routed ones, e2e.py:66-68 and 146-147): w holds E = E_r + S experts,
 * experts E_r .. E_r + S - 1 being the shared ones (same d, F, format and packing as the routed ones: the two
 * sets' rows concatenated, with tile copies packed over all E). Token t's slots are its k routed slots (idx, wts
 * as moe_experts_run; ids outside [0, E_r) join no group) followed by the S shared slots, expert E_r + s with
 * weight g_t = sigmoid(x_t . gate) (gate: bf16 [d]) or 1 when gate is NULL:
 *   y[t] = residual[t] + sum_j wts[t,j] * expert_{idx[t,j]}(x_t) + g_t * sum_s expert_{E_r + s}(x_t),
 * the experts and path as in moe_experts_run. One grouping, one combine, and the shared experts' work inside
 * the routed launches (the two-call form costs a second grouping, combine and slot-list launch, and runs the few
 * shared experts on grids too small to fill the chip). Limits: 1 <= S < E, k >= 1, k + S <= 64.
 *   workspace: moe_experts_shared_workspace_bytes(w, S, T, k, path) bytes (any contents).
 */
int moe_experts_run_shared(const moe_experts_t* w, int S, const void* x, int x_dtype, const int32_t* idx,
                           const float* wts, int T, int k, int act, int path, const void* gate, void* y, int y_dtype,
                           const void* residual, void* workspace, size_t workspace_bytes, void* stream);
size_t moe_experts_shared_workspace_bytes(const moe_experts_t* w, int S, int T, int k, int path);

/*
 * Read-bandwidth probe of the timing harness's contention guard (the reference's guard times a read-bound reduction,
 * moelab/guard.py:31-45): MOE_PROBE_SINK workgroups stream src [nbytes] (16-byte aligned, nbytes % 16 == 0) with
 * 16-byte loads, the expert kernels' weight-load pattern, and nothing else; workgroup b writes the XOR of the 32-bit
 * words it read to sink[b] (so the XOR of sink [MOE_PROBE_SINK] uint32 is the XOR of the buffer's words).
 */
#define MOE_PROBE_SINK 1024
int moe_probe_read(const void* src, size_t nbytes, uint32_t* sink, void* stream);

/* Library version and build target, for logs. */
const char* moe_version(void);

#ifdef __cplusplus
}
#endif
#endif /* MOE_MI355X_H */
