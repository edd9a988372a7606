/*
 * etmoe.h -- C ABI of the MI355X (gfx950) Expert-Threshold MoE token-dispatch
 * library, libetmoe.so.
 *
 * The path: per-expert threshold routing on sigmoid router scores with a
 * zero-expert fallback to argmax, an EMA threshold update, a histogram +
 * exclusive-scan CSR of expert offsets, a stable permutation of tokens into
 * expert-major slots (ordered by expert, then token id), the gate-weighted
 * un-permute ("combine"), and the backward of both (dX, dYp, dgate, and the
 * router-logit gradient).  Also the router producer that feeds the path: the
 * router-logits GEMM on the matrix cores, the same GEMM fused with routing,
 * and its backward (the router input gradient fused into dispatch backward,
 * and the router weight gradient).  And the consumer of the dispatch: the
 * expert grouped GEMM over the CSR slot blocks, with the dispatch gather
 * fused into its operand load.
 *
 * Reference interface.  The reference tree (bat0001/peer-review-agents) holds
 * no operator, plugin or FFI interface for this path -- its only extension
 * points are an agent-backend registry (cli/reva/backends.py:28-131) and a
 * log-translator table (cli/reva/translators/__init__.py:33-53).  So no entry
 * point below replaces a reference symbol; each says which step of the path it
 * implements, and the signatures are this library's own.
 *
 * Conventions (all entry points):
 *  - Every pointer argument is a DEVICE pointer unless its comment says
 *    otherwise.  Arrays are dense and row-major; activations have row stride d.
 *  - `stream` is a hipStream_t (NULL = the legacy default stream).  Calls only
 *    enqueue work; they never synchronise the stream and never allocate.
 *  - Return 0 on success, a negative ET_ERR_* code otherwise; et_last_error()
 *    then describes the failure (thread-local, valid until the next call on the
 *    same host thread).  Argument errors are detected before anything is
 *    enqueued.
 *  - Index arrays are int32: T*E must stay below 2^31.
 *  - `slot_capacity` is the allocated length of the slot arrays (sorted_token,
 *    slot_gate, token_slot, dgate) and the row count of the slot-major
 *    activation buffers (Xp, Yp, dYp, dXp).  T*E is always a sufficient
 *    capacity.  The number of routed slots S is expert_offsets[E] (also
 *    token_offsets[T]); compare it with the capacity after routing.  With an
 *    undersized capacity nothing is written out of bounds and data is lost:
 *    a routed pair is kept only if both its slot index and its entry in the
 *    token-major list are below the capacity.  The row kernels skip every
 *    other pair, so combine and dispatch backward sum the kept pairs only,
 *    dlogits is 0 at dropped pairs, and the rows of dropped slots below the
 *    capacity are left as they were (their dgate is 0 or left as it was).
 *  - Concurrent calls on different streams are safe when their buffers are
 *    disjoint.  One entry point holds device state: et_route_noalloc's static
 *    scratch (one per GPU, shared by its calls); every other entry point
 *    keeps none.
 */
#ifndef ETMOE_H
#define ETMOE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define ET_ABI_VERSION 11

/* activation dtypes */
#define ET_DTYPE_F32 0
#define ET_DTYPE_BF16 1

/* status codes */
#define ET_OK 0
#define ET_ERR_INVALID_ARGUMENT -1
#define ET_ERR_WORKSPACE_TOO_SMALL -2
#define ET_ERR_LAUNCH -3
#define ET_ERR_UNSUPPORTED -4

/* Largest expert count the routing kernels accept. */
#define ET_MAX_EXPERTS 1024

int et_abi_version(void);

/* Message of the last failed call on this host thread ("" if none). */
const char* et_last_error(void);

/* Bytes of device workspace et_route needs for T tokens and E experts: the
 * routed pairs of every 8-token group (8 * E entries of 8 bytes reserved per
 * group, about 8 * T * E bytes in all) plus per-group and per-tile counts.
 * Where that would pass 1 GiB (T * E above about 134 M), et_route runs the
 * two-read kernels instead (same outputs), and this is their workspace: per-
 * block counts, a few MB. */
size_t et_route_workspace_bytes(int64_t num_tokens, int64_t num_experts);

/*
 * Routing: threshold selection + histogram/scan CSR + stable permutation.
 *   logits         f32 [T, E]  router logits; score = sigmoid(logit)
 *   thr            f32 [E]     per-expert thresholds
 * Selection: (t, e) is routed iff score[t,e] >= thr[e]; a token with no such
 * expert is routed to argmax_e score[t,e] (NaN lowest, ties to the lowest e).
 * Outputs:
 *   counts         i32 [E]     tokens per expert
 *   expert_offsets i32 [E+1]   exclusive scan of counts (expert_offsets[E] = S)
 *   token_offsets  i32 [T+1]   exclusive scan of per-token expert counts
 *   sorted_token   i32 [cap]   slot -> token id, slots ordered by (expert, token)
 *   slot_gate      f32 [cap]   gate of each slot = its sigmoid score
 *   token_slot     i32 [cap]   token-major slot lists, ascending expert
 * Deterministic and atomics-free: repeated calls give identical bits.
 * Implements the routing step of the path (no reference counterpart).
 */
int et_route(const float* logits, const float* thr, int64_t num_tokens, int64_t num_experts,
             int32_t* counts, int32_t* expert_offsets, int32_t* token_offsets,
             int32_t* sorted_token, float* slot_gate, int32_t* token_slot,
             int64_t slot_capacity, void* workspace, size_t workspace_bytes, void* stream);

/* Size of the static device scratch of et_route_noalloc (bytes, per GPU). */
#define ET_ROUTE_NOALLOC_SCRATCH_BYTES ((size_t)8 << 20)

/*
 * Routing without a workspace argument and without any device allocation:
 * et_route with its workspace in a static device array of
 * ET_ROUTE_NOALLOC_SCRATCH_BYTES per GPU (held until the process ends), for
 * callers that cannot allocate: code under HIP graph capture, serving loops
 * and harnesses that forbid hipMalloc.  Arguments and outputs are those of
 * et_route (bit-identical results); the call runs on the current device, whose
 * scratch address it looks up once (on its first call there).  It runs the
 * two-read routing kernels (a count pass and a fill pass that both read the
 * logits), whose workspace is O(E) per block, not et_route's pair lists; sizes
 * whose two-read workspace exceeds the scratch are rejected with
 * ET_ERR_WORKSPACE_TOO_SMALL (every T fits for E <= 408).  All calls on
 * one GPU share the scratch: calls that overlap in time on one GPU (different
 * streams or host threads) race.
 * No counterpart in the reference: an extra entry point of this library.
 */
int et_route_noalloc(const float* logits, const float* thr, int64_t num_tokens, int64_t num_experts,
                     int32_t* counts, int32_t* expert_offsets, int32_t* token_offsets,
                     int32_t* sorted_token, float* slot_gate, int32_t* token_slot,
                     int64_t slot_capacity, void* stream);

/*
 * Dispatch (permute / scatter) forward:  Xp[slot, :] = X[token(slot), :].
 *   x  [T, d] of `dtype`,  xp [cap, d] of `dtype`.  Exact row copies.
 * Implements the dispatch step of the path (no reference counterpart).
 */
int et_dispatch_fwd(const void* x, int64_t num_tokens, int64_t d, int dtype,
                    const int32_t* token_offsets, const int32_t* token_slot,
                    int64_t slot_capacity, void* xp, void* stream);

/*
 * Combine (un-permute / gather) forward:
 *   Y[t, c] = cast(acc), acc = 0; for t's slots s in ascending expert order:
 *             acc = fma(slot_gate[s], Yp[s, c], acc)      (binary32)
 *   yp [cap, d], y [T, d] of `dtype`.  Bit-exact with that definition.
 * Implements the combine step of the path (no reference counterpart).
 */
int et_combine_fwd(const void* yp, const float* slot_gate, const int32_t* token_offsets,
                   const int32_t* token_slot, int64_t num_tokens, int64_t d, int dtype,
                   int64_t slot_capacity, void* y, void* stream);

/* Bytes of device workspace et_combine_bwd needs when a row is a whole number
 * of 16-byte chunks (else 0): slot_capacity * ceil(ceil(d * elem / 1024) / 2)
 * doubles of partial dot products (one per 2 KiB of the row), then, from the
 * next 256-byte boundary, the slot walk order (slot_capacity int32).
 * num_tokens does not enter.  The workspace must be 8-byte aligned. */
size_t et_combine_bwd_workspace_bytes(int64_t num_tokens, int64_t slot_capacity, int64_t d, int dtype);

/*
 * Combine backward (fused): for every slot s of token t = token(s), expert e:
 *   dYp[s, c]     = cast(slot_gate[s] * dY[t, c])
 *   dgate[s]      = sum_c dY[t, c] * Yp[s, c], accumulated in binary64 (every
 *                   product is exact there) and rounded once to binary32
 *   dlogits[t, e] = dgate[s] * (g * (1 - g)) in binary32, g = slot_gate[s];
 *                   0 elsewhere
 * dlogits (f32 [T, E]) may be NULL.
 * workspace holds the per-piece partial dot products and the slot walk order
 * (et_combine_bwd_workspace_bytes); it may be NULL when that size is 0.
 * Implements the combine backward of the path (no reference counterpart).
 */
int et_combine_bwd(const void* dy, const void* yp, const float* slot_gate,
                   const int32_t* sorted_token, const int32_t* token_offsets,
                   const int32_t* token_slot, const int32_t* expert_offsets,
                   int64_t num_tokens, int64_t num_experts, int64_t d, int dtype,
                   int64_t slot_capacity, void* dyp, float* dgate, float* dlogits,
                   void* workspace, size_t workspace_bytes, void* stream);

/*
 * Dispatch backward:  dX[t, c] = cast(sum of dXp[s, c] over t's slots, added in
 * ascending expert order in binary32).  dxp [cap, d], dx [T, d] of `dtype`.
 * Implements the dispatch backward of the path (no reference counterpart).
 */
int et_dispatch_bwd(const void* dxp, const int32_t* token_offsets, const int32_t* token_slot,
                    int64_t num_tokens, int64_t d, int dtype, int64_t slot_capacity,
                    void* dx, void* stream);

/* Bytes of device workspace et_dispatch_bwd_router needs (8 per slot of capacity). */
size_t et_dispatch_bwd_router_workspace_bytes(int64_t slot_capacity);

/*
 * Dispatch backward plus the router's input gradient, one pass:
 *   dX[t, c] = cast(acc), acc = 0; for t's slots s in ascending expert order, e = e(s):
 *       acc = acc + dXp[s, c];   acc = fma(dl(s), W[e, c], acc)          (binary32)
 *   dl(s) = dgate[s] * (g * (1 - g)), g = slot_gate[s]  -- the dlogits[t, e]
 *   entry of et_combine_bwd, so dX = dispatch backward + dlogits . W.
 *   w_router [E, d] is the router weight, in the dtype of dxp/dx.  dgate is
 *   et_combine_bwd's output.  expert_offsets gives each slot's expert.
 * Implements the dispatch backward fused with the router producer's input
 * gradient (no reference counterpart).
 */
int et_dispatch_bwd_router(const void* dxp, const int32_t* token_offsets, const int32_t* token_slot,
                           int64_t num_tokens, int64_t d, int dtype, int64_t slot_capacity,
                           const float* slot_gate, const float* dgate, const int32_t* expert_offsets,
                           int64_t num_experts, const void* w_router, void* dx, void* workspace,
                           size_t workspace_bytes, void* stream);

/* Bytes of device workspace et_threshold_update needs for T tokens and E experts
 * (it holds room for T*E candidate keys, of which a selected digit bin's few
 * are written, and the per-block digit histograms: about 4*T*E bytes). */
size_t et_threshold_workspace_bytes(int64_t num_tokens, int64_t num_experts);

/*
 * EMA threshold update, in place on thr (f32 [E]):
 *   stat[e] = the c-th largest score of expert e's column, c = ceil(T*k/E)
 *             clamped to [1, T] (NaN scores order as 0)
 *   thr[e]  = fma(momentum, thr[e], (1 - momentum) * stat[e])
 * stat (f32 [E]) may be NULL.  T == 0 leaves thr unchanged.  Exact selection
 * (a histogram of the scores' digits floor(score * 256), then a radix select
 * over the score bits of the selected digit's keys), so thr is bit-exact with
 * the definition.
 * Implements the EMA threshold update of the path (no reference counterpart).
 */
int et_threshold_update(const float* logits, float* thr, int64_t num_tokens, int64_t num_experts,
                        int64_t k_target, float momentum, float* stat,
                        void* workspace, size_t workspace_bytes, void* stream);

/*
 * Routing and the EMA threshold update of one training batch in one call:
 * the results of et_route (with the thresholds from before the update)
 * followed by et_threshold_update, bit for bit, with every kernel on
 * `stream`.  Where et_route takes its pair lists (up to 256 experts), the
 * update's small passes run in the routing's launches (histogram; count with
 * the bin select; scan with the collect pass; place with the final select):
 * four launches for the two calls' seven (five below 32768 tokens).
 * Workspaces: route_workspace as et_route's, thr_workspace as
 * et_threshold_update's; their byte ranges must not overlap
 * (ET_ERR_INVALID_ARGUMENT).
 * Composes et_route and et_threshold_update (no reference counterpart).
 */
int et_route_update(const float* logits, float* thr, int64_t num_tokens, int64_t num_experts,
                    int32_t* counts, int32_t* expert_offsets, int32_t* token_offsets,
                    int32_t* sorted_token, float* slot_gate, int32_t* token_slot, int64_t slot_capacity,
                    void* route_workspace, size_t route_workspace_bytes,
                    int64_t k_target, float momentum, float* stat,
                    void* thr_workspace, size_t thr_workspace_bytes, void* stream);

/* Largest expert count of the router GEMM (all experts of a token tile are
 * accumulated in registers). */
#define ET_MAX_ROUTER_EXPERTS 256

/*
 * Router logits (the producer of et_route's input):
 *   logits[t, e] = sum_k x[t, k] * w[e, k]        (f32 out, binary32 accumulate)
 *   x bf16 [T, d], w bf16 [E, d] (the router weight in nn.Linear layout),
 *   16-byte aligned; d a multiple of 8 below 2^22; 1 <= E <= ET_MAX_ROUTER_EXPERTS.
 * Products of bf16 values are exact in binary32; the sum over k runs in a
 * fixed order, in k-steps of 16 ascending from k0(t) = (floor(t / 256) mod 4) *
 * 64 * floor(d / 256) and wrapping to 0 (staggered so that concurrent blocks
 * read different column ranges of X).  So repeated calls give identical bits,
 * and integer-valued inputs whose partial sums stay below 2^24 give the exact
 * integer result.
 * Implements the router producer that feeds the path (no reference counterpart).
 */
int et_router_logits(const void* x, const void* w, int64_t num_tokens, int64_t d, int64_t num_experts,
                     float* logits, void* stream);

/* Bytes of device workspace et_router_wgrad needs (per-split partial dW tiles;
 * 0 for invalid sizes). */
size_t et_router_wgrad_workspace_bytes(int64_t num_tokens, int64_t d, int64_t num_experts);

/*
 * Router weight gradient:  dw[e, c] = sum_t dlogits[t, e] * x[t, c]  (f32 [E, d])
 *   dlogits f32 [T, E] (et_combine_bwd's output), x bf16 [T, d] (16-byte
 *   aligned, d a multiple of 8 below 2^22, T*d below 2^30, T*E below 2^29).
 * On the matrix cores with dl split into two bf16 terms (hi + lo, ~16 bits
 * more than bf16), binary32 accumulation; the token sum is split over blocks
 * and the partials are added in a fixed order, so repeated calls give
 * identical bits.  Exact for integer-valued inputs whose sums stay below 2^24.
 * Implements the router producer's weight gradient (no reference counterpart).
 */
int et_router_wgrad(const float* dlogits, const void* x, int64_t num_tokens, int64_t d, int64_t num_experts,
                    float* dw, void* workspace, size_t workspace_bytes, void* stream);

/* Bytes of device workspace et_router_route needs for T tokens and E experts
 * (0 if E is outside [1, ET_MAX_ROUTER_EXPERTS]). */
size_t et_router_route_workspace_bytes(int64_t num_tokens, int64_t num_experts);

/*
 * Fused router producer + routing: the router GEMM of et_router_logits with the
 * selection of et_route applied to the logits in registers, so the [T, E]
 * score matrix is never written (only the routed pairs' gates pass through
 * the workspace).  All outputs are bit-identical to
 *     et_router_logits(x, w) -> logits;  et_route(logits, thr, ...)
 * with the same slot_capacity.  `logits` (f32 [T, E]) may be NULL; if given,
 * the logits are written as well (for an EMA threshold update on this batch).
 * Arguments as et_router_logits and et_route.
 * Implements the router producer fused with the routing step (no reference
 * counterpart).
 */
int et_router_route(const void* x, const void* w, const float* thr, int64_t num_tokens, int64_t d,
                    int64_t num_experts, int32_t* counts, int32_t* expert_offsets, int32_t* token_offsets,
                    int32_t* sorted_token, float* slot_gate, int32_t* token_slot, int64_t slot_capacity,
                    float* logits, void* workspace, size_t workspace_bytes, void* stream);

/* Epilogues of et_expert_gemm. */
#define ET_GEMM_PLAIN 0      /* c = the product                                      */
#define ET_GEMM_ROW_SCALE 1  /* c[s, :] = row_scale[s] * the product (binary32)      */
#define ET_GEMM_SWIGLU 2     /* c[s, f] = (g * sigmoid(g)) * u, g = product column f,
                                u = product column F + f, F = N / 2 (binary32)       */

/*
 * Expert grouped GEMM over the routing CSR (the expert FFN's projections):
 *   p[s, n] = sum_k a[row(s), k] * w[e(s), n, k]   (bf16 operands, binary32
 *                                                   accumulation)
 * for every slot s below min(expert_offsets[E], slot_capacity), e(s) the
 * expert whose block [expert_offsets[e], expert_offsets[e + 1]) holds s, and
 * c[s, :] = the epilogue of p[s, :], rounded once to bf16.
 *   sorted_token != NULL (gather mode): row(s) = sorted_token[s] and a is the
 *       token matrix X bf16 [a_rows = T, K] -- the dispatch fused into the
 *       operand load, so Xp is never written;
 *   sorted_token == NULL: row(s) = s and a is slot-major bf16
 *       [slot_capacity, K] (a_rows is ignored).
 *   w bf16 [E, N, K]: expert e's weight in nn.Linear layout (row n = output
 *       feature n).  c bf16 [slot_capacity, N], or [slot_capacity, N / 2] for
 *       ET_GEMM_SWIGLU, whose weight holds the gate rows then the up rows.
 *   row_scale f32 [slot_capacity] (ET_GEMM_ROW_SCALE only; may be NULL
 *       otherwise), e.g. slot_gate: a per-slot factor commutes with the sum.
 *   sigmoid is the one routing uses (one exp of -|g|, one division).
 * K a multiple of 8 below 2^22, N a multiple of 8 (of 16 for SwiGLU),
 * N*K*2 below 2^31 bytes; in gather mode a_rows*K*2 below 2^31 bytes.  a, w
 * and c 16-byte aligned.  Rows of c past the routed slots are left as they
 * were.  Every output sums its k-steps of 16 in ascending k (each k-step
 * inside one MFMA), so the gather and slot-major modes give identical bits,
 * repeated calls give identical bits, and integer-valued inputs whose partial
 * sums stay below 2^24 give the exact product before the epilogue.
 * Implements the expert grouped GEMM that consumes the dispatch (no reference
 * counterpart).
 */
int et_expert_gemm(const void* a, int64_t a_rows, const int32_t* sorted_token, const void* w,
                   const int32_t* expert_offsets, int64_t num_experts, int64_t K, int64_t N,
                   int64_t slot_capacity, int epilogue, const float* row_scale, void* c, void* stream);

/*
 * The expert grouped GEMM on fp8 operands, on gfx950's fp8 matrix cores (twice
 * the bf16 rate):
 *   c[s, n] = ((sum_k a[row(s), k] * w[e(s), n, k]) * a_scale[row(s)]) * w_scale[e(s), n]
 * with a and w in OCP fp8 e4m3 (one byte per element), their products summed
 * in binary32 in ascending k-steps of 64 (one MFMA each, unit block scales),
 * the two scale products rounded in the order written, and one rounding to
 * bf16.  row(s), the modes (gather with sorted_token, or slot-major with
 * NULL), slot_capacity and the output are those of et_expert_gemm; a_scale
 * [a_rows] f32 scales each row of a (a token in gather mode), w_scale [E, N]
 * f32 each weight row.  epilogue: ET_GEMM_PLAIN or ET_GEMM_SWIGLU (h =
 * (g * sigmoid(g)) * u of the scaled gate and up values).  K a multiple of 16
 * below 2^22, N a multiple of 8 (16 for SwiGLU), N*K below 2^31; a, w and c
 * 16-byte aligned, a_scale and w_scale 4-byte aligned.  Integer-valued operands
 * with power-of-two scales and partial sums below 2^24 give the exact
 * product before the bf16 rounding.  Implements an fp8 form of the expert
 * GEMM that consumes the dispatch (no reference counterpart).
 */
int et_expert_gemm_fp8(const void* a, int64_t a_rows, const float* a_scale, const int32_t* sorted_token,
                       const void* w, const float* w_scale, const int32_t* expert_offsets, int64_t num_experts,
                       int64_t K, int64_t N, int64_t slot_capacity, int epilogue, void* c, void* stream);

/*
 * Weight transpose for the expert GEMM's input gradient:
 *   wt[e, k, n] = w[e, n, k]   (bf16, exact copies)
 * for every expert with at least one slot below slot_capacity (the others are
 * left as they were).  With it, dA = dC . W_e -- the input gradient of
 * c = a . W_e^T -- is et_expert_gemm(dC, wt) (K' = N, N' = K).  N and K
 * multiples of 8, N*K below 2^31; w and wt 16-byte aligned, not aliased.
 * Implements the layout change the expert GEMM's backward needs (no reference
 * counterpart).
 */
int et_expert_weight_transpose(const void* w, const int32_t* expert_offsets, int64_t num_experts,
                               int64_t N, int64_t K, int64_t slot_capacity, void* wt, void* stream);

/*
 * Weight gradient of the expert GEMM:
 *   dw[e, n, k] = sum over e's slots s (s < slot_capacity) of dc[s, n] * a[s, k]
 * dc bf16 [slot_capacity, N] (the gradient of c), a bf16 [slot_capacity, K]
 * slot-major (the operand of the forward product; dispatch(X) for a gathered
 * forward), dw f32 [E, N, K]; experts without slots get zeros.  Binary32
 * accumulation on the matrix cores over the slots in ascending order, in steps
 * of 16 (one MFMA each): repeated calls give identical bits, and integer-valued
 * inputs whose partial sums stay below 2^24 give the exact result.  N and K
 * multiples of 8, N*K*4 below 2^31 bytes; dc and a 16-byte aligned.
 * Implements the expert GEMM's weight gradient (no reference counterpart).
 */
int et_expert_wgrad(const void* dc, const void* a, const int32_t* expert_offsets, int64_t num_experts,
                    int64_t N, int64_t K, int64_t slot_capacity, float* dw, void* stream);

/*
 * SwiGLU of the expert FFN, element-wise over the routed slots
 * s < min(expert_offsets[E], slot_capacity), j < F:
 *   et_swiglu_fwd:  h[s, j] = (g * sigmoid(g)) * u
 *   et_swiglu_bwd:  dgu[s, j]     = (dh * u) * (sigmoid(g) * (1 + g * (1 - sigmoid(g))))
 *                   dgu[s, F + j] = dh * (g * sigmoid(g))
 * with g = gu[s, j], u = gu[s, F + j], dh = dh[s, j].  gu bf16 [slot_capacity,
 * 2F] is the gate/up projection's output (et_expert_gemm without epilogue:
 * gate rows of the weight first), h and dh bf16 [slot_capacity, F], dgu bf16
 * [slot_capacity, 2F].  Binary32 arithmetic, each operation rounded in the
 * order written (no fused multiply-add), the routing's sigmoid; one rounding
 * to bf16 per output.  The forward gives the same bits as the
 * ET_GEMM_SWIGLU epilogue applied to the rounded gu (the epilogue itself works
 * on the unrounded accumulators).  Rows past the routed slots are left as they
 * were; the slot count is read on the device (no host synchronisation).  F a
 * multiple of 8; every pointer 16-byte aligned.  Implements the expert FFN's
 * activation for training, where gu is kept for the backward (no reference
 * counterpart).
 */
int et_swiglu_fwd(const void* gu, int64_t F, const int32_t* expert_offsets, int64_t num_experts,
                  int64_t slot_capacity, void* h, void* stream);
int et_swiglu_bwd(const void* gu, const void* dh, int64_t F, const int32_t* expert_offsets,
                  int64_t num_experts, int64_t slot_capacity, void* dgu, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* ETMOE_H */
