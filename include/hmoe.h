/*
 * hmoe: C ABI of the MI355X-native (gfx950) mixture-of-experts SwiGLU layer.
 *
 * Every entry point takes device pointers, sizes and a HIP stream (as void*), is asynchronous on that stream,
 * never synchronises the device, never reads data back to the host and never allocates: the caller allocates
 * outputs and any workspace (sized by the matching *_workspace_size query).  Return value 0 = success, negative =
 * an HMOE_ERR_* code (hmoe_error_string gives the text).  Element types are passed as HMOE_DT_* codes.
 *
 * Conventions shared with the reference (adamo1139/trenowanie_generatora_obrazkow):
 *   - flat routed row f = token * k + slot (topk_ids.reshape(-1), aurora/hf_compat.py:70);
 *   - sorted row r: rows grouped by expert in expert order, stable in f (argsort(stable=True), :71);
 *     order[r] = f, a_idx[r] = f / k, y_idx[r] = f (:78), inv_pos[f] = r;
 *   - stacked expert weights wgu (E, d, 2h) = [gate | up] and wd (E, h, d), N contiguous (:154-155);
 *   - 16-bit storage, fp32 accumulation, one rounding on store; the routing weight is rounded to the activations'
 *     type before use (:80) and applied to the fp32 accumulator (aurora/moe_triton.py:52-56).
 * Activation types: the forward entry points (dispatch, the gate/up and down projections, grouped_mm, combine) take
 * bf16 or fp16 activations, selected by a `dtype` argument (HMOE_DT_BF16 / HMOE_DT_F16) that also types their 16-bit
 * weights, 16-bit row scales and outputs -- the reference's grouped_mm returns a.dtype for any floating input
 * (aurora/moe_triton.py:80) and its LM loader takes a dtype (aurora/hf_compat.py:42).  fp16 runs on
 * v_mfma_f32_32x32x16_f16 with fp16 rounding points in place of bf16 ones.  The routers and the backward are bf16.
 * Row offsets are 64-bit.  Index arrays (a_idx, y_idx, ...) are trusted to be in range.
 */
#ifndef HMOE_H_
#define HMOE_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define HMOE_ABI_VERSION 2

#define HMOE_OK 0
#define HMOE_ERR_ARG (-1)       /* null pointer, negative size, misaligned pointer or leading dimension */
#define HMOE_ERR_SHAPE (-2)     /* shape the kernels do not support (e.g. K or N not a multiple of 8) */
#define HMOE_ERR_DTYPE (-3)     /* element type not supported for this argument */
#define HMOE_ERR_LAUNCH (-4)    /* hipGetLastError reported a launch failure */
#define HMOE_ERR_WORKSPACE (-5) /* workspace missing or smaller than the *_workspace_size query */
#define HMOE_ERR_DEVICE (-6)    /* device query failed */
#define HMOE_ERR_TOO_LARGE (-7) /* input beyond the fixed device scratch of an allocation-free entry point */

#define HMOE_DT_BF16 0
#define HMOE_DT_F16 1
#define HMOE_DT_F32 2
#define HMOE_DT_I32 3
#define HMOE_DT_I64 4
#define HMOE_DT_I8 5

typedef void* hmoe_stream_t; /* a hipStream_t (0 = the null stream) */

int hmoe_abi_version(void);
const char* hmoe_error_string(int code);

/* ---------------------------------------------------------------------------------------------------------------
 * Routing
 * ------------------------------------------------------------------------------------------------------------- */

/* Softmax top-k router.  No counterpart in the reference's own code: its production gate is remote HF code
 * (aurora/hf_compat.py:49-51); conventions follow aurora/hf_pipeline.py:352-359 (fp32 logits of
 * F.linear(x.float(), W.float()), top-k, w / (sum + 1e-20) * scaling).
 * x (T, d) bf16 with row stride ldx, wr (E, d) bf16, bias (E,) fp32 or NULL.  Outputs topk_ids (T, k) int32 and
 * topk_w (T, k) fp32 (slots in descending order, ties to the lower expert), logits (T, E) fp32 (NULL to skip).
 * Each logit is a fixed-order fp32 sum, so ids, weights and logits are bit-reproducible by a host restatement: the
 * row in 64-element blocks, block b feeding fma chain b % 4 (each from +0, its blocks in order, step s of block b
 * taking elements 64b + 16q + s for q = 0..3), logit = (c0 + c1) + (c2 + c3), plus the bias (one rounded addition).
 * With E > 16, T * E <= 2^18 and a logits buffer, the logits are first written there per (16 tokens, 16 experts)
 * block and the selection then reads them (two launches spread over the chip; the same results): passing logits is
 * faster for small inputs even when they are not needed.  d % 8 == 0, E <= 256, k <= 16. */
int hmoe_route_topk(const void* x, int64_t ldx, const void* wr, const float* bias, int64_t T, int64_t d, int E,
                    int k, int renorm, float scaling, float* logits, int32_t* topk_ids, float* topk_w,
                    hmoe_stream_t stream);

/* Sigmoid, group-limited top-k router of BailingMoeV2: replaces the routing of aurora/hf_pipeline.py:352-359
 * (PoziomkaMoE.forward).  Logits in fp32, each the fixed-order sum of hmoe_route_topk (no bias in them);
 * score = 1 / (1 + exp(-logit)) (the exp of the softmax router, IEEE division); routing = score + expert_bias (fp32,
 * NULL = 0) for selection only; the experts form n_group groups of E / n_group, a group's value is the sum of its two
 * largest routing values, the topk_group best groups are kept (ties to the lower group) and the k best experts among
 * them selected (descending, ties to the lower expert); topk_w = selected scores / (their sum in slot order + 1e-20)
 * * scaling.  scores (T, E) fp32 receives the sigmoid scores (NULL to skip; for T * E <= 2^18 the logits pass
 * through it as in hmoe_route_topk, so passing it is faster for small inputs).  E % n_group == 0; unless
 * topk_group >= n_group (every group kept), E / n_group is a power of two in [2, 64] and k <= topk_group *
 * E / n_group.  Other limits as hmoe_route_topk. */
int hmoe_route_sigmoid_group(const void* x, int64_t ldx, const void* wr, const float* expert_bias, int64_t T,
                             int64_t d, int E, int k, int n_group, int topk_group, float scaling, float* scores,
                             int32_t* topk_ids, float* topk_w, hmoe_stream_t stream);

/* Workspace bytes for hmoe_dispatch. */
size_t hmoe_dispatch_workspace_size(int64_t T, int k, int E);

/* Token dispatch: replaces aurora/hf_compat.py:69-72 (flat ids, stable argsort, bincount), :78 (a_idx, y_idx),
 * :80 (routing weight in sorted order, rounded to bf16) and the row gather x[order // k] of :83.
 * topk_ids (T, k) int32 or int64 (ids_dtype), topk_w (T, k) fp32 or bf16 (w_dtype; NULL to skip w_sorted).
 * Outputs (NULL skips an optional one): counts (E,) int32 [required], counts64 (E,) int64, starts (E+1,) int32
 * [required; starts[e] = first sorted row of expert e], order (M,) int32 (= y_idx), a_idx (M,) int32,
 * inv_pos (M,) int32, w_sorted (M,) bf16, xs (M, d) bf16 = x[a_idx] (needs x (T, d) bf16 with row stride ldx),
 * n_invalid (1,) int32.  dtype: the 16-bit type of x / xs and of w_sorted (topk_w, fp32, bf16 or fp16, is rounded
 * to it).
 * Expert ids outside [0, E) route nowhere: their flat rows are counted in no expert and get inv_pos = -1, the
 * Sigma counts sorted rows hold the valid ones (the sorted rows past that are not written), and n_invalid receives
 * how many there are (on the device, no host sync: the caller reads it when it chooses).  hmoe_combine with inv_pos
 * then adds zeros for those slots and hmoe_unpermute_bwd skips them, so the layer's output is defined (the slot
 * contributes nothing).  The reference leaves such ids undefined (torch.bincount raises on negative ones and grows
 * the count array for ids >= E, aurora/hf_compat.py:72).  E <= 1024. */
int hmoe_dispatch(const void* topk_ids, int ids_dtype, const void* topk_w, int w_dtype, int64_t T, int k, int E,
                  const void* x, int64_t ldx, int64_t d, void* xs, int32_t* counts, int64_t* counts64,
                  int32_t* starts, int32_t* order, int32_t* a_idx, int32_t* inv_pos, uint16_t* w_sorted,
                  int32_t* n_invalid, void* workspace, size_t workspace_bytes, int dtype, hmoe_stream_t stream);

/* Bytes of the row-group tiles (xs_tiles) for M sorted rows of width d over E experts (an upper bound: it does not
 * depend on the counts).  0 for invalid sizes. */
size_t hmoe_xs_tiles_bytes(int64_t M, int E, int64_t d);

/* hmoe_dispatch that can also write the permuted rows as row-group tiles (xs_tiles, NULL to skip;
 * hmoe_xs_tiles_bytes(T * k, E, d) bytes, 16-byte aligned), the A operand of hmoe_gate_up_swiglu_tiles: the gather
 * x[order // k] of aurora/hf_compat.py:83 in a layout for the gate/up GEMM's copies.  Layout: the sorted rows of
 * expert e form groups of 128 rows (the last partial), expert e's first group being the sum over e' < e of
 * ceil(count[e'] / 128); group g and 32-column slice s occupy the 8 KB at byte (g * ceil(d / 32) + s) * 8192; row r
 * of a group at r * 64 within it, its 16-byte chunk c (columns 32 s + 8 c ..) at chunk position c ^ ((r >> 2) & 3).
 * Positions of rows or columns that do not exist are not written.  Other arguments as hmoe_dispatch. */
int hmoe_dispatch_tiles(const void* topk_ids, int ids_dtype, const void* topk_w, int w_dtype, int64_t T, int k, int E,
                        const void* x, int64_t ldx, int64_t d, void* xs, void* xs_tiles, int32_t* counts,
                        int64_t* counts64, int32_t* starts, int32_t* order, int32_t* a_idx, int32_t* inv_pos,
                        uint16_t* w_sorted, int32_t* n_invalid, void* workspace, size_t workspace_bytes, int dtype,
                        hmoe_stream_t stream);

/* Allocation-free form of hmoe_dispatch.  No counterpart in the reference: it is for callers that cannot allocate
 * (code under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc).  Same arguments, checks and
 * outputs as hmoe_dispatch, without the workspace: the kernels use a fixed device array of 8 MiB inside the library
 * (one per GPU, held until the process ends), so the call allocates nothing.  Inputs whose workspace
 * (hmoe_dispatch_workspace_size(T, k, E)) exceeds 8 MiB are refused with HMOE_ERR_TOO_LARGE before any launch
 * (about 1.9 million routed rows T * k at E <= 16; C3 needs 136 KiB).  Every call on a GPU shares that GPU's array: calls
 * that overlap in time on one GPU (other streams, other host threads) race and must be serialised by the caller.
 * Each call writes every scratch entry it reads, so no state carries over between calls. */
int hmoe_dispatch_noalloc(const void* topk_ids, int ids_dtype, const void* topk_w, int w_dtype, int64_t T, int k,
                          int E, const void* x, int64_t ldx, int64_t d, void* xs, int32_t* counts, int64_t* counts64,
                          int32_t* starts, int32_t* order, int32_t* a_idx, int32_t* inv_pos, uint16_t* w_sorted,
                          int32_t* n_invalid, int dtype, hmoe_stream_t stream);

/* make_schedule: replaces aurora/moe_triton.py:93-107.  For each of the ceil(M / block_m) + E blocks: the expert
 * (or -1), the first sorted row and the end row of that expert, int32, computed on the device from counts
 * (int32 or int64).  E <= 1024. */
int hmoe_make_schedule(const void* counts, int counts_dtype, int E, int64_t M, int block_m, int32_t* block_e,
                       int32_t* block_row, int32_t* row_end, hmoe_stream_t stream);

/* ---------------------------------------------------------------------------------------------------------------
 * Grouped GEMMs (bf16 MFMA, fp32 accumulation, persistent tile scheduler over ragged expert groups)
 * Every grouped GEMM takes E <= 1024 experts and M < 2^31 sorted rows (HMOE_ERR_SHAPE otherwise).
 * ------------------------------------------------------------------------------------------------------------- */

/* grouped_mm: replaces aurora/moe_triton.py:65-90 (_grouped_kernel :22-56).
 * y[y_idx[r] or r, :] = bf16((a[a_idx[r] or r, :] @ w[e(r)]) * w_scale[e, :] * scale[r]) for the M sorted rows r,
 * e(r) the expert owning row r under counts, the two scale products in that order on the fp32 sum.  a bf16 or fp16
 * (a_dtype; rows of lda elements), w (E, K, N) with element strides (stride_we, stride_wk, 1): a's type (w_scale
 * NULL) or int8 (HMOE_DT_I8, weight-only quantisation of aurora/moe_triton.py:44-51: w_scale (E, N) bf16 or fp32
 * required, N, stride_wk and stride_we multiples of 16); scale (M,) fp32 or a's type, or NULL; y of a's type with
 * row stride ldy.
 * K % 8 == 0, N % 8 == 0, lda/ldy/stride_wk % 8 == 0.  Rows of y not named by the schedule are not written. */
int hmoe_grouped_mm(const void* a, int64_t lda, int a_dtype, const void* w, int w_dtype, int64_t E, int64_t K,
                    int64_t N, int64_t stride_we, int64_t stride_wk, const void* counts, int counts_dtype, int64_t M,
                    const int32_t* a_idx, const int32_t* y_idx, const void* scale, int scale_dtype,
                    const void* w_scale, int w_scale_dtype, void* y, int64_t ldy, hmoe_stream_t stream);

/* Gate/up projection with the SwiGLU fused into the epilogue: replaces aurora/hf_compat.py:79 (grouped_mm(x,
 * _wgu, counts, sched, a_idx=a_idx).chunk(2)) and the self._act(g) * u of :81.
 * A rows: xs (M, d) in sorted order (a_idx NULL) or x (T, d) gathered through a_idx.  wgu (E, d, 2h).
 * act (M, h) = R(R(silu(g)) * u) with g, u the rounded gate / up outputs, R the rounding to dtype (bf16 or fp16, the
 * type of x, wgu, act and gu); gu (M, 2h) = [g | u] when not NULL (kept for the backward).  d % 8 == 0,
 * h % 8 == 0. */
int hmoe_gate_up_swiglu(const void* x, int64_t ldx, const int32_t* a_idx, const void* wgu, int64_t E, int64_t d,
                        int64_t h, const void* counts, int counts_dtype, int64_t M, void* act, void* gu, int dtype,
                        hmoe_stream_t stream);

/* hmoe_gate_up_swiglu with the A rows taken from the row-group tiles of hmoe_dispatch_tiles (xs_tiles, written by
 * a dispatch with the same counts, d and M): the same products and sums, so act and gu are identical; the copies of
 * the GEMM then read 1 KB runs instead of 64-byte row pieces.  hmoe_xs_tiles_bytes(M, E, d) below 2^31. */
int hmoe_gate_up_swiglu_tiles(const void* xs_tiles, const void* wgu, int64_t E, int64_t d, int64_t h,
                              const void* counts, int counts_dtype, int64_t M, void* act, void* gu, int dtype,
                              hmoe_stream_t stream);

/* Down projection with routing weight and scatter: replaces aurora/hf_compat.py:80-81 (grouped_mm(act, _wd,
 * counts, sched, y_idx=y_idx, scale=w)).  y[y_idx[r]] = R(fp32(act[r] @ wd[e]) * w_sorted[r]); yhat (M, d)
 * = R(act[r] @ wd[e]) in sorted order when not NULL (kept for the backward); act, wd, w_sorted, y and yhat of type
 * dtype (bf16 or fp16), R the rounding to it. */
int hmoe_down_scatter(const void* act, const void* wd, int64_t E, int64_t h, int64_t d, const void* counts,
                      int counts_dtype, int64_t M, const uint16_t* w_sorted, const int32_t* y_idx, void* y,
                      void* yhat, int dtype, hmoe_stream_t stream);

/* int8-weight forms of the two fused projections: replace aurora/hf_compat.py:79-80 on a layer fused with
 * quant="int8" (weights and scales from aurora/hf_compat.py:106-110, the kernel's int8 branch at
 * aurora/moe_triton.py:44-51).  wgu_q (E, d, 2h) int8 with scales wgu_s (E, 2h); wd_q (E, h, d) int8 with scales
 * wd_s (E, d); scales bf16 or fp32 (*_s_dtype).  Same outputs as hmoe_gate_up_swiglu / hmoe_down_scatter with the
 * per-column scale applied to the fp32 sum before any other step (inference only: no gu / yhat); activations,
 * w_sorted and outputs of type dtype (bf16 or fp16; int8 widens exactly to either).  h % 16 == 0 and d % 16 == 0. */
int hmoe_gate_up_swiglu_i8(const void* x, int64_t ldx, const int32_t* a_idx, const void* wgu_q, const void* wgu_s,
                           int wgu_s_dtype, int64_t E, int64_t d, int64_t h, const void* counts, int counts_dtype,
                           int64_t M, void* act, int dtype, hmoe_stream_t stream);
int hmoe_down_scatter_i8(const void* act, const void* wd_q, const void* wd_s, int wd_s_dtype, int64_t E, int64_t h,
                         int64_t d, const void* counts, int counts_dtype, int64_t M, const uint16_t* w_sorted,
                         const int32_t* y_idx, void* y, int dtype, hmoe_stream_t stream);

/* Combine: replaces aurora/hf_compat.py:82 (y.view(n, k, -1).sum(1)): out[t] = R(sum_j fp32(y[t*k + j])), y and
 * out of type dtype (bf16 or fp16), R the rounding to it.
 * inv_pos (T * k,) int32 from the dispatch, or NULL: slots with a negative inv_pos (expert ids outside [0, E)) are
 * read as zeros instead of their (unwritten) row of y. */
int hmoe_combine(const void* y, const int32_t* inv_pos, int64_t T, int k, int64_t d, void* out, int dtype,
                 hmoe_stream_t stream);

/* Combine plus a per-token addend: replaces aurora/hf_pipeline.py:370 (out.to(x.dtype) + self.shared_experts(x)):
 * out[t] = bf16(bf16(sum_j fp32(y[t*k + j])) + add[t]), add (T, d) bf16 (the shared expert's output).  The
 * reference sums the slots with index_add_ in expert order (:369); here they are summed in slot order (the same
 * terms, fp32 accumulation). */
int hmoe_combine_add(const void* y, const int32_t* inv_pos, int64_t T, int k, int64_t d, const void* add, void* out,
                     int dtype, hmoe_stream_t stream);

/* Whole routed forward in one call (inference): replaces the body of aurora/hf_compat.py:69-82 (route, sort,
 * gather, grouped gate/up, act * up, grouped down with weight and scatter, sum over slots) for a softmax top-k router
 * (conventions of aurora/hf_pipeline.py:352-359).  It runs hmoe_route_topk, hmoe_dispatch_tiles,
 * hmoe_gate_up_swiglu_tiles (h >= 4096, tiles below 2^31 bytes) or hmoe_gate_up_swiglu (rows gathered through
 * a_idx), hmoe_down_scatter and hmoe_combine in that order, with the intermediates (sort arrays, tiles, act, y) in
 * the workspace, so out, topk_ids, topk_w and logits (NULL to skip) are those the five calls give one by one.  x (T,
 * d) bf16 with row stride ldx; wr (E, d), wgu (E, d, 2h), wd (E, h, d) bf16; bias (E,) fp32 or NULL; out (T, d) bf16.
 * workspace: hmoe_moe_forward_workspace_size(T, d, E, k, h) bytes, 256-byte aligned.  Limits as the five entry
 * points (d % 8 == 0, h % 8 == 0, E <= 256, k <= 16). */
size_t hmoe_moe_forward_workspace_size(int64_t T, int64_t d, int E, int k, int64_t h);
int hmoe_moe_forward(const void* x, int64_t ldx, const void* wr, const float* bias, const void* wgu, const void* wd,
                     int64_t T, int64_t d, int E, int k, int64_t h, int renorm, float scaling, void* out,
                     int32_t* topk_ids, float* topk_w, float* logits, void* workspace, size_t workspace_bytes,
                     hmoe_stream_t stream);

/* The expert part of the routed forward in one call, for routing decided by the model's own gate: replaces
 * aurora/hf_compat.py:69-81 (sort, gather, grouped gate/up, act * up, grouped down with weight and scatter) for a
 * silu block.  It runs hmoe_dispatch_tiles, then hmoe_gate_up_swiglu_tiles (16-bit weights, h >= 4096, tiles below
 * 2^31 bytes), hmoe_gate_up_swiglu_i8 (w_dtype HMOE_DT_I8, scales wgu_s / wd_s as in the _i8 entry points) or
 * hmoe_gate_up_swiglu (rows gathered through a_idx), then hmoe_down_scatter(_i8), with the sort arrays, tiles and act
 * in the workspace, so y, inv_pos and n_invalid are what those calls give one by one.  topk_ids / topk_w as
 * hmoe_dispatch; 16-bit weights have the activations' type dtype (bf16 or fp16).  Outputs: y (T * k, d) of dtype in
 * (token, slot) order (rows of slots routed nowhere are not written), inv_pos (T * k,) int32 (negative for those
 * slots; hmoe_combine with it reads them as zeros), n_invalid (1,) int32.  workspace:
 * hmoe_moe_experts_workspace_size(T, d, E, k, h, w_dtype, dtype) bytes, 256-byte aligned.  Limits as the entry points
 * it runs. */
size_t hmoe_moe_experts_workspace_size(int64_t T, int64_t d, int E, int k, int64_t h, int w_dtype, int dtype);
int hmoe_moe_experts(const void* x, int64_t ldx, const void* topk_ids, int ids_dtype, const void* topk_w,
                     int topk_w_dtype, const void* wgu, const void* wgu_s, int wgu_s_dtype, const void* wd,
                     const void* wd_s, int wd_s_dtype, int w_dtype, int64_t T, int64_t d, int E, int k, int64_t h,
                     void* y, int32_t* inv_pos, int32_t* n_invalid, void* workspace, size_t workspace_bytes,
                     int dtype, hmoe_stream_t stream);

/* ---------------------------------------------------------------------------------------------------------------
 * Backward.  The reference has no backward for this path (aurora/hf_compat.py:62 is @torch.no_grad); each entry
 * point below differentiates the forward line it names.
 * ------------------------------------------------------------------------------------------------------------- */

/* Backward of :80-82 (weight multiply + combine).  For each sorted row r (token t = a_idx[r], flat f = order[r]):
 * dys[r] = bf16(w_sorted[r] * dout[t]) (M, d) and dtopk_w[f] = <dout[t], yhat[r]> (fp32, fixed order).  yhat NULL:
 * dys only (order and dtopk_w unused; hmoe_down_dgrad_swiglu_dw then gives dtopk_w). */
int hmoe_combine_bwd(const void* dout, const void* yhat, const int32_t* order, const int32_t* a_idx,
                     const uint16_t* w_sorted, int64_t M, int k, int64_t d, void* dys, float* dtopk_w,
                     hmoe_stream_t stream);

/* Backward of :81 through the down projection and the SwiGLU: dact[r] = w_sorted[r] * (dy[a_idx[r]] @ wd[e]^T)
 * (fp32; a_idx NULL: dy holds the sorted rows (M, d); w_sorted NULL: no scale), then
 * dgu[r] = [bf16(dact * u * silu'(g)) | bf16(dact * silu(g))] with [g | u] = gu[r].  dy is the upstream gradient of
 * the combined output (T, d) bf16: the routing weight enters in fp32, not through a rounded copy. */
int hmoe_down_dgrad_swiglu(const void* dy, const int32_t* a_idx, const uint16_t* w_sorted, const void* wd,
                           int64_t E, int64_t h, int64_t d, const void* counts, int counts_dtype, int64_t M,
                           const void* gu, void* dgu, hmoe_stream_t stream);

/* hmoe_down_dgrad_swiglu plus the routing-weight gradient from the same product (backward of :81's scale): for each
 * sorted row r (flat f = order[r]), dtopk_w[f] = sum_n (dy[a_idx[r]] @ wd[e]^T)[n] * act[r][n] with
 * act = bf16(bf16(silu(g)) * u) recomputed from gu[r] exactly as the forward rounds it -- <dy[t], act[r] @ wd[e]> in
 * fp32, without a rounded copy of the down projection's output.  Per-(row, column block) partials go to the
 * workspace (hmoe_down_dgrad_dw_workspace_size(M, h) bytes, 16-byte aligned) and are added in column-block order.
 * Has no counterpart in the reference (its MoE path has no backward). */
size_t hmoe_down_dgrad_dw_workspace_size(int64_t M, int64_t h);
int hmoe_down_dgrad_swiglu_dw(const void* dy, const int32_t* a_idx, const uint16_t* w_sorted, const void* wd,
                              int64_t E, int64_t h, int64_t d, const void* counts, int counts_dtype, int64_t M,
                              const void* gu, void* dgu, const int32_t* order, float* dtopk_w, void* workspace,
                              size_t workspace_bytes, hmoe_stream_t stream);

/* Backward of :79 to the sorted input rows: dxs[r] = dgu[r] @ wgu[e]^T, stored bf16 or fp32 (dxs_dtype). */
int hmoe_gate_up_dgrad(const void* dgu, const void* wgu, int64_t E, int64_t d, int64_t h, const void* counts,
                       int counts_dtype, int64_t M, void* dxs, int dxs_dtype, hmoe_stream_t stream);

/* Weight gradients of :79 and :81: dw[e] = a[rows of e]^T @ b[rows of e] (fp32 accumulation over the expert's
 * ragged row range, no split, deterministic); a (M, P) row stride lda, b (M, N) row stride ldb, both bf16 in
 * sorted order; dw (E, P, N) fp32 or bf16 (dw_dtype).  Experts with no rows get zeros (M = 0: all of dw, and a,
 * b may be NULL).  P, N % 8 == 0. */
int hmoe_grouped_wgrad(const void* a, int64_t lda, const void* b, int64_t ldb, int64_t E, int64_t P, int64_t N,
                       const void* counts, int counts_dtype, int64_t M, void* dw, int dw_dtype,
                       hmoe_stream_t stream);

/* Workspace bytes for hmoe_router_bwd. */
size_t hmoe_router_bwd_workspace_size(int64_t T, int E, int64_t d);

/* Router backward (softmax -> top-k gather -> renormalise, as in hmoe_route_topk): dlogits (T, E) fp32 from
 * dtopk_w (T, k) fp32, and dwr (E, d) = dlogits^T @ x (fp32 or bf16 per dwr_dtype; fixed-order reduction, on the
 * fp32 MFMA when E <= 16).  x is bf16 with row stride ldx >= d (ldx and d multiples of 8, x 16-byte aligned).
 * T = 0 writes zeros to dwr; the per-token pointers may then be NULL. */
int hmoe_router_bwd(const float* logits, const int32_t* topk_ids, const float* dtopk_w, int64_t T, int E, int k,
                    int renorm, float scaling, const void* x, int64_t ldx, int64_t d, float* dlogits, void* dwr,
                    int dwr_dtype, void* workspace, size_t workspace_bytes, hmoe_stream_t stream);

/* Input gradient: backward of the gather x[order // k] (:83 / a_idx of :78) plus the router's x.float() @ wr^T:
 * dx[t] = bf16(sum_j dxs[inv_pos[t*k + j]] + sum_e dlogits[t, e] * wr[e]) in fp32 (dlogits NULL: expert part
 * only); dxs (M, d) bf16 or fp32 (dxs_dtype); slots with a negative inv_pos add nothing. */
int hmoe_unpermute_bwd(const void* dxs, int dxs_dtype, const int32_t* inv_pos, const float* dlogits, const void* wr,
                       int64_t T, int k, int64_t d, int E, void* dx, hmoe_stream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* HMOE_H_ */
