/*
 * mingmoe.h — C ABI of libmingmoe.so, the MI355X (gfx950) kernels of the Ming thinker MoE block.
 *
 * Every entry point takes raw device pointers, element counts, row strides (in elements), dtype codes,
 * scalars and a hipStream_t (passed as void*), enqueues its kernels on that stream and returns an int
 * status (0 = ok). Nothing here allocates, frees or synchronises: scratch buffers are passed in by the
 * caller, so every call can be captured into a hipGraph. On a nonzero status, mm_last_error() gives
 * the message of the last failure on the calling thread; launch failures contain the text "HIP error".
 *
 * Each entry point names the reference Python interface it replaces (file:line in the Ming Voice
 * sources); the Python modules fused_ops.py, fused_moe.py and fastlinear.py of this package keep
 * those signatures and call these functions through ctypes.
 */
#ifndef MINGMOE_H
#define MINGMOE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define MM_ABI_VERSION 16

/* status codes */
#define MM_OK 0
#define MM_ERR_ARG 1     /* bad shape, dtype, stride, alignment or null pointer */
#define MM_ERR_HIP 2     /* a HIP launch failed; message starts with "HIP error" */

/* dtype codes (torch dtypes of the tensors behind the pointers) */
#define MM_BF16 0
#define MM_FP16 1
#define MM_FP32 2
#define MM_INT8 3
#define MM_INT32 4
#define MM_INT64 5

/* router scoring modes */
#define MM_SCORE_SIGMOID_GROUP 0 /* sigmoid + bias, group-limited top-k (the Ming thinker router) */
#define MM_SCORE_SOFTMAX 1       /* softmax over (logits + bias), top-k, renormalised */

/* phase masks of mm_moe_decode / mm_moe_prefill (0 = every phase). A later phase run alone reuses the
 * scratch (a_buf, o_buf) left by an earlier call with the same arguments; this lets a profiler or a
 * benchmark bracket one kernel with events. */
#define MM_PHASE_ALL 0
#define MM_PHASE_GATE_UP 1
#define MM_PHASE_DOWN 2
#define MM_PHASE_COMBINE 4

/* small_linear activations */
#define MM_ACT_NONE 0
#define MM_ACT_GELU_TANH 1
#define MM_ACT_SILU 2
/* ORed into small_linear's act: the norm prologue rounds once, bf16(x * rstd * g), as torch's F.rms_norm does on
 * the reference's path for more than 16 rows (fastlinear.py:151-160), instead of bf16(bf16(x * rstd) * g). */
#define MM_NORM_ROUND_ONCE 0x100

/* Stacked expert weights, as the thinker lays them out (engine.py:150-188, 313-391):
 *   w_gu [n_slots, 2*inter, hidden]  rows 0..inter-1 = gate, inter..2*inter-1 = up
 *   w_d  [n_slots, hidden, inter]
 * with the shared expert in the last slot. The last dim must be contiguous and every row 16-byte
 * aligned. For int8 weights (w_dtype = MM_INT8) s_gu [n_slots, 2*inter] and s_d [n_slots, hidden]
 * hold one scale per output row (s_dtype MM_FP32 or MM_BF16); for bf16 weights they are NULL.
 * w_gu_slabs (optional; NULL for none) is a second copy of w_gu in the prefill layout that mm_gate_up_slabs
 * writes: [n_slots][2*inter/R][hidden/64][R][64] of w_gu's type, contiguous, R = 8 for bf16 and 16 for int8, so
 * that each 64-wide k-slab of R consecutive rows is one 1 KB piece. When it is set the prefill gate/up GEMM reads
 * it instead of w_gu (same results, bit for bit); decode always reads w_gu. w_d_slabs (optional) is the same for
 * w_d, written by mm_down_slabs: [n_slots][hidden/R][inter/64][R][64], read by the prefill down GEMM. */
typedef struct mm_experts {
  const void* w_gu;
  const void* w_d;
  const void* s_gu;
  const void* s_d;
  int32_t w_dtype;
  int32_t s_dtype;
  int64_t n_slots;
  int64_t hidden;
  int64_t inter;
  int64_t gu_stride_e, gu_stride_n; /* element strides of w_gu dims 0 and 1 */
  int64_t d_stride_e, d_stride_n;   /* element strides of w_d dims 0 and 1 */
  int64_t sgu_stride_e, sd_stride_e; /* element strides of s_gu / s_d dim 0 */
  const void* w_gu_slabs;             /* optional prefill copy of w_gu (see above) */
  const void* w_d_slabs;              /* optional prefill copy of w_d (see above) */
} mm_experts;

/* ABI version (MM_ABI_VERSION) and the last error message of this thread (returns its length). */
int mm_version(void);
size_t mm_last_error(char* buf, size_t len);

/* RMSNorm, one row per token: y = (w * bf16(x * rsqrt(mean(x^2) + eps))) cast to y_dtype.
 * Replaces fused_ops.rms_norm / _rms_norm (fused_ops.py:16-37). x, w, y: bf16 / fp16 / fp32. */
int mm_rms_norm(const void* x, int x_dtype, int64_t rows, int64_t n, int64_t x_row_stride,
                const void* w, int w_dtype, float eps,
                void* y, int y_dtype, int64_t y_row_stride, void* stream);

/* MoE router for n_tokens rows: logits = x . w32^T in fp32, then top_k selection and weights.
 * Replaces fused_ops.moe_route / _gate_gemv / _route (fused_ops.py:40-103) and the multi-token gate
 * forward (engine.py:326-333).
 *   scoring MM_SCORE_SIGMOID_GROUP: s = sigmoid(logit); r = s + bias; groups of n_experts/n_group rank
 *     by the sum of their two largest r; the topk_group best groups stay; top_k of r (ties: lowest
 *     index); weight = s / (sum s + 1e-20) * scale.
 *   scoring MM_SCORE_SOFTMAX (n_group must be 1): z = logit + bias; top_k of z (ties: lowest index);
 *     p = softmax(z); weight = p / (sum p_selected + 1e-20) * scale.
 * append_shared != 0 writes id n_experts with weight 1.0 after the top_k routed ones (the shared
 * expert), so each output row holds top_k + 1 entries. bias may be NULL. ids: MM_INT32 / MM_INT64.
 * logits [n_tokens, n_experts] fp32 (row stride n_experts); ids / wts rows of stride out_row_stride. */
int mm_router(const void* x, int x_dtype, int64_t n_tokens, int64_t hidden, int64_t x_row_stride,
              const float* w32, int64_t n_experts, const float* bias,
              int scoring, int n_group, int topk_group, int top_k, float scale, int append_shared,
              float* logits, void* ids, int ids_dtype, float* wts, int64_t out_row_stride,
              void* stream);

/* Selection half of mm_router on logits already in device memory (same semantics and outputs). */
int mm_router_select(const float* logits, int64_t n_tokens, int64_t n_experts, const float* bias,
                     int scoring, int n_group, int topk_group, int top_k, float scale, int append_shared,
                     void* ids, int ids_dtype, float* wts, int64_t out_row_stride, void* stream);

/* Stable counting sort of the P (token, slot) pairs by expert, each expert's run padded to block_m.
 * Replaces fused_moe._align_blocks (fused_moe.py:154-173), bit-exact:
 *   sorted_ids [nb*block_m] int32: pair indices grouped by expert in ascending pair order, pad = P;
 *   bexp [nb] int32: expert of each block, -1 past the last used block;
 *   nb must equal ceil((P + n_slots*(block_m-1)) / block_m).
 *   expert_offsets (optional, may be NULL) [n_slots+1] int32: padded start row of each expert and,
 *   in the last entry, the number of used rows.
 * flat: MM_INT32 / MM_INT64 expert ids; ids outside [0, n_slots) are dropped. P <= 2^30. */
int mm_align_blocks(const void* flat, int flat_dtype, int64_t P, int32_t n_slots, int32_t block_m,
                    int32_t* sorted_ids, int32_t* bexp, int64_t nb, int32_t* expert_offsets,
                    void* stream);

/* Decode MoE for 1..8 tokens: for each token t and slot k (expert e = ids[t,k]):
 *   g = bf16(x_t . Wg[e]^T [* s]), u = bf16(x_t . Wu[e]^T [* s]), a = bf16(bf16(silu(g)) * u)
 *   y_t = bf16(sum_k wts[t,k] * bf16(a . Wd[e]^T [* s]))          (fp32 sum in slot order)
 *   with residual: y_t = bf16(y_t + residual_t)
 * Each distinct expert of the batch is streamed from HBM once. Replaces fused_moe.fused_moe_decode /
 * _moe_gate_up / _moe_down (fused_moe.py:13-83) and, for 2..8 tokens, the prefill kernels the
 * reference falls back to (engine.py:379-382). n_tokens * nk <= 64.
 * x, residual, y: bf16. ids: MM_INT32 / MM_INT64 [n_tokens, nk]; wts fp32 [n_tokens, nk].
 * a_buf: bf16 scratch [n_tokens*nk, inter] (row p = t*nk + k), also an output of the call. */
int mm_moe_decode(const void* x, int64_t n_tokens, int64_t x_row_stride, const mm_experts* ex,
                  const void* ids, int ids_dtype, int64_t nk, int64_t ids_row_stride,
                  const float* wts, int64_t wts_row_stride,
                  const void* residual, int64_t res_row_stride,
                  void* a_buf, void* y, int64_t y_row_stride, int phases, void* stream);

/* One decode MoE block for 1..8 bf16 tokens in four kernels:
 *   router:  xn = RMSNorm(x; norm_w bf16, eps) on the fly (bit-identical to mm_rms_norm), logits = xn . w32^T,
 *            xn stored to the workspace;
 *   select:  as mm_router's selection (shared expert n_experts appended with weight 1), into ids / wts;
 *   gate/up, down: as mm_moe_decode on xn, y = MoE(xn) (+ x when add_residual).
 * Same results as mm_rms_norm -> mm_router -> mm_moe_decode(residual = x). No single call of the reference
 * does this: it fuses the per-layer sequence of engine.py:229, 284-297, 371-386.
 * ex->n_slots must be n_experts + 1. logits fp32 [n_tokens, n_experts], ids [n_tokens, top_k+1]
 * (MM_INT32 / MM_INT64), wts fp32 [n_tokens, top_k+1], a_buf bf16 [n_tokens*(top_k+1), inter],
 * y bf16 [n_tokens, hidden] (must not alias x when add_residual). workspace: 16-byte aligned device
 * scratch of n_tokens * hidden bf16 (the normalised rows); calls that share one workspace must not overlap. */
int mm_moe_block_decode(const void* x, int64_t n_tokens, int64_t x_row_stride, const void* norm_w, float eps,
                        const float* w32, int64_t n_experts, const float* bias, int scoring, int n_group,
                        int topk_group, int top_k, float scale, const mm_experts* ex, float* logits,
                        void* ids, int ids_dtype, float* wts, void* a_buf, void* workspace, int add_residual,
                        void* y, int64_t y_row_stride, void* stream);

/* mm_moe_block_decode with its scratch (the normalised rows and the gated activations, the `workspace` and
 * `a_buf` of mm_moe_block_decode) held in a static device array of MM_NOALLOC_SCRATCH_BYTES per GPU instead of
 * caller buffers: the call allocates nothing and takes no scratch argument; the caller passes the inputs and
 * the outputs (logits, ids, wts, y). Same kernels and bit-identical results as mm_moe_block_decode.
 * No counterpart in the reference: it is for callers that cannot allocate device memory (code under hipGraph
 * capture, tight serving loops, harnesses that forbid hipMalloc). Limit: mm_moe_block_decode_noalloc_bytes()
 * of the shape must not exceed MM_NOALLOC_SCRATCH_BYTES (larger shapes return MM_ERR_ARG). Each GPU holds its
 * own array from the first call on it until the process ends; calls that overlap on one GPU (two streams or
 * threads at once) share that array and race. */
#define MM_NOALLOC_SCRATCH_BYTES (2 * 1024 * 1024)
/* Bytes of that scratch a shape needs: the normalised rows (n_tokens * hidden bf16, rounded up to 256 bytes)
 * then the activations (n_tokens * (top_k + 1) * inter bf16); -1 for an invalid shape. */
int64_t mm_moe_block_decode_noalloc_bytes(int64_t n_tokens, int64_t top_k, int64_t hidden, int64_t inter);
int mm_moe_block_decode_noalloc(const void* x, int64_t n_tokens, int64_t x_row_stride, const void* norm_w, float eps,
                                const float* w32, int64_t n_experts, const float* bias, int scoring, int n_group,
                                int topk_group, int top_k, float scale, const mm_experts* ex, float* logits,
                                void* ids, int ids_dtype, float* wts, int add_residual, void* y,
                                int64_t y_row_stride, void* stream);

/* Grouped prefill MoE over the blocks produced by mm_align_blocks (same math as mm_moe_decode).
 * Replaces fused_moe.fused_moe_prefill / _moe_gu_grouped / _moe_down_grouped (fused_moe.py:92-196).
 * x [n_tokens, hidden] bf16; ids [n_tokens*nk] (MM_INT32 / MM_INT64, the flat ids given to align; pairs
 * p = t*nk + k whose id lies outside [0, n_slots) contribute nothing); wts fp32 [n_tokens*nk];
 * sorted_ids / bexp / expert_offsets / nb / block_m from mm_align_blocks, block_m = 64 or, for bf16 experts,
 * 128 (mm_prefill_block_m gives the faster one for a shape); a_buf bf16 [nb*block_m, 64*ceil(inter/64)]
 * (the gated activations of each expert block in 64-column slabs, [nb][ceil(inter/64)][block_m][64], so that the
 * down GEMM reads each of its activation slabs as one contiguous piece) and part_buf bf16 [n_tokens*nk, hidden]
 * (per-pair expert outputs bf16(a . Wd^T), before the slot weight) are scratch; y bf16 [n_tokens, hidden]. */
/* Rows per expert block the prefill kernels take for a shape (the align padding): 128 for bf16 experts
 * (w_dtype MM_BF16) averaging at least 128 pairs (n_tokens * nk >= 128 * n_slots: each weight slab then
 * feeds twice the MFMA rows), else 64. No counterpart in the reference (its grouped kernels take BM = 64,
 * fused_moe.py:176-196). */
int32_t mm_prefill_block_m(int64_t n_tokens, int64_t nk, int64_t n_slots, int w_dtype);

int mm_moe_prefill(const void* x, int64_t n_tokens, int64_t x_row_stride, const mm_experts* ex,
                   int64_t nk, const void* ids, int ids_dtype, const float* wts,
                   const int32_t* sorted_ids, const int32_t* bexp, const int32_t* expert_offsets,
                   int64_t nb, int32_t block_m, const void* residual, int64_t res_row_stride,
                   void* a_buf, void* part_buf, void* y, int64_t y_row_stride, int phases, void* stream);

/* One MoE block for a prefill batch (any n_tokens >= 1): xn = RMSNorm(x; norm_w bf16, eps) (stored;
 * fused into the router GEMV up to 8 tokens, bit-identical to mm_rms_norm), router logits of xn, the
 * selection (shared expert n_experts appended with weight 1), mm_align_blocks, then mm_moe_prefill on xn
 * with x as residual when add_residual. Same results as mm_rms_norm -> mm_router -> mm_align_blocks ->
 * mm_moe_prefill(residual = x). No single call of the reference does this: it fuses the per-layer
 * sequence of engine.py:229, 284-309.
 * ex->n_slots must be n_experts + 1. logits fp32 [n_tokens, n_experts]; ids [n_tokens, top_k+1]
 * (MM_INT32 / MM_INT64); wts fp32 [n_tokens, top_k+1]; xn bf16 [n_tokens, hidden] (16-byte aligned);
 * sorted_ids / bexp / expert_offsets / nb sized as for mm_align_blocks with block_m =
 * mm_prefill_block_m(n_tokens, top_k + 1, n_experts + 1, ex->w_dtype); a_buf / part_buf
 * as for mm_moe_prefill; y bf16 [n_tokens, hidden] (must not alias x when add_residual). */
int mm_moe_block_prefill(const void* x, int64_t n_tokens, int64_t x_row_stride, const void* norm_w, float eps,
                         const float* w32, int64_t n_experts, const float* bias, int scoring, int n_group,
                         int topk_group, int top_k, float scale, const mm_experts* ex, float* logits,
                         void* ids, int ids_dtype, float* wts, void* xn, int32_t* sorted_ids, int32_t* bexp,
                         int32_t* expert_offsets, int64_t nb, void* a_buf, void* part_buf, int add_residual,
                         void* y, int64_t y_row_stride, void* stream);

/* y = act(norm?(x) . W^T + b) [+ residual] for M <= 16 rows.
 * Replaces fastlinear.small_linear / _small_m_linear (fastlinear.py:123-174) including the rounding
 * points of its epilogue: bf16 before the activation and before the residual add.
 * x, w, b, residual, norm_g, y: bf16. norm_g (optional): RMSNorm prologue with norm_eps,
 * x -> bf16(bf16(x * rstd) * g), or bf16(x * rstd * g) with MM_NORM_ROUND_ONCE in act (the rounding of the
 * reference's torch path for M > 16, which callers run as 16-row pieces). b, residual, norm_g may be NULL.
 * act: MM_ACT_* (| MM_NORM_ROUND_ONCE).
 * xn_buf: bf16 scratch [M, K], used only when a norm prologue is given and K > 8192 (may be NULL otherwise);
 * shorter rows get the norm fused into the GEMV. x_row_stride 0 repeats one activation row M times. */
int mm_small_linear(const void* x, int64_t M, int64_t K, int64_t x_row_stride,
                    const void* w, int64_t N, int64_t w_row_stride,
                    const void* b, int act, const void* residual, int64_t res_row_stride,
                    const void* norm_g, float norm_eps, void* xn_buf,
                    void* y, int64_t y_row_stride, void* stream);

/* act = silu_mul(small_linear(norm?(x), W)) in one kernel: W [2*inter, K] holds the gate rows then the up
 * rows; y[:, p] = bf16(bf16(silu(g_p)) * u_p) with g_p, u_p the bf16-rounded projections of rows p and
 * inter + p, so the result equals small_linear followed by silu_mul bit for bit. No counterpart in the
 * reference: it fuses fast_talker.py:258-260 (gate|up small_linear, _silu_mul) for callers that own the
 * layer loop. x, w, norm_g, y: bf16; M <= 16; K <= 8192, a multiple of 8; norm_g may be NULL. */
int mm_small_linear_glu(const void* x, int64_t M, int64_t K, int64_t x_row_stride, const void* w, int64_t inter,
                        int64_t w_row_stride, const void* norm_g, float norm_eps, void* y, int64_t y_row_stride,
                        void* stream);

/* Symmetric per-row int8: amax = max(max|w|, 1e-8); scale = amax / 127;
 * q = clamp(round_half_even(w / scale), -127, 127).
 * Replaces fused_moe.quantize_rows_int8 (fused_moe.py:199-204). w: bf16 / fp16 / fp32 [rows, K];
 * q int8 [rows, K]; scale [rows] in MM_FP32 (reference) or MM_BF16 (then the scale is rounded to bf16
 * first and q divides by the rounded value). */
int mm_quantize_rows_int8(const void* w, int w_dtype, int64_t rows, int64_t K, int64_t w_row_stride,
                          int8_t* q, int64_t q_row_stride, void* scale, int scale_dtype, void* stream);

/* ---- Talker kernels (fast_talker.py). bf16 activations; latency-bound, a few KB to a few 100 KB per call. */

/* Rotary attention over seq <= 8 tokens per (batch, head), for the Talker's DiT and aggregator blocks.
 * Replaces fast_talker.rope_attn / _tiny_rope_attn (fast_talker.py:34-79).
 * qkv bf16 [batch, seq, 3*dim] contiguous (q | k | v, head h at columns h*hd .. h*hd+hd-1 of each part);
 * cos_t, sin_t fp32 [seq, hd/2] (one angle per interleaved pair); out bf16 [batch, seq, dim].
 * Pair (x[2p], x[2p+1]) is rotated by angle p and rounded to bf16 for q and k; scores are scaled by
 * 1/sqrt(hd); the softmax weights are rounded to bf16 before p . v. hd = dim/heads must be even, <= 256. */
int mm_rope_attn(const void* qkv, int64_t batch, int64_t seq, int64_t dim, int heads, const float* cos_t,
                 const float* sin_t, void* out, void* stream);

/* Bytes of fp32 workspace mm_qwen_decode_attn needs: nh * ceil(max_len/64) * (hd + 2) * 4 (0 if invalid). */
int64_t mm_decode_attn_workspace(int nh, int hd, int64_t max_len);

/* Single-token GQA decode attention of the Talker's Qwen2 over its static KV cache.
 * Replaces fast_talker._qwen_decode_attn (fast_talker.py:165-212, launched at :255-256).
 * qkv bf16 [(nh + 2*nkv) * hd] (q heads, then k heads, then v heads); k_cache, v_cache bf16
 * [nkv, max_len, hd] (one layer of StaticQwen2's cache, engine.py:1258-1259); pos: device scalar
 * (MM_INT64 / MM_INT32), the position of this token; inv_freq fp32 [hd/2]; out bf16 [nh * hd].
 * Rotary (rotate-half form, cos / sin of pos * inv_freq rounded to bf16) is applied to q and k, rounded to
 * bf16; k and v are written into the caches at row pos; out = softmax(scale * q . K[0..pos]) . V[0..pos].
 * A pos outside [0, max_len) writes nothing to the caches and sets the output to NaN.
 * nh must be a multiple of nkv with nh/nkv <= 16; hd a multiple of 32 in [32, 256]; max_len <= 65536.
 * workspace: at least mm_decode_attn_workspace(nh, hd, max_len) bytes of device memory, 16-byte aligned;
 * its contents need no initialisation. Two kernels, both on `stream`. */
int mm_qwen_decode_attn(const void* qkv, int nh, int nkv, int hd, void* k_cache, void* v_cache, int64_t max_len,
                        const void* pos, int pos_dtype, const float* inv_freq, float scale, void* out,
                        void* workspace, int64_t workspace_bytes, void* stream);

/* The flow-matching update of the Talker tail in one kernel: y_out = y + (pred + (pred - null) * cfg) * dt
 * with bf16 rounding after every operation, as the bf16 torch expression of fast_talker.py:151-152 rounds.
 * y, y_out: bf16 [n] (may alias); pred_null: bf16, rows pred and null `pn_row_stride` elements apart;
 * dt: device scalar (MM_BF16 or MM_FP32). No counterpart kernel in the reference (five torch launches). */
int mm_cfg_update(const void* y, const void* pred_null, int64_t pn_row_stride, int64_t n, float cfg, const void* dt,
                  int dt_dtype, void* y_out, void* stream);

/* out = bf16(bf16(silu(g)) * u) for rows of gu = [g | u], each 2*inter wide.
 * Replaces fast_talker._silu_mul (fast_talker.py:215-222, launched at :259-260). gu, out bf16;
 * rows <= 65535; row strides in elements. */
int mm_silu_mul(const void* gu, int64_t rows, int64_t inter, int64_t gu_row_stride, void* out,
                int64_t out_row_stride, void* stream);

/* ---- Thinker attention mixers (the hybrid thinker's KDA and MLA layers, engine.py:234-267, 495-548, 665-713).
 * bf16 activations, fp32 state and statistics; every call enqueues on `stream` and allocates nothing. */

/* Kimi delta attention, recurrent form, for T tokens of one sequence: what fla's fused_recurrent_kda (fla-core 0.5.2,
 * called at engine.py:258 and by the model's KDA layers) computes. Per head h and token t, in fp32:
 *   q, k = l2norm(q), l2norm(k) (x / sqrt(sum x^2 + 1e-6)) when use_qk_l2norm; q *= scale
 *   g' = -exp(A_log[h]) * softplus(g + dt_bias[h]) (lower_bound NaN) or lower_bound * sigmoid(exp(A_log[h]) * (g + dt_bias))
 *        when use_gate, else g' = g (already a log decay)
 *   S = S * exp(g')[:, None]; u = beta * (v - S^T k); S = S + k u^T; o = S^T q   (S [K, V])
 * q, k [T, H, K] bf16, v [T, H, V] bf16, g [T, H, K] (MM_BF16 / MM_FP32), beta [T, H] (MM_BF16 / MM_FP32; the write
 * strength, or with beta_logits the projection whose sigmoid it is), each with its token stride in elements; A_log [H], dt_bias [H * K] fp32 (used when
 * use_gate); state [H, K, V] fp32, read and updated in place; o [T, H, V] bf16 (token stride o_ts).
 * K: 64 or 128; V: a multiple of 8 up to 4096 (of 16 for T <= 2). workspace: at least
 * mm_kda_recurrent_workspace(T, H, K) bytes, 16-byte aligned (the per-token inputs prepared for all tokens at once,
 * then read by the sequential part); T <= 2 (a decode step) runs in one launch and needs none (NULL allowed).
 * n_valid: NULL, or an int64 device scalar n: tokens n .. T - 1 are padding and leave the state exactly unchanged
 * (decay 1, write strength 0: the padded prefill of engine.py:252-253, where the gate is -1e30 and beta 0); their
 * outputs are unspecified. */
int mm_kda_recurrent(const void* q, int64_t q_ts, const void* k, int64_t k_ts, const void* v, int64_t v_ts,
                     const void* g, int g_dtype, int64_t g_ts, const void* beta, int beta_dtype, int64_t beta_ts,
                     const float* A_log, const float* dt_bias, float lower_bound, int use_qk_l2norm, int use_gate,
                     int beta_logits, float scale, int64_t T, int64_t H, int64_t K, int64_t V, float* state, void* o,
                     int64_t o_ts, const int64_t* n_valid, void* workspace, int64_t workspace_bytes, void* stream);

/* Bytes of fp32 workspace mm_kda_recurrent needs: T * H * (3 K + 4) * 4, 0 for T <= 2 (-1 if invalid). */
int64_t mm_kda_recurrent_workspace(int64_t T, int64_t H, int64_t K);

/* The same recurrence in chunked form: what fla's chunk_kda (fla-core 0.5.2) computes, which the engine's eager
 * prefill selects for prompt pieces of more than 192 tokens (engine.py:946-949, 964-967; the model's KDA layers call
 * it). Same arguments, checks and outputs as mm_kda_recurrent up to the order of fp32 sums: the tokens go 16 at a
 * time, each chunk in closed form (the decay products and the chunk's k-k and q-k products computed for all chunks
 * at once, then a forward substitution per chunk), so a token no longer waits for the sums of the token before it.
 * workspace: at least mm_kda_chunk_workspace(T, H, K) bytes, 16-byte aligned; T <= 2 runs as mm_kda_recurrent. */
int mm_kda_chunk(const void* q, int64_t q_ts, const void* k, int64_t k_ts, const void* v, int64_t v_ts,
                 const void* g, int g_dtype, int64_t g_ts, const void* beta, int beta_dtype, int64_t beta_ts,
                 const float* A_log, const float* dt_bias, float lower_bound, int use_qk_l2norm, int use_gate,
                 int beta_logits, float scale, int64_t T, int64_t H, int64_t K, int64_t V, float* state, void* o,
                 int64_t o_ts, const int64_t* n_valid, void* workspace, int64_t workspace_bytes, void* stream);

/* Bytes of fp32 workspace mm_kda_chunk needs: ceil(T / 16) * H * (49 K + 512) * 4 (one block per 16-token chunk and
 * head), 0 for T <= 2 (-1 if invalid). */
int64_t mm_kda_chunk_workspace(int64_t T, int64_t H, int64_t K);

/* Depthwise causal convolution over time, the step form of fla's ShortConvolution (the q / k / v convolutions of a
 * KDA layer, engine.py:247-249, caches engine.py:645-647): per channel, for each of T tokens in order, the window
 * (cache[ch, 1..W-1], x[t, ch]) replaces the cache and y[t, ch] = act(sum_j w[ch, j] * window[j] + b[ch]) (act 1:
 * SiLU, 0: none; fp32, one rounding). x, y [T, C] bf16 with token strides; cache [C, W], w [C, W] (a conv1d weight
 * [C, 1, W]) bf16; b [C] bf16 or NULL. 2 <= W <= 8. n_valid: NULL, or an int64 device scalar n: the cache ends on
 * the first n tokens' inputs (the padded prefill's conv_idx, engine.py:261-262); every y row is still computed. */
int mm_short_conv(const void* x, int64_t x_ts, int64_t T, int64_t C, void* cache, int64_t W, const void* w,
                  const void* b, int act, void* y, int64_t y_ts, const int64_t* n_valid, void* stream);

/* mm_short_conv (no bias) on n <= 4 convolutions over the same T tokens and width W in one launch: the q, k and v
 * convolutions of a KDA layer over a prompt (engine.py:247-249), which the reference runs as three ShortConvolution
 * calls. Host arrays of n entries: x[i], y[i] [T, C[i]] bf16 with token strides x_ts[i], y_ts[i]; cache[i], w[i]
 * [C[i], W] bf16. act and n_valid as for mm_short_conv; each convolution's results equal its own mm_short_conv. */
int mm_short_conv_many(int64_t n, const void* const* x, const int64_t* x_ts, const int64_t* C, void* const* cache,
                       const void* const* w, void* const* y, const int64_t* y_ts, int64_t T, int64_t W, int act,
                       const int64_t* n_valid, void* stream);

/* y = bf16(x * rsqrt(mean(x^2) + eps) * w * sigmoid(g)) per row of n <= 512 elements: fla's FusedRMSNormGated with a
 * sigmoid gate, the output norm of a KDA layer (o_norm, engine.py:265). x, g, y [rows, n] bf16 with row strides;
 * w [n] bf16. */
int mm_rms_norm_gated(const void* x, int64_t x_rs, const void* g, int64_t g_rs, const void* w, int64_t rows, int64_t n,
                      float eps, void* y, int64_t y_rs, void* stream);

/* One decode token of a KDA layer's core in one kernel: the chain mm_short_conv (q, k, v; SiLU) ->
 * f = bf16(f_b . fa) -> mm_kda_recurrent (l2-normed q / k, the in-kernel gate, beta as logits) -> g = bf16(g_b . ga)
 * -> mm_rms_norm_gated of engine.py:242-265 for one token, on the layer's projection row
 * pr = [q | k (H K each) | v (H V) | fa | ga (R each) | beta logits (H)] (bf16, pr_len elements). conv_w[3] and
 * conv_cache[3]: the q, k and v conv weights ([C, 1, W] as the conv1d modules hold them) and the layer's three conv
 * caches ([1, C, W], shifted in place), C = H K, H K, H V, bf16, 8-byte aligned; f_b [H K, R], g_b [H V, R] bf16 (LoRA
 * up-projections); A_log [H], dt_bias [H K] fp32; state [H, K, V] fp32 (16-byte aligned), updated in place;
 * o_norm [V] bf16; y [H, V] bf16 out. K = 128, V a multiple of 16 up to 512, W = 4, R a multiple of 16 up to 256. No single call of
 * the reference does this: it fuses the five launches of one KDA layer step; results equal the chain's except
 * where the f / g dots round differently in the last bf16 place. */
int mm_kda_decode_step(const void* pr, int64_t pr_len, const void* const* conv_w, void* const* conv_cache, int64_t W,
                       const void* f_b, const void* g_b, int64_t R, const float* A_log, const float* dt_bias,
                       float lower_bound, float scale, float* state, int64_t H, int64_t K, int64_t V,
                       const void* o_norm, float eps, void* y, void* stream);

/* Bytes of fp32 workspace mm_mla_decode_attn needs: nh * ceil(max_len / 32) * (dv + 2) * 4 (0 if invalid). */
int64_t mm_mla_attn_workspace(int nh, int dv, int64_t max_len);

/* Single-token attention of an MLA layer over its static cache (the StaticHybridCache update and the masked
 * attention of engine.py:537-548, 679-686): k_new / v_new are written at row pos of k_cache [nh, max_len, dqk] and
 * v_cache [nh, max_len, dv] (bf16), then out[h] = softmax(scale * q[h] . K[h, 0..pos]^T) . V[h, 0..pos] in fp32,
 * rounded to bf16. q, k_new [nh, dqk], v_new [nh, dv], out [nh, dv] bf16; pos a device scalar (MM_INT64 /
 * MM_INT32). A pos outside [0, max_len) writes nothing to the caches and sets out to NaN. dqk a multiple of 8 up
 * to 512, dv a multiple of 8 up to 256; rows past pos are never read. q, k_new, v_new, the caches and the
 * workspace (at least mm_mla_attn_workspace(nh, dv, max_len) bytes) 16-byte aligned. */
int mm_mla_decode_attn(const void* q, const void* k_new, const void* v_new, int nh, int dqk, int dv, void* k_cache,
                       void* v_cache, int64_t max_len, const void* pos, int pos_dtype, float scale, void* out,
                       void* workspace, int64_t workspace_bytes, void* stream);

/* The T tokens of a prompt through an MLA layer's attention (engine.py:938-972 prefill: the StaticHybridCache
 * index_copy_ of engine.py:537-541 at positions pos .. pos + T - 1, then the causal attention of the mask at
 * engine.py:679-682): token t's k_new / v_new rows go to cache row pos + t of k_cache [nh, max_len, dqk] and
 * v_cache [nh, max_len, dv] (bf16), then out_t[h] = softmax(scale * q_t[h] . K[h, 0..pos+t]^T) . V[h, 0..pos+t],
 * accumulated in fp32 (the probabilities enter the value product as bf16), rounded to bf16. q, k_new: T rows of
 * [nh, dqk] at token strides q_ts, k_ts; v_new, out: T rows of [nh, dv] at v_ts, out_ts (elements); pos a device
 * scalar (MM_INT64 / MM_INT32), the first token's position. A prompt outside [0, max_len) (pos < 0 or
 * pos + T > max_len) writes nothing to the caches and sets out to NaN. dqk a multiple of 8 up to 256, dv a multiple of
 * 8 up to 128; q, k_new, v_new and the caches 16-byte aligned with rows at 16-byte strides, out 8-byte aligned. With
 * T = 1 it computes what mm_mla_decode_attn does. */
int mm_mla_prefill_attn(const void* q, int64_t q_ts, const void* k_new, int64_t k_ts, const void* v_new, int64_t v_ts,
                        int64_t T, int nh, int dqk, int dv, void* k_cache, void* v_cache, int64_t max_len,
                        const void* pos, int pos_dtype, float scale, void* out, int64_t out_ts, void* stream);

/* ---- The two ends of a greedy decode step (engine.py:685-689). */

/* out[i, :] = table[ids[i], :] for i < n: word_embeddings(tok_buf) (engine.py:686). table [V, H] and out rows of
 * bf16 / fp16 / fp32 (dtype), 16-byte aligned rows, H * element size a multiple of 16; ids MM_INT32 / MM_INT64 [n]
 * on the device. An id outside [0, V) gives a row of zeros (torch's embedding stops on a device-side assert). */
int mm_embed_rows(const void* table, int dtype, int64_t V, int64_t H, int64_t table_row_stride, const void* ids,
                  int ids_dtype, int64_t n, void* out, int64_t out_row_stride, void* stream);

/* out[r] = logits[r].argmax() (engine.py:688, logits.argmax(-1)) for each of `rows` rows of n elements (bf16 or
 * fp32, x_row_stride elements apart): torch's order, the largest value, NaN above every number, the lowest index
 * among equals. out: int64 [rows] on the device. */
int mm_argmax_rows(const void* x, int x_dtype, int64_t rows, int64_t n, int64_t x_row_stride, int64_t* out,
                   void* stream);

/* mm_argmax_rows with the row split over many workgroups (one CU draws a long row only at the rate its outstanding
 * lines allow; the LM head's 126464 logits take 17 us that way) and a second launch merging their partial results,
 * same results. workspace: device memory of mm_argmax_rows_workspace_bytes(rows, n, x_dtype) bytes, 16-byte aligned
 * (-1: bad arguments); calls that share a workspace must not overlap; rows <= 65535. Rows that are short, not
 * 16-byte aligned or not a whole number of 16-byte pieces take mm_argmax_rows. No counterpart in the reference beyond
 * logits.argmax(-1) (engine.py:688). */
int64_t mm_argmax_rows_workspace_bytes(int64_t rows, int64_t n, int x_dtype);
int mm_argmax_rows_ws(const void* x, int x_dtype, int64_t rows, int64_t n, int64_t x_row_stride, int64_t* out,
                      void* workspace, int64_t workspace_bytes, void* stream);

/* ---- Expert ingestion from safetensors shards (engine.py:126-188, direct_load.py:81-131). */

#define MM_PART_GATE 0 /* rows 0..I-1 of w_gu[slot] */
#define MM_PART_UP 1   /* rows I..2I-1 of w_gu[slot] */
#define MM_PART_DOWN 2 /* w_d[slot] */

/* One expert matrix in a file: `nbytes` bytes at absolute `offset` of `path` hold a row-major
 * [rows, cols] tensor of src_dtype (MM_BF16 / MM_FP16 / MM_FP32). */
typedef struct mm_ingest_item {
  const char* path;
  int64_t offset;
  int64_t nbytes;
  int32_t src_dtype;
  int32_t part;
  int64_t slot;
  int64_t rows;
  int64_t cols;
} mm_ingest_item;

/* Reads every item and writes it into the stack `dst`: as bf16 (fp16 / fp32 file data rounded to nearest
 * even), or, when dst->w_dtype is MM_INT8, quantised per row as mm_quantize_rows_int8 does (scales in
 * dst->s_dtype). Replaces the per-tensor loader hooks of engine.py:126-147 (quantize-on-load) and the
 * restacking of engine.py:150-188 / 343-361. n_threads workers read with pread in file order, each through
 * two pinned host slots and one device slot of slot_bytes (host_staging: 2 * n_threads * slot_bytes of
 * pinned host memory; dev_staging: n_threads * slot_bytes of device memory; slot_bytes >= every item's
 * nbytes). Blocking: returns when every matrix is in place, on streams of its own; the caller finishes its
 * own work on dst before the call. Shapes must match the stack: gate / up [inter, hidden], down [hidden, inter]. */
int mm_ingest_experts(const mm_ingest_item* items, int64_t n_items, const mm_experts* dst, void* host_staging,
                      void* dev_staging, int64_t slot_bytes, int n_threads);

/* Bytes of the prefill copy of ex->w_gu (n_slots * 2 * inter * hidden * weight bytes), or 0 when the experts
 * cannot have one (hidden not a multiple of 64, or 2 * inter not a multiple of R: 8 for bf16, 16 for int8). */
int64_t mm_gate_up_slabs_bytes(const mm_experts* ex);

/* Writes the prefill copy of ex->w_gu (any row strides) into `out` (mm_gate_up_slabs_bytes bytes, 16-byte
 * aligned): out[e][q][t][j][c] = w_gu[e][R q + j][64 t + c]. A load-time step like the quantise-on-load
 * hooks (engine.py:126-147); no call of the reference does this: its Triton GEMM reads the row layout. The
 * copy costs a second gate/up stack (750 MB in bf16, 375 MB in int8 per 64+1-expert layer of hidden 2048, inter
 * 1408) and lets the prefill gate/up GEMM read each k-slab of a weight tile as 1 KB pieces, one per direct-load
 * instruction, instead of 128-byte (bf16) or 64-byte (int8) row slices. */
int mm_gate_up_slabs(const mm_experts* ex, void* out, void* stream);

/* Bytes of the prefill copy of ex->w_d (n_slots * hidden * inter * weight bytes), or 0 when the experts cannot
 * have one (inter not a multiple of 64, or hidden not a multiple of R: 8 for bf16, 16 for int8). */
int64_t mm_down_slabs_bytes(const mm_experts* ex);

/* Writes the prefill copy of ex->w_d (any row strides) into `out` (mm_down_slabs_bytes bytes, 16-byte
 * aligned): out[e][q][t][j][c] = w_d[e][R q + j][64 t + c]. The same load-time step as mm_gate_up_slabs, for
 * the down GEMM's weights (375 MB in bf16, 188 MB in int8 more per 64+1-expert layer of hidden 2048, inter 1408);
 * no counterpart in the reference. */
int mm_down_slabs(const mm_experts* ex, void* out, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* MINGMOE_H */
