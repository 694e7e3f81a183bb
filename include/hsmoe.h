/*
 * libhsmoe -- C ABI of the MI355X (gfx950) routed-expert MoE hot path.
 *
 * Conventions
 *   - Every pointer argument named *_dev is device memory; the library never
 *     allocates, frees or copies user memory.  Scratch memory comes from a
 *     caller-provided `workspace` of at least the size the matching
 *     *_workspace_size() call returns, zero-filled once when it is allocated
 *     (kernels leave their counters at zero when they finish); the one
 *     exception, hsmoe_moe_layer_decode_noalloc, uses a static scratch array
 *     of the library instead.
 *   - bf16 tensors are passed as raw 16-bit storage, row-major, contiguous
 *     unless a row stride argument says otherwise.
 *   - All work is enqueued on `stream` (a hipStream_t; NULL is the default
 *     stream); nothing blocks the host.
 *   - Return value: HSMOE_OK (0) or a negative HSMOE_ERR_* code; the text of
 *     the last error of the calling thread is hsmoe_last_error().
 *   - Calls that share one workspace must not overlap in time.
 */
#ifndef HSMOE_H_
#define HSMOE_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define HSMOE_VERSION 1

#define HSMOE_OK 0
#define HSMOE_ERR_ARG (-1)        /* null pointer, bad count, bad enum */
#define HSMOE_ERR_SHAPE (-2)      /* shape/alignment outside what a kernel supports */
#define HSMOE_ERR_LAUNCH (-3)     /* HIP reported an error at launch */
#define HSMOE_ERR_WORKSPACE (-4)  /* workspace missing or too small */

/* Scale encodings of FP4 weights (one scale per 32 consecutive columns). */
#define HSMOE_SCALE_E8M0 0 /* uint8 exponent e: 2^(e-127), e == 255 is NaN */
#define HSMOE_SCALE_F32 1  /* fp32 value */

typedef void* hsmoe_stream_t; /* a hipStream_t */

int hsmoe_version(void);
const char* hsmoe_last_error(void);
void hsmoe_clear_error(void);

/* ---------------------------------------------------------------------------
 * FP4 (e2m1, two codes per byte, low nibble = even column) -> bf16.
 *   out[n, c] = bf16(e2m1(code[n, c]) * scale[n, c / 32])
 * Replaces triton_dequantize_fp4_to_bf16 / _dequantize_fp4_to_bf16
 * (reference src/home_seek/fused_moe.py:672-710 and fused_moe.py:11-31) and the
 * dequant of load_fp4_weight (src/home_seek/inference_engine/weight_loader.py:35-45).
 * k must be a multiple of 32; row strides are in elements of each tensor
 * (bytes for packed, scale entries, bf16 entries for out) and keep 16-byte
 * alignment of packed rows.
 */
int hsmoe_fp4_dequant_bf16(const void* packed_dev, const void* scale_dev, int scale_kind, int64_t n_rows,
                           int64_t k, int64_t packed_row_stride, int64_t scale_row_stride, void* out_dev,
                           int64_t out_row_stride, hsmoe_stream_t stream);

/* ---------------------------------------------------------------------------
 * FP8 e4m3fn with one scale per 128x128 block -> bf16.
 *   out[n, c] = bf16(fp32(e4m3[n, c]) * scale[n / 128, c / 128])
 * Replaces load_fp8_weight -> cast_back(..., 'bf16', (128, 128))
 * (reference src/home_seek/inference_engine/weight_loader.py:22-32,
 * src/home_seek/_fp4.py:98-110).  scale is fp32 [ceil(n/128), ceil(k/128)].
 */
int hsmoe_fp8_dequant_bf16(const void* data_dev, const float* scale_dev, int64_t n_rows, int64_t k, void* out_dev,
                           hsmoe_stream_t stream);

/* ---------------------------------------------------------------------------
 * Block-scaled dequant of FP4 or FP8 data with any block shape, to fp32 or bf16.
 *   out[n, c] = fp32(code[n, c]) * scale[n / block_rows, c / block_cols]   (one fp32 rounding)
 *   bf16 output: that fp32 value rounded to nearest even.
 * Replaces cast_back for every block size (reference src/home_seek/_fp4.py:98-110:
 * repeat_interleave of the scales, product in fp32, then .to(fp32 | bf16)) and,
 * with one scale 1.0 covering the whole tensor, unpack_from_e2m1fn_x2
 * (_fp4.py:72-95) for any row length.
 * data_kind HSMOE_DATA_FP4: packed bytes [n_rows, k/2] (low nibble = even
 * column, k even); HSMOE_DATA_E4M3: bytes [n_rows, k].  scale: fp32 rows of
 * scale_cols >= ceil(k / block_cols) entries, ceil(n_rows / block_rows) rows.
 * out: [n_rows, k] fp32 (HSMOE_OUT_F32) or bf16 (HSMOE_OUT_BF16), contiguous.
 */
#define HSMOE_DATA_FP4 0
#define HSMOE_DATA_E4M3 1
#define HSMOE_OUT_F32 0
#define HSMOE_OUT_BF16 1
int hsmoe_dequant_blocked(const void* data_dev, int data_kind, const float* scale_dev, int64_t n_rows, int64_t k,
                          int64_t block_rows, int64_t block_cols, int64_t scale_cols, void* out_dev, int out_kind,
                          hsmoe_stream_t stream);

/* ---------------------------------------------------------------------------
 * Router: sqrt(softplus) scores, stable top-k, renormalised weights.
 * Replaces compute_expert_affinity_with_bias / compute_expert_affinity
 * (reference src/home_seek/router.py:10-36) as called by
 * HomeSeekInferenceEngine._compute_routing_experts (engine.py:1025-1031).
 *   logit[m, e] = bf16(x[m] . gate_w[e])        (exact sum, one rounding)
 *   if bias:      logit = bf16(logit + bf16(bias[e]))
 *   score       = sqrt(softplus(float(logit)))  (softplus threshold 20)
 *   idx[m, :]   = indices of the top_k scores, ties -> lower index first
 *   w[m, j]     = score[idx[m, j]] / max(sum_j score[idx[m, j]], 1e-20) * scaling
 * x: bf16 [m, d]; gate_w: bf16 [n_experts, d]; bias: fp32 [n_experts] or NULL.
 * idx_out: int64 [m, top_k]; w_out: fp32 [m, top_k]; logits_out: bf16
 * [m, n_experts] or NULL.  n_experts <= 1024, top_k <= 16, d % 512 == 0, d <= 8192.
 */
size_t hsmoe_router_workspace_size(int64_t m, int64_t n_experts);
int hsmoe_router_topk(const void* x_dev, const void* gate_w_dev, const float* bias_dev, int64_t m, int64_t d,
                      int64_t n_experts, int top_k, float scaling, int64_t* idx_out_dev, float* w_out_dev,
                      void* logits_out_dev, void* workspace_dev, size_t workspace_bytes, hsmoe_stream_t stream);

/* ---------------------------------------------------------------------------
 * Fused routed-expert SwiGLU FFN for m <= 8 tokens (decode, MTP verify).
 * Replaces FusedMoEFFN.forward / .forward_m1_fp4 and, when `shared` is given,
 * the SharedExpertFFN add of _forward_ffn (reference src/home_seek/fused_moe.py:447-563,
 * 573-598, 980-1227; src/home_seek/inference_engine/engine.py:1386-1541).
 *   for every token t and selected expert e (topk_idx[t, j] = e, 0 <= e < n_experts):
 *     gate = x[t] . W1e^T, up = x[t] . W3e^T          (fp32 accumulation)
 *     a    = min(gate, L) * sigmoid(min(gate, L)) * clamp(up, -L, L)
 *     out[t] += topk_w[t, j] * (a . W2e^T)
 *   plus, if shared != NULL, the same FFN of the FP8 shared expert with weight 1.
 * W = bf16(dequant) of the FP4 weights, exactly as hsmoe_fp4_dequant_bf16.
 * expert_table: device uint64 [n_experts][6] = {w1, w1_scale, w3, w3_scale,
 * w2, w2_scale} device addresses, w1/w3 packed [i, d/2], w2 packed [d, i/2],
 * scales [i, d/32] / [d, i/32] of `scale_kind`.  An entry whose w1_scale is 0
 * holds bf16 weights instead (w1/w3 [i, d], w2 [d, i]: the 3-tuple loaders of
 * the reference).  A zero w1 address marks an absent expert (skipped, like a
 * loader returning None).
 * shared: device uint64 [6] of e4m3 w1 [i, d], w3 [i, d], w2 [d, i] and fp32
 * block scales [i/128, d/128], [i/128, d/128], [d/128, i/128] (or, with zero
 * scale addresses, bf16 weights); or NULL.
 * Ids < 0 or >= n_experts are ignored.  out_f32 (fp32 [m, d], optional) and
 * out_bf16 (bf16 [m, d], optional) receive the result.
 * m in [1, 8], d % 512 == 0, i % 512 == 0, top_k <= 16.
 */
size_t hsmoe_moe_decode_workspace_size(int64_t m, int64_t d, int64_t i, int top_k);
int hsmoe_moe_decode(const void* x_dev, int64_t m, int64_t d, int64_t i, const int64_t* topk_idx_dev,
                     const float* topk_w_dev, int top_k, const uint64_t* expert_table_dev, int64_t n_experts,
                     int scale_kind, const uint64_t* shared_dev, float swiglu_limit, float* out_f32_dev,
                     void* out_bf16_dev, void* workspace_dev, size_t workspace_bytes, hsmoe_stream_t stream);

/* The two stages of hsmoe_moe_decode as separate launches (same arguments and
 * workspace): stage 1 computes the weighted SwiGLU activations of every
 * selected expert into the workspace, stage 2 the down projection and the
 * cross-expert sum.  hsmoe_moe_down must follow hsmoe_moe_gate_up on the same
 * stream with the same inputs and workspace.  Lets a caller place other work
 * between the stages or time each one; no separate counterpart in the
 * reference (whose M=1 route also runs a gate/up and a down kernel per expert,
 * fused_moe.py:980-1144). */
int hsmoe_moe_gate_up(const void* x_dev, int64_t m, int64_t d, int64_t i, const int64_t* topk_idx_dev,
                      const float* topk_w_dev, int top_k, const uint64_t* expert_table_dev, int64_t n_experts,
                      int scale_kind, const uint64_t* shared_dev, float swiglu_limit, void* workspace_dev,
                      size_t workspace_bytes, hsmoe_stream_t stream);
int hsmoe_moe_down(const void* x_dev, int64_t m, int64_t d, int64_t i, const int64_t* topk_idx_dev,
                   const float* topk_w_dev, int top_k, const uint64_t* expert_table_dev, int64_t n_experts,
                   int scale_kind, const uint64_t* shared_dev, float* out_f32_dev, void* out_bf16_dev,
                   void* workspace_dev, size_t workspace_bytes, hsmoe_stream_t stream);

/* ---------------------------------------------------------------------------
 * One MoE layer at decode in a single persistent launch: the router of
 * hsmoe_router_topk, then the routed experts and the shared expert of
 * hsmoe_moe_decode, with no host round trip and no launch between them.
 * Replaces HomeSeekInferenceEngine._forward_ffn for m <= 8 tokens (reference
 * src/home_seek/inference_engine/engine.py:1410-1541): _compute_routing_experts
 * (engine.py:1025-1031 -> src/home_seek/router.py:22-36), FusedMoEFFN.forward
 * (src/home_seek/fused_moe.py:447-563) and the shared-expert add
 * (engine.py:1530-1536).
 * Inputs and results are those of the two calls it fuses, and bit-identical
 * to them: x bf16 [m, d]; gate_w bf16 [n_experts, d]; gate_bias fp32
 * [n_experts] or NULL; expert_table / scale_kind / shared as in
 * hsmoe_moe_decode; topk_idx_out int64 [m, top_k] and topk_w_out fp32
 * [m, top_k] receive the routing; logits_out bf16 [m, n_experts] or NULL;
 * out_f32 / out_bf16 as in hsmoe_moe_decode.
 * m in [1, 8], d % 512 == 0, d <= 8192, i % 512 == 0, n_experts <= 256,
 * top_k <= 16 (larger expert counts: hsmoe_router_topk + hsmoe_moe_decode).
 * The workgroups hand work to each other through the workspace, with words
 * tagged by a launch number kept in the workspace; the launch never has more
 * workgroups than the device holds at once.  The workspace is zero-filled
 * once, before its first launch; launches on one stream then need nothing
 * between them, whatever their shapes (every 2^31 launches the last
 * workgroup zeroes the whole workspace and the numbering restarts).  The
 * uint32 at byte hsmoe_moe_layer_status_offset() of the workspace stays 0
 * unless a cross-workgroup wait gave up (then the outputs are not valid).
 */
size_t hsmoe_moe_layer_workspace_size(int64_t m, int64_t d, int64_t i, int64_t n_experts, int top_k);
int hsmoe_moe_layer_decode(const void* x_dev, int64_t m, int64_t d, int64_t i, const void* gate_w_dev,
                           const float* gate_bias_dev, int64_t n_experts, int top_k, float routed_scaling,
                           const uint64_t* expert_table_dev, int scale_kind, const uint64_t* shared_dev,
                           float swiglu_limit, int64_t* topk_idx_out_dev, float* topk_w_out_dev,
                           void* logits_out_dev, float* out_f32_dev, void* out_bf16_dev, void* workspace_dev,
                           size_t workspace_bytes, hsmoe_stream_t stream);
size_t hsmoe_moe_layer_status_offset(void);

/* The same one-launch layer with the routing given instead of computed:
 * routed + shared experts of m <= 8 tokens in one persistent launch.
 * Replaces _forward_ffn on the hash-routed layers (reference
 * src/home_seek/inference_engine/engine.py:1425-1428, _compute_hash_experts
 * engine.py:1018-1023: ids tid2eid[input_ids], every weight 1/k) and
 * FusedMoEFFN.forward with caller-given top-k (src/home_seek/fused_moe.py:
 * 447-563) + the shared-expert add (engine.py:1530-1536), bit-identical to
 * hsmoe_moe_decode on the same ids and weights.
 * token_ids_dev == NULL: topk_idx_dev is int64 [m, top_k].  Otherwise
 * topk_idx_dev is a token table int64 [table_rows, top_k] and token t's ids
 * are row token_ids_dev[t] (a token id outside [0, table_rows) selects no
 * expert).  topk_w_dev: fp32 [m, top_k], or NULL: every weight is weight_all.
 * Ids < 0 or >= n_experts and absent table entries are skipped; an id given
 * twice for one token has its weights added (in k order), as in
 * hsmoe_moe_decode.  Workspace, status word, shapes and outputs as in
 * hsmoe_moe_layer_decode (hsmoe_moe_layer_workspace_size).
 */
int hsmoe_moe_layer_decode_routed(const void* x_dev, int64_t m, int64_t d, int64_t i, const int64_t* topk_idx_dev,
                                  const int64_t* token_ids_dev, int64_t table_rows, const float* topk_w_dev,
                                  float weight_all, int top_k, const uint64_t* expert_table_dev, int64_t n_experts,
                                  int scale_kind, const uint64_t* shared_dev, float swiglu_limit, float* out_f32_dev,
                                  void* out_bf16_dev, void* workspace_dev, size_t workspace_bytes,
                                  hsmoe_stream_t stream);

/* The two one-launch layers above, ended by the next layer's residual adds
 * and RMSNorm in the same launch (the "norm tail"), so that a stack of layers
 * runs one launch per layer.  Replaces, after _forward_ffn, the residual add
 * of the FFN output (reference src/home_seek/inference_engine/engine.py:2690)
 * and the next layer's pre-FFN adds and rms_norm (engine.py:2653-2690,
 * src/home_seek/utils.py:6-9), or the final norm after the last layer
 * (engine.py:2480-2482).  With out = this layer's output rounded to bf16:
 *   h_out    = bf16(bf16(h + out) + residual)   (no second add without residual)
 *   norm_out = RMSNorm(h_out) * weight
 * bit-identical to hsmoe_moe_layer_decode[_routed] with out_bf16 followed by
 * hsmoe_add_rms_norm(h, out_bf16, residual, weight, m, d, eps, h_out,
 * norm_out).  h, h_out, norm_out: bf16 [m, d]; residual: bf16 [d] or NULL;
 * weight: bf16 [d]; h_out may be h; norm_out overlaps no other operand
 * (x included).  out_f32 / out_bf16 may both be NULL here.  Other arguments,
 * workspace and status word as in hsmoe_moe_layer_decode[_routed].
 */
typedef struct hsmoe_norm_tail {
  const void* h_dev;
  const void* residual_dev;
  const void* weight_dev;
  float eps;
  void* h_out_dev;
  void* norm_out_dev;
} hsmoe_norm_tail;
int hsmoe_moe_layer_decode_norm(const void* x_dev, int64_t m, int64_t d, int64_t i, const void* gate_w_dev,
                                const float* gate_bias_dev, int64_t n_experts, int top_k, float routed_scaling,
                                const uint64_t* expert_table_dev, int scale_kind, const uint64_t* shared_dev,
                                float swiglu_limit, int64_t* topk_idx_out_dev, float* topk_w_out_dev,
                                void* logits_out_dev, float* out_f32_dev, void* out_bf16_dev,
                                const hsmoe_norm_tail* tail, void* workspace_dev, size_t workspace_bytes,
                                hsmoe_stream_t stream);
int hsmoe_moe_layer_decode_routed_norm(const void* x_dev, int64_t m, int64_t d, int64_t i,
                                       const int64_t* topk_idx_dev, const int64_t* token_ids_dev, int64_t table_rows,
                                       const float* topk_w_dev, float weight_all, int top_k,
                                       const uint64_t* expert_table_dev, int64_t n_experts, int scale_kind,
                                       const uint64_t* shared_dev, float swiglu_limit, float* out_f32_dev,
                                       void* out_bf16_dev, const hsmoe_norm_tail* tail, void* workspace_dev,
                                       size_t workspace_bytes, hsmoe_stream_t stream);

/* hsmoe_moe_layer_decode without a workspace and without any allocation.
 * No counterpart in the reference: for callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc).  Arguments and results are those of
 * hsmoe_moe_layer_decode, bit for bit, with the library's own scratch in
 * place of the workspace: a static device array of HSMOE_LAYER_SCRATCH_BYTES
 * per GPU, held from the library's load until the process ends.  Shapes whose
 * hsmoe_moe_layer_workspace_size exceeds it are rejected with
 * HSMOE_ERR_WORKSPACE (8 MiB holds m <= 5 at d = 4096, i = 2048, 256 experts,
 * top-6).  status_out: device uint32 that receives 0, or 1 + the code of a
 * cross-workgroup wait that gave up in this launch (its outputs are then not
 * valid).  Every call on one GPU shares that GPU's scratch: calls that overlap
 * on one GPU (other streams, other threads) race and must be serialised by the
 * caller; consecutive calls on one stream need nothing between them.  The
 * first call on a device looks up its scratch and clears it on `stream`.
 */
#define HSMOE_LAYER_SCRATCH_BYTES ((size_t)8 << 20)
int hsmoe_moe_layer_decode_noalloc(const void* x_dev, int64_t m, int64_t d, int64_t i, const void* gate_w_dev,
                                   const float* gate_bias_dev, int64_t n_experts, int top_k, float routed_scaling,
                                   const uint64_t* expert_table_dev, int scale_kind, const uint64_t* shared_dev,
                                   float swiglu_limit, int64_t* topk_idx_out_dev, float* topk_w_out_dev,
                                   void* logits_out_dev, float* out_f32_dev, void* out_bf16_dev,
                                   uint32_t* status_out_dev, hsmoe_stream_t stream);

/* ---------------------------------------------------------------------------
 * Routed-expert SwiGLU FFN for many tokens (prefill, m > 8): a grouped GEMM
 * over the (token, expert) pairs the routing selects.  Replaces
 * FusedMoEFFN.forward at B > 8 (reference src/home_seek/fused_moe.py:447-551,
 * _forward_legacy, whose union route runs every token through every selected
 * expert) and the FP4 grouped route of fused_expert_ffn_triton
 * (fused_moe.py:269-380), plus the shared-expert add of _forward_ffn
 * (src/home_seek/inference_engine/engine.py:1530-1536).
 * Arguments, formats and results as hsmoe_moe_decode (same arithmetic:
 * exact bf16 products, fp32 accumulation, fp32 SwiGLU, hi/lo activation),
 * with out[t] = sum_j topk_w[t, j] * FFN_{topk_idx[t, j]}(x[t]) in slot order j,
 * then + shared FFN(x[t]); a (t, j) with an invalid id or absent expert adds
 * nothing.  Each selected expert's W1 and W3 are read once per chunk of up
 * to 32 of its tokens (64 for an expert with more than 32), its W2 once per
 * chunk of up to 32.  Deterministic (no atomics).
 * 1 <= m * top_k <= 12288, n_experts <= 1024, top_k <= 16, d % 1024 == 0,
 * i % 512 == 0; x and out_f32 16-byte aligned, out_bf16 8-byte aligned.
 * The workspace (any contents) must hold hsmoe_moe_prefill_workspace_size bytes. */
size_t hsmoe_moe_prefill_workspace_size(int64_t m, int64_t d, int64_t i, int64_t n_experts, int top_k);
int hsmoe_moe_prefill(const void* x_dev, int64_t m, int64_t d, int64_t i, const int64_t* topk_idx_dev,
                      const float* topk_w_dev, int top_k, const uint64_t* expert_table_dev, int64_t n_experts,
                      int scale_kind, const uint64_t* shared_dev, float swiglu_limit, float* out_f32_dev,
                      void* out_bf16_dev, void* workspace_dev, size_t workspace_bytes, hsmoe_stream_t stream);

/* ---------------------------------------------------------------------------
 * lm_head logits + greedy argmax + longest-prefix draft acceptance.
 * Replaces the logits / acceptance loop of _mtp_verify_batched
 * (reference src/home_seek/inference_engine/engine.py:2480-2497) and the greedy
 * decode argmax (engine.py:2846-2853).
 *   logits[t, v] = bf16(h[t] . lm_head[v])   (exact sum, one rounding)
 *   pred[t]      = argmax_v logits[t, v]     (first index on ties)
 *   n_accept     = number of leading t < n_tok-1 with pred[t] == ids[t+1]
 *   bonus_row    = n_accept (the first mismatch or the last row)
 * h: bf16 [n_tok, d]; lm_head: bf16 [vocab, d]; ids: int64 [n_tok] (may be
 * NULL when n_tok == 1); logits_out: bf16 [n_tok, vocab] or NULL;
 * pred_out: int64 [n_tok]; result_out: int64 [2] = {n_accept, bonus_row}.
 * n_tok in [1, 8], d % 512 == 0.
 */
size_t hsmoe_lm_head_workspace_size(int64_t n_tok, int64_t vocab);
int hsmoe_lm_head_accept(const void* h_dev, const void* lm_head_dev, int64_t n_tok, int64_t d, int64_t vocab,
                         const int64_t* ids_dev, void* logits_out_dev, int64_t* pred_out_dev,
                         int64_t* result_out_dev, void* workspace_dev, size_t workspace_bytes,
                         hsmoe_stream_t stream);

/* ---------------------------------------------------------------------------
 * RMSNorm of bf16 rows with a bf16 weight (reference src/home_seek/utils.py:6-9):
 *   out[r] = bf16(float(w) * (float(x[r]) * rsqrt(mean(float(x[r])^2) + eps)))
 */
int hsmoe_rms_norm(const void* x_dev, const void* w_dev, int64_t rows, int64_t d, float eps, void* out_dev,
                   hsmoe_stream_t stream);

/* The residual adds of a layer fused in front of its RMSNorm (reference
 * engine.py:2653-2690, the attention output and the FFN output added to the
 * residual stream, as torch bf16 adds: fp32 sum rounded once):
 *   h = x; if add: h = bf16(h + add[r]); if res: h = bf16(h + res)   (res is one [d] row)
 *   h_out[r] = h (if h_out); out[r] = RMSNorm(h) as hsmoe_rms_norm.
 * d must be a multiple of 8 (<= 16384); all rows 16-byte aligned.  hsmoe_rms_norm
 * is this entry point with add = res = h_out = NULL. */
int hsmoe_add_rms_norm(const void* x_dev, const void* add_dev, const void* res_dev, const void* w_dev, int64_t rows,
                       int64_t d, float eps, void* h_out_dev, void* out_dev, hsmoe_stream_t stream);

/* The first layer's input of a forward: the token embedding lookup
 * (engine.py:2475 and 2814, self.embed[ids].to(bfloat16)) followed by hsmoe_add_rms_norm with
 * no add: row r of x is row ids[r] of table [vocab, d] (an id outside
 * [0, vocab) reads zeros), h = bf16(x + res) when res is given,
 * h_out[r] = h, out[r] = RMSNorm(h).  Same arithmetic and order as the lookup
 * followed by hsmoe_add_rms_norm, bit for bit. */
int hsmoe_embed_add_rms_norm(const int64_t* ids_dev, int64_t rows, const void* table_dev, int64_t vocab,
                             const void* res_dev, const void* w_dev, int64_t d, float eps, void* h_out_dev,
                             void* out_dev, hsmoe_stream_t stream);

/* The MTP block's input for one draft token (the data flow of the reference's
 * draft step, engine.py:2251-2339, without its attention and projections):
 *   e = RMSNorm(embed[tok[0]]) * enorm_w;  g = RMSNorm(h_prev) * hnorm_w;
 *   h = bf16(g + e);  if res: h = bf16(h + res);
 *   h_out = h;  out = RMSNorm(h) * w
 * Each RMSNorm and add as hsmoe_add_rms_norm; bit-identical to the lookup,
 * two norms, the add and the add + norm it replaces.  tok: one int64 on the
 * device (read there: no host synchronisation); rows bf16 [d], d % 8 == 0,
 * d <= 8192, 16-byte aligned. */
int hsmoe_mtp_input(const int64_t* tok_dev, const void* embed_dev, int64_t vocab, const void* h_prev_dev,
                    const void* enorm_w_dev, const void* hnorm_w_dev, const void* res_dev, const void* w_dev,
                    int64_t d, float eps, void* h_out_dev, void* out_dev, hsmoe_stream_t stream);

/* One greedy decode step's emission (engine.py:2862-2922 at temperature 0),
 * from the verify's device outputs, with no host synchronisation:
 * tokens = [a, d_0 .. d_{n-1}] (the verify's input ids, n = n_draft <= 15),
 * pred = the verify's argmax per row, result = {n_accept, bonus_row} as
 * hsmoe_lm_head_accept writes them (both unused when n_draft == 0).
 *   row   = [a, d_0 .. d_{n-1}, pred[bonus_row]]   ([a] without drafts)
 *   count = 1 + (n_accept > 0) * (n_accept + 1)    tokens emitted
 *   next  = pred[bonus_row] if n_accept > 0 else a
 * Each output pointer may be NULL.  With rows (then counts, n_accepts, k and
 * capacity >= 1 too): row k of rows [capacity][width] (width n + 2, or 1),
 * counts[k] and n_accepts[k] are written for k = *k in [0, capacity), then
 * *k += 1; *cur = next (if cur).  One single-thread launch. */
int hsmoe_decode_step_record(const int64_t* tokens_dev, int64_t n_draft, const int64_t* pred_dev,
                             const int64_t* result_dev, int64_t* row_out_dev, int64_t* count_out_dev,
                             int64_t* next_out_dev, int64_t* n_accept_out_dev, int64_t* rows_dev,
                             int64_t* counts_dev, int64_t* n_accepts_dev, int64_t* k_dev, int64_t capacity,
                             int64_t* cur_dev, hsmoe_stream_t stream);

/* ---------------------------------------------------------------------------
 * XOR checksum of a device buffer: out (16 bytes) = XOR of the buffer's
 * 16-byte words.  Verifies the HBM expert store (or any slice of it) against a
 * host-side checksum of the same bytes; the checksum of a concatenation is
 * the XOR of its pieces' checksums.  No counterpart in the reference, whose
 * weight loader checks shapes only (src/home_seek/inference_engine/
 * weight_loader.py:48-134); it is also the library's read-only stream, the
 * measure of the HBM read rate a single pass over the weights can reach.
 * nbytes % 16 == 0 (0 gives zeros); data and out 16-byte aligned; workspace of
 * hsmoe_xor_checksum_workspace_size() bytes, any contents.
 */
size_t hsmoe_xor_checksum_workspace_size(void);
int hsmoe_xor_checksum(const void* data_dev, int64_t nbytes, void* out_dev, void* workspace_dev,
                       size_t workspace_bytes, hsmoe_stream_t stream);

/* ---------------------------------------------------------------------------
 * Synthetic data generators (counter-based, reproducible on the host): value i
 * of a stream is derived from r = splitmix64 output number i+1 for seed `key`.
 * These have no counterpart in the reference (which loads a checkpoint); they
 * fill the HBM expert store and the inputs of the benchmarks.
 */
int hsmoe_gen_bytes(uint64_t key, int64_t n, void* out_dev, hsmoe_stream_t stream);
int hsmoe_gen_e4m3(uint64_t key, int64_t n, void* out_dev, hsmoe_stream_t stream);
int hsmoe_gen_e8m0(uint64_t key, int64_t n, int lo, int span, void* out_dev, hsmoe_stream_t stream);
int hsmoe_gen_normal(uint64_t key, int64_t n, float mean, float std, int as_bf16, void* out_dev,
                     hsmoe_stream_t stream);
int hsmoe_gen_uniform(uint64_t key, int64_t n, float lo, float hi, float mul, float* out_dev,
                      hsmoe_stream_t stream);
/* int64 index uniform over [0, n_values): ((r >> 32) * n_values) >> 32. */
int hsmoe_gen_index(uint64_t key, int64_t n, int64_t n_values, int64_t* out_dev, hsmoe_stream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* HSMOE_H_ */
