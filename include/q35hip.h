/*
 * q35hip: C ABI of the MI355X (gfx950) kernels for the Qwen3.5 hybrid-attention hot path.
 *
 * Every entry point takes raw device pointers, explicit int64 sizes and a HIP stream, enqueues its kernels on that
 * stream and returns a status code (Q35_OK or one of the Q35_E* values below). No entry point allocates device
 * memory, synchronises the host, or throws: scratch memory comes from a caller-provided workspace whose size the
 * matching *_workspace_bytes function reports. Tensors are dense and row-major in the layouts stated per function.
 *
 * Reference interfaces replaced (paths relative to the scasella/duo-mech-interp checkout; HF: is
 * transformers 5.15.0 models/qwen3_5/modeling_qwen3_5.py, which the reference's PyTorch mirror
 * tests/engine_ref.py runs):
 *   q35_gdn_recurrent        HF:331-380 torch_recurrent_gated_delta_rule; engine/kernels_qwen35.js:183-247 `delta`
 *   q35_gdn_chunk_prefill    HF:249-327 torch_chunk_gated_delta_rule (chunk_size 64)
 *   q35_gated_attn_prefill   HF:554-589 apply_rotary_pos_emb (partial) + HF:604-626 eager_attention_forward (causal)
 *                            + HF:698 sigmoid gate; engine/kernels_qwen35.js:73-123 `attention`
 *   q35_gated_attn_prefill_cached  the same for T new tokens per row over a KV cache at per-row positions
 *                            (engine/kernels_qwen35.js:90; engine/model.js:486-491 chunked prefill)
 *   q35_gated_attn_decode    same as above for one new token per row over a KV cache (engine/kernels_qwen35.js:73-123
 *                            with T = 1; HF decode through DynamicCache)
 *   q35_gated_attn_decode_proj  the decode step from the fused projection output: engine/kernels_qwen35.js:18-69
 *                            `attnPrep` (q / k RMSNorm, RoPE, cache append) and :73-123 `attention` for T = 1
 *                            in one call (HF:667-701 for one cached token)
 *   q35_gated_attn_prefill_proj  the multi-token attention of a call's own tokens from the fused projection
 *                            output: engine/kernels_qwen35.js:18-69 `attnPrep` and :73-123 `attention` in one call
 *                            (HF:667-701 at positions pos0 .. pos0 + T - 1)
 *   q35_gated_attn_prefill_cached_proj  the same over a KV cache at per-row positions (engine/model.js:486-491
 *                            chunked prefill; HF:667-701 with a DynamicCache)
 *   q35_resid_add_rows       tests/engine_ref.py:49-53 residual vector hook; engine/kernels.js:190-203 `resAdd`
 *   q35_gdn_conv             HF:454-499 (causal_conv1d_fn / causal_conv1d_update + SiLU, split, beta, g);
 *                            engine/kernels_qwen35.js:127-178 `conv` + `convState`, :226-229 (gate terms of `delta`)
 *   q35_gated_rmsnorm        HF:168-184 Qwen3_5RMSNormGated; engine/kernels_qwen35.js:237-243 (epilogue of `delta`)
 *   q35_gdn_chunk_prefill_conv  HF:454-530 for a multi-token call: q35_gdn_conv (fp32) + q35_gdn_chunk_prefill
 *                            (fp32, l2norm on) with the front end in the chunk kernel's load phase;
 *                            engine/kernels_qwen35.js:127-247
 *   q35_gdn_decode_fused     HF:454-543 for one cached token: q35_gdn_conv + q35_gdn_recurrent +
 *                            q35_gated_rmsnorm in one launch; engine/kernels_qwen35.js:127-247
 *   q35_attn_prep            HF:667-680 (q / gate split, q_norm / k_norm, partial RoPE of k, cache update);
 *                            engine/kernels_qwen35.js:18-69 `attnPrep`
 *   q35_gemv                 engine/kernels.js:57-90 `matvec` (int8 weights per 128-input group, or per row)
 *                            and, with the SwiGLU epilogue, engine/kernels_qwen35.js:250-279 `swiglu` with the
 *                            neuron pushes; HF:704-717 Qwen3_5MLP for the decode step
 *   q35_gemv_norm_argmax     q35_gemv_norm (store) with the greedy pick of each row folded in: engine/kernels.js
 *                            :260-283 `argmax` over the logits the LM head writes (engine/model.js:494-497)
 *   q35_gemv_norm            q35_gemv behind the layer's residual add + RMSNorm (HF:753-793, :720-734;
 *                            engine/kernels.js:226-246 `addInto` + `rmsnorm` ahead of the matvec)
 *   q35_swiglu_push          engine/kernels_qwen35.js:250-279 `swiglu` over a [gate | up] projection (prefill form)
 *   q35_gemm_q8              engine/kernels.js:97-151 `matmul` (int8 weights, many rows: the prefill projections),
 *                            with the SwiGLU + push epilogue of `swiglu` (engine/kernels_qwen35.js:250-279)
 *   q35_add_rmsnorm          HF:720-734 Qwen3_5RMSNorm (1 + w) with the residual add before it (HF:753-793);
 *                            engine/kernels.js:226-246 `rmsnorm` (OFFSET) and `addInto`
 *   q35_gemm_q8_bf16,        q35_gemm_q8 on bf16 activations (the attention output; no counterpart either)
 *   q35_gemm_q8_split,       the same on activations handed over already split into bf16 hi + lo parts (no
 *   q35_add_rmsnorm_split,   counterpart in the reference's interface: a layout between the producers and the
 *   q35_gated_rmsnorm_split  GEMM)
 *   q35_argmax_rows          engine/kernels.js:260-283 `argmax` (greedy token of each row, engine/model.js:494-497)
 */
#ifndef Q35HIP_H
#define Q35HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* hipStream_t without pulling in the HIP headers (identical type). */
typedef struct ihipStream_t* q35_stream_t;

enum q35_status {
  Q35_OK = 0,
  Q35_EINVAL = 1,       /* null pointer, non-positive size, or inconsistent sizes */
  Q35_EUNSUPPORTED = 2, /* a size or dtype this build has no kernel for (e.g. head dim other than 128 / 256) */
  Q35_EWORKSPACE = 3,   /* workspace pointer null or smaller than *_workspace_bytes */
  Q35_ELAUNCH = 4,      /* the HIP runtime refused a kernel launch */
  Q35_ESCRATCH = 5      /* an allocation-free entry point's fixed scratch is too small for the request */
};

/* Weight formats of the GEMV / GEMM entry points: Q35_I8 is int8 with one fp32 scale per output row (w_scale [N]);
 * Q35_I8_G128 is the engine's q8 format, int8 with one fp32 scale per group of 128 consecutive inputs of a row
 * (w_scale [N, K / 128] row-major; engine/kernels.js:1-5, :15-47). */
enum q35_dtype { Q35_F32 = 0, Q35_BF16 = 1, Q35_I8 = 2, Q35_I8_G128 = 3 };

/* One neuron push of the MLP hook (engine/model.js:8, :412-423): neuron -1 applies to every neuron of the layer;
 * mode 0 adds vals[row], mode 1 multiplies by it; row = min(m / T, 3) for input row m of a call with T tokens per
 * sequence row. */
typedef struct q35_push {
  int32_t neuron;
  int32_t mode;
  float vals[4];
} q35_push;

/* Human-readable name of a status code (static storage). */
const char* q35_status_string(int status);
/* ABI version of this library: bumped when a signature changes. */
int q35_abi_version(void);

/*
 * Gated delta rule, token-serial form (decode, or any T).
 * Replaces torch_recurrent_gated_delta_rule(query, key, value, g, beta, initial_state, output_final_state,
 * use_qk_l2norm_in_kernel) at HF:331-380, and the recurrence inside the WGSL `delta` kernel
 * (engine/kernels_qwen35.js:229-236).
 *   q, k:  [B, T, Hk, Dk]   dtype           v, out: [B, T, H, Dv]   dtype
 *   g, beta: [B, T, H] fp32 (g is the log decay, alpha = exp(g))
 *   initial_state: [B, H, Dk, Dv] fp32 or NULL (zeros); final_state: [B, H, Dk, Dv] fp32 (may alias initial_state);
 *   both 16-byte aligned (Q35_EUNSUPPORTED otherwise)
 *   H must be a multiple of Hk (q/k head h / (H / Hk) serves value head h, as repeat_interleave at HF:500-502).
 *   Dk = Dv = 128 (the reference engine requires it: engine/model.js:52).
 *   scale multiplies q after the optional l2 normalisation (HF uses 1/sqrt(Dk)).
 */
int q35_gdn_recurrent(const void* q, const void* k, const void* v, const float* g, const float* beta,
                      const float* initial_state, float* final_state, void* out,
                      int64_t B, int64_t T, int64_t Hk, int64_t H, int64_t Dk, int64_t Dv,
                      int dtype, float scale, int use_qk_l2norm, q35_stream_t stream);

/*
 * Gated delta rule, chunked form (prefill). Replaces torch_chunk_gated_delta_rule at HF:249-327: the same
 * arguments and layouts as q35_gdn_recurrent, chunk_size 64 (the only size this build supports). T need not be a
 * multiple of 64 (the tail chunk is zero-padded as HF:271-277 does). Needs a workspace of
 * q35_gdn_chunk_workspace_bytes(B, T, H, Dk, Dv, 64, dtype) bytes (256-byte aligned).
 * The arithmetic follows the input dtype: bf16 q/k/v use bf16 MFMA products with fp32 accumulation (relative error
 * a few 1e-3 against the fp32 recurrence); fp32 q/k/v compute every product in fp32 (agreement with the fp32
 * recurrence to fp32 rounding, about 1e-6). The state is fp32 in both.
 */
size_t q35_gdn_chunk_workspace_bytes(int64_t B, int64_t T, int64_t H, int64_t Dk, int64_t Dv, int64_t chunk_size,
                                     int dtype);
int q35_gdn_chunk_prefill(const void* q, const void* k, const void* v, const float* g, const float* beta,
                          const float* initial_state, float* final_state, void* out,
                          int64_t B, int64_t T, int64_t Hk, int64_t H, int64_t Dk, int64_t Dv,
                          int dtype, float scale, int use_qk_l2norm, int64_t chunk_size,
                          void* workspace, size_t workspace_bytes, q35_stream_t stream);

/*
 * Gated causal GQA softmax attention over one call's tokens, with partial rotary embedding and the sigmoid output
 * gate fused. Replaces, at HF:656-698, apply_rotary_pos_emb -> attention_interface (eager_attention_forward,
 * HF:604-626, causal mask, softmax in fp32) -> reshape -> * sigmoid(gate); and the WGSL `attention` kernel
 * (engine/kernels_qwen35.js:73-123) plus the rotary part of `attnPrep` (engine/kernels_qwen35.js:50-59).
 *   q: [B, T, Hq, D] bf16   k, v: [B, T, Hkv, D] bf16   gate: [B, T, Hq * D] bf16   out: [B, T, Hq * D] bf16
 *   cos, sin: [P, rot / 2] fp32 tables by absolute position (position of token t is pos0 + t, P > pos0 + T - 1);
 *   rotary pairs (i, i + rot/2) on the first rot dims (rotate_half, HF:546-551). rot = 0 disables the rotation.
 *   scale is the softmax scale (HF: head_dim ** -0.5). D = 256, Hq / Hkv in {1, 2, 4, 8}.
 *   Needs q35_gated_attn_prefill_workspace_bytes(B, T, Hq, Hkv, D) bytes of workspace (256-byte aligned): the
 *   keys rotated once and the values transposed once ([B, Hkv, T rounded up to 64, D] bf16 each) and, for long
 *   sequences, the fp32 partial results of the query blocks whose keys are split over two work items (combined by
 *   a third kernel). The workspace is overwritten by every call; calls that share one workspace must not overlap.
 */
size_t q35_gated_attn_prefill_workspace_bytes(int64_t B, int64_t T, int64_t Hq, int64_t Hkv, int64_t D);
int q35_gated_attn_prefill(const void* q, const void* k, const void* v, const void* gate,
                           const float* cos, const float* sin, int64_t pos0, void* out,
                           int64_t B, int64_t T, int64_t Hq, int64_t Hkv, int64_t D, int64_t rot,
                           float scale, void* workspace, size_t workspace_bytes, q35_stream_t stream);

/*
 * Gated causal GQA attention of T new tokens per row over a bf16 KV cache that already holds their keys and values
 * (written by q35_attn_prep): the reference's multi-token attention, where token t of a call at position pos[r]
 * attends to cache keys 0 .. pos[r] + t (engine/kernels_qwen35.js:90, n = pos + t + 1; prefill in chunks,
 * engine/model.js:486-491), and HF:656-698 over a DynamicCache. Rows may sit at different positions.
 *   q: [B, T, Hq, D] bf16, not rotated (rotated here at position pos[b] + t)   gate: [B, T, Hq * D] bf16
 *   k_cache, v_cache: [B, Hkv, max_len, D] bf16, keys rotated; max_len a multiple of 64 (Q35_EUNSUPPORTED otherwise)
 *   pos: [B] int32 on the device, clamped to 0 .. max_len - T; cos, sin: [P, rot / 2] fp32, P >= max_len
 *   out: [B, T, Hq * D] bf16. D = 256, Hq / Hkv in {1, 2, 4, 8}, rot a multiple of 16 (at most 64).
 *   Needs q35_gated_attn_prefill_cached_workspace_bytes(B, Hkv, D, max_len) bytes of workspace (256-byte aligned:
 *   the values of the rows' key ranges, transposed). Calls that share one workspace must not overlap.
 */
size_t q35_gated_attn_prefill_cached_workspace_bytes(int64_t B, int64_t Hkv, int64_t D, int64_t max_len);
int q35_gated_attn_prefill_cached(const void* q, const void* k_cache, const void* v_cache, const void* gate,
                                  const int32_t* pos, const float* cos, const float* sin, void* out, int64_t B,
                                  int64_t T, int64_t Hq, int64_t Hkv, int64_t D, int64_t max_len, int64_t rot,
                                  float scale, void* workspace, size_t workspace_bytes, q35_stream_t stream);

/*
 * Gated GQA attention for one new token per row over a bf16 KV cache (split-K over the context, then a merge).
 *   q: [B, Hq, D] bf16 (not yet rotated; rotated here at position cache_len[b] - 1)
 *   k_cache, v_cache: [B, Hkv, max_len, D] bf16, keys already rotated; row b uses keys 0 .. cache_len[b] - 1
 *   cache_len: [B] int32 on the device (1 <= cache_len[b] <= max_len)
 *   gate: [B, Hq * D] bf16    out: [B, Hq * D] in out_dtype (Q35_BF16, or Q35_F32 for an fp32 consumer)
 *   cos, sin: [P, rot / 2] fp32 by position (P >= max_len); rot a multiple of 8 (Q35_EUNSUPPORTED otherwise)
 *   splits <= 0 lets the library choose the split count (a request is rounded to whole 64-key multiples of a
 *   power-of-two span, so the count used may be lower). Needs
 *   q35_gated_attn_decode_workspace_bytes(B, Hq, Hkv, D, max_len, splits) bytes of workspace.
 */
size_t q35_gated_attn_decode_workspace_bytes(int64_t B, int64_t Hq, int64_t Hkv, int64_t D, int64_t max_len,
                                             int64_t splits);
int q35_gated_attn_decode(const void* q, const void* k_cache, const void* v_cache, const void* gate,
                          const int32_t* cache_len, const float* cos, const float* sin, void* out, int out_dtype,
                          int64_t B, int64_t Hq, int64_t Hkv, int64_t D, int64_t max_len, int64_t rot,
                          float scale, int64_t splits, void* workspace, size_t workspace_bytes,
                          q35_stream_t stream);

/*
 * The attention decode step from the fused projection output of one token per row (engine/kernels_qwen35.js:18-69
 * `attnPrep` followed by :73-123 `attention` with T = 1; HF:667-701 with a DynamicCache): y [B, ldy] fp32 rows
 * holding [q | gate] per query head (Hq * 2D), then k (Hkv * D), then v (Hkv * D) from column 0. q and k are
 * normalised with (1 + q_norm_w / k_norm_w) (RMS, eps) and rotated at position pos[b] (device int32, so that a
 * captured step replays at the row's current position); the token attends to cache keys 0 .. pos[b] - 1 and to
 * itself; its rotated key and its value are written into k_cache / v_cache at pos[b] (bf16, when pos[b] < max_len).
 * out = attention * sigmoid(gate), [B, Hq * D] in out_dtype. Same workspace as q35_gated_attn_decode
 * (q35_gated_attn_decode_workspace_bytes), same limits (D 256, Hq / Hkv in 1, 2, 4, 8, rot a multiple of 8); y,
 * ldy and the norm weights 16-byte aligned. The cached keys are those the front end (q35_attn_prep) would have
 * written, and the key written here is bitwise the one it writes.
 */
int q35_gated_attn_decode_proj(const float* y, int64_t ldy, const float* q_norm_w, const float* k_norm_w, float eps,
                               void* k_cache, void* v_cache, const int32_t* pos, const float* cos, const float* sin,
                               void* out, int out_dtype, int64_t B, int64_t Hq, int64_t Hkv, int64_t D,
                               int64_t max_len, int64_t rot, float scale, int64_t splits, void* workspace,
                               size_t workspace_bytes, q35_stream_t stream);

/*
 * Gated causal GQA attention of the call's own T tokens per row from their fused projection output
 * (engine/kernels_qwen35.js:18-69 `attnPrep` followed by :73-123 `attention`; HF:667-701 for a prompt at positions
 * pos0 .. pos0 + T - 1 with nothing cached before pos0 attended to): y holds B * T rows (row b T + t, stride ldy) of
 * fp32 [q | gate] per query head (Hq * 2D), then k (Hkv * D), then v (Hkv * D) from column 0. q and k are normalised
 * with (1 + q_norm_w / k_norm_w) (RMS, eps) and rotated at position pos0 + t; token t attends to the call's tokens
 * 0 .. t. The rotated keys and the values are written into k_cache / v_cache [B, Hkv, max_len, D] bf16 at rows
 * pos0 + t (pos0 + T <= max_len), bitwise the rows q35_attn_prep writes. out = attention * sigmoid(gate),
 * [B, T, Hq * D] bf16. Limits as q35_gated_attn_prefill (D 256, Hq / Hkv in 1, 2, 4, 8, rot a multiple of 16, at
 * most 64); y, ldy and the norm weights 16-byte aligned; cos, sin [P, rot / 2] fp32 with P >= pos0 + T. Needs
 * q35_gated_attn_prefill_proj_workspace_bytes(B, T, Hq, Hkv, D) bytes of workspace (256-byte aligned); calls that
 * share one workspace must not overlap.
 */
size_t q35_gated_attn_prefill_proj_workspace_bytes(int64_t B, int64_t T, int64_t Hq, int64_t Hkv, int64_t D);
int q35_gated_attn_prefill_proj(const float* y, int64_t ldy, const float* q_norm_w, const float* k_norm_w, float eps,
                                void* k_cache, void* v_cache, int64_t pos0, const float* cos, const float* sin,
                                void* out, int64_t B, int64_t T, int64_t Hq, int64_t Hkv, int64_t D, int64_t max_len,
                                int64_t rot, float scale, void* workspace, size_t workspace_bytes,
                                q35_stream_t stream);

/*
 * The multi-token attention over a bf16 KV cache from the fused projection output (engine/kernels_qwen35.js:18-69
 * `attnPrep` followed by :73-123 `attention`, token t of row b at position P_b + t with P_b = pos[b] clamped to
 * 0 .. max_len - T; engine/model.js:486-491 chunked prefill; HF:667-701 with a DynamicCache): y as for
 * q35_gated_attn_prefill_proj. q and k are normalised and rotated at P_b + t; the tokens' rotated keys and values
 * are written into k_cache / v_cache at rows P_b + t (bitwise the rows q35_attn_prep writes for positions with
 * pos[b] + T <= max_len), and token t attends to cache keys 0 .. P_b + t. out [B, T, Hq * D] bf16. Limits as
 * q35_gated_attn_prefill_cached (max_len a multiple of 64); y, ldy and the norm weights 16-byte aligned. Needs
 * q35_gated_attn_prefill_cached_proj_workspace_bytes(B, T, Hq, Hkv, D, max_len) bytes of workspace (256-byte
 * aligned); calls that share one workspace must not overlap.
 */
size_t q35_gated_attn_prefill_cached_proj_workspace_bytes(int64_t B, int64_t T, int64_t Hq, int64_t Hkv, int64_t D,
                                                          int64_t max_len);
int q35_gated_attn_prefill_cached_proj(const float* y, int64_t ldy, const float* q_norm_w, const float* k_norm_w,
                                       float eps, void* k_cache, void* v_cache, const int32_t* pos, const float* cos,
                                       const float* sin, void* out, int64_t B, int64_t T, int64_t Hq, int64_t Hkv,
                                       int64_t D, int64_t max_len, int64_t rot, float scale, void* workspace,
                                       size_t workspace_bytes, q35_stream_t stream);

/*
 * q35_gated_attn_decode without a workspace argument, for callers that cannot allocate device memory (code under HIP
 * graph capture, tight serving loops, harnesses that forbid allocation). This entry point has no counterpart in the
 * reference. The split-K partials go to a fixed device array of q35_gated_attn_decode_noalloc_max_bytes() bytes
 * (9 MiB; one copy per device, held until the process ends); a call whose q35_gated_attn_decode_workspace_bytes(...)
 * exceeds it returns Q35_ESCRATCH without launching (9 MiB covers B <= 142 at an 8192-token cache with Hq 8, Hkv 2,
 * D 256 and the default splits: 66,048 bytes of partials per row).
 * The stream's device must be the current device. Calls that overlap on one device race for the array. No memory
 * is allocated or freed; the array's device address is looked up on the first call per device. Arguments and
 * results are otherwise exactly those of q35_gated_attn_decode (same kernels, bitwise identical outputs).
 */
size_t q35_gated_attn_decode_noalloc_max_bytes(void);
int q35_gated_attn_decode_noalloc(const void* q, const void* k_cache, const void* v_cache, const void* gate,
                                  const int32_t* cache_len, const float* cos, const float* sin, void* out,
                                  int out_dtype, int64_t B, int64_t Hq, int64_t Hkv, int64_t D, int64_t max_len,
                                  int64_t rot, float scale, int64_t splits, q35_stream_t stream);

/*
 * Residual steering add: x[r, t, :] += vecs[vec_of_row[r], :] for every row r and position t; rows whose index is
 * negative are left alone. Replaces the layer-12 forward hook of tests/engine_ref.py:49-53 (out + s * vec at every
 * position) and the WGSL `resAdd` (engine/kernels.js:190-203, vector row = min(row, 3)).
 *   x: [rows, T, H] dtype (fp32 or bf16)   vecs: [nvec, H] fp32   vec_of_row: [rows] int32 on the device, or NULL
 *   for min(r, nvec - 1) as the WGSL kernel does.
 */
int q35_resid_add_rows(void* x, const float* vecs, const int32_t* vec_of_row, int64_t rows, int64_t T, int64_t H,
                       int64_t nvec, int dtype, q35_stream_t stream);

/*
 * Gated DeltaNet front end over the fused projection output y (one row per token):
 *   y: [B, T, ldy] fp32, columns [0, C) the q|k|v channels (C = 2 Hk dk + Hv dv), columns b_off .. b_off + Hv the
 *      beta logits b, a_off .. a_off + Hv the decay inputs a
 *   conv_w: [C, K] fp32, conv_bias: [C] fp32 or NULL; conv_state: [B, K - 1, C] fp32, the previous K - 1 inputs
 *      (oldest first), advanced in place by the call's T inputs
 *   A_log, dt_bias: [Hv] fp32
 *   out: q, k [B, T, Hk, dk] and v [B, T, Hv, dv] in dtype (silu(causal conv)), g, beta [B, T, Hv] fp32 with
 *      beta = sigmoid(b), g = -exp(A_log) * softplus(a + dt_bias) (softplus threshold 20)
 *   K <= 8; y, conv_state (and conv_bias) 16-byte aligned, ldy, dk * Hk and dv * Hv multiples of 4.
 */
int q35_gdn_conv(const float* y, int64_t ldy, const float* conv_w, const float* conv_bias, float* conv_state,
                 const float* A_log, const float* dt_bias, int64_t b_off, int64_t a_off, void* q, void* k, void* v,
                 float* g, float* beta, int64_t B, int64_t T, int64_t Hk, int64_t dk, int64_t Hv, int64_t dv,
                 int64_t K, int dtype, q35_stream_t stream);

/*
 * A Gated DeltaNet layer's multi-token call after its input projection, up to the gated norm: q35_gdn_conv with fp32
 * outputs followed by q35_gdn_chunk_prefill on them (fp32 path, use_qk_l2norm on, chunk 64), with the conv + SiLU,
 * the l2 norms and the gate terms computed in the chunk kernel's load phase, so that q, k, v, g and beta are never
 * written out. The same arithmetic in the same order as that pair of calls (the same results, bit for bit).
 * HF:454-530 (causal_conv1d_fn + SiLU, split, beta / g, torch_chunk_gated_delta_rule); engine/kernels_qwen35.js
 * :127-247 (`conv`, `convState`, `delta`).
 *   y, conv_w [C, conv_k], conv_bias, conv_state [B, conv_k - 1, C], A_log, dt_bias, b_off, a_off: as q35_gdn_conv,
 *      conv_state advanced in place; conv_k must be 4 (Qwen3.5's conv kernel size); conv_w 16-byte aligned too
 *   initial_state (or NULL: zeros), final_state [B, H, 128, 128] fp32 (they may be the same buffer: the state is
 *      then advanced in place); out [B, T, H, 128] fp32; Hk k heads, H v heads (H % Hk == 0), Dk = Dv = 128
 *   workspace: q35_gdn_chunk_workspace_bytes(B, T, H, 128, 128, 64, Q35_F32) bytes, 256-byte aligned
 */
int q35_gdn_chunk_prefill_conv(const float* y, int64_t ldy, const float* conv_w, const float* conv_bias,
                               float* conv_state, const float* A_log, const float* dt_bias, int64_t b_off,
                               int64_t a_off, const float* initial_state, float* final_state, float* out,
                               int64_t B, int64_t T, int64_t Hk, int64_t H, int64_t Dk, int64_t Dv, int64_t conv_k,
                               float scale, void* workspace, size_t workspace_bytes, q35_stream_t stream);

/*
 * One decode step of a Gated DeltaNet layer after its input projection, fused: q35_gdn_conv (T = 1), then
 * q35_gdn_recurrent (one token, l2norm on, fp32) on the head's state, then q35_gated_rmsnorm, with the same
 * arithmetic in the same reduction order (results equal to fp32 rounding). HF:454-543 for one cached token
 * (causal_conv1d_update, torch_recurrent_gated_delta_rule, Qwen3_5RMSNormGated); engine/kernels_qwen35.js:127-247
 * (`conv`, `convState`, `delta`).
 *   y: [B, ldy] fp32 with the q|k|v channels at [0, C), C = 3 H d (Hk = Hv = H, dk = dv = d), z at z_off, b at b_off,
 *      a at a_off; conv_w [C, K], conv_bias [C] or NULL, conv_state [B, K - 1, C] (advanced in place);
 *   A_log, dt_bias, head_scale (or NULL): [H]; norm_w: [d]; state: [B, H, d, d] fp32 (updated in place);
 *   scale: the q scale (1 / sqrt(d)); out: [B, H d] fp32, the gated-normed output.
 *   d = 128, K <= 8; y, conv_state, state (and conv_bias) 16-byte aligned, ldy a multiple of 4.
 */
int q35_gdn_decode_fused(const float* y, int64_t ldy, const float* conv_w, const float* conv_bias,
                         float* conv_state, const float* A_log, const float* dt_bias, int64_t b_off, int64_t a_off, int64_t z_off,
                         float* state, const float* norm_w, const float* head_scale, float eps, float scale,
                         float* out, int64_t B, int64_t H, int64_t d, int64_t K, q35_stream_t stream);

/*
 * The recurrent part of one GDN decode step, for a projection row whose q|k|v channels already went through the
 * causal conv + SiLU (q35_gemv_norm_conv): q35_gdn_recurrent (one token, l2norm on, fp32) on the head's state with
 * beta = sigmoid(b) and g = -exp(A_log) softplus(a + dt_bias) from the row, leaving out the gated RMSNorm (the
 * output projection applies it: q35_gemv_gated_norm). HF:454-543 for one cached token from the recurrent rule on;
 * engine/kernels_qwen35.js:183-236 (`delta` before its gated norm). The column sums are formed in the order of
 * q35_gdn_decode_fused, over four blocks per (head, row).
 *   y: [B, ldy] fp32, q|k|v (convolved) at [0, 3 H d), b at b_off, a at a_off; A_log, dt_bias: [H];
 *   state: [B, H, d, d] fp32 (updated in place); out: [B, H d] fp32, the raw output o.
 *   d = 128; y, state, out 16-byte aligned, ldy a multiple of 4.
 */
int q35_gdn_decode_sliced(const float* y, int64_t ldy, const float* A_log, const float* dt_bias, int64_t b_off,
                          int64_t a_off, float* state, float scale, float* out, int64_t B, int64_t H, int64_t d,
                          q35_stream_t stream);

/*
 * Gated RMSNorm per (token, head): out = w * (o * rsqrt(mean(o^2) + eps)) * silu(z) * head_scale[h], the
 * normalised o rounded to dtype before the weight multiply as HF does (plain w, not 1 + w).
 *   o, out: [M, Hv, dv] dtype (may alias); z: [M, ldz] fp32, head h's gate at columns h dv .. h dv + dv - 1;
 *   w: [dv] fp32; head_scale: [Hv] fp32 or NULL (ones). dv = 128.
 */
int q35_gated_rmsnorm(const void* o, const float* z, int64_t ldz, const float* w, const float* head_scale, void* out,
                      int64_t M, int64_t Hv, int64_t dv, float eps, int dtype, q35_stream_t stream);

/*
 * q35_gated_rmsnorm on fp32 o with out written in the int8 GEMM's split layout (each value as hi = bf16(v),
 * lo = bf16(v - hi); per row of Hv dv values, each group of 8 as its 8 hi parts then its 8 lo parts): the input of
 * the output projection's q35_gemm_q8_split. out: [M, Hv dv] 4-byte words, 16-byte aligned. Same reference lines.
 */
int q35_gated_rmsnorm_split(const float* o, const float* z, int64_t ldz, const float* w, const float* head_scale,
                            void* out, int64_t M, int64_t Hv, int64_t dv, float eps, q35_stream_t stream);

/*
 * Gated-attention front end over the fused projection output y: [B, T, ldy] fp32 holding per token
 * [q_proj (Hq heads of [q (D) | gate (D)]) | k_proj (Hkv x D) | v_proj (Hkv x D)].
 *   q_norm_w, k_norm_w: [D] fp32, RMSNorm with (1 + w) in fp32; cos, sin: [P, rot / 2] fp32 by absolute position
 *   pos: [B] int32 on the device, the position of each row's first token of this call
 *   out: q_out [B, T, Hq, D] bf16 (normalised, not rotated), gate_out [B, T, Hq * D] bf16, k_out / v_out
 *        [B, T, Hkv, D] bf16 (normalised unrotated keys / values; either may be NULL), and the caches
 *        k_cache, v_cache [B, Hkv, max_len, D] bf16 receive the rotated keys and the values at positions pos[b] + t
 *        (positions at or past max_len are not written)
 *   D = 256, rot a multiple of 8; y 16-byte aligned, ldy a multiple of 4.
 */
int q35_attn_prep(const float* y, int64_t ldy, const float* q_norm_w, const float* k_norm_w, float eps,
                  const float* cos, const float* sin, int64_t rot, const int32_t* pos, void* q_out, void* gate_out,
                  void* k_out, void* v_out, void* k_cache, void* v_cache, int64_t max_len, int64_t B, int64_t T,
                  int64_t Hq, int64_t Hkv, int64_t D, q35_stream_t stream);

/*
 * Residual add + RMSNorm with (1 + w) per row: x[m] += y[m] in place (y may be NULL: no add), then
 * h[m] = x[m] * rsqrt(mean(x[m]^2) + eps) * (1 + w), all fp32. x: [M, ldx], y: [M, ldy], h: [M, ldh], w: [H];
 * H a multiple of 4 and at most 8192; pointers 16-byte aligned, leading dimensions multiples of 4.
 */
int q35_add_rmsnorm(float* x, int64_t ldx, const float* y, int64_t ldy, const float* w, float* h, int64_t ldh,
                    int64_t M, int64_t H, float eps, q35_stream_t stream);

/*
 * q35_add_rmsnorm with h written in the split layout that q35_gemm_q8_split reads (the same norm, then each value
 * as hi = bf16(h), lo = bf16(h - hi), rounded to nearest even; per row, each group of 8 inputs is 32 bytes: the 8
 * hi parts, then the 8 lo parts). hs: [M, ldh] 4-byte words (the bytes of an fp32 [M, ldh] array), H a multiple
 * of 8; everything else as q35_add_rmsnorm. Same reference lines (the norm before the prefill projections).
 */
int q35_add_rmsnorm_split(float* x, int64_t ldx, const float* y, int64_t ldy, const float* w, void* hs, int64_t ldh,
                          int64_t M, int64_t H, float eps, q35_stream_t stream);

/*
 * Small-M matrix-vector product for the decode step: y[m, n] = sum_k x[m, k] W[n, k] s(n, k), m < M <= 8, with
 * s(n, k) = w_scale[n] for Q35_I8, w_scale[n, k / 128] for Q35_I8_G128, 1 for Q35_F32 (w_scale NULL).
 *   x: [M, ldx] fp32 (16-byte aligned, ldx a multiple of 4); W: [N, K] row-major int8 or fp32 (w_dtype);
 *   K a multiple of 256, M * K * 4 <= 64 KiB.
 *   epilogue 0: y[m, n] = v; 1: y[m, n] += v (a residual add); 2: SwiGLU over interleaved row pairs (row 2 j the
 *   gate, row 2 j + 1 the up projection of neuron j): y[m, j] = silu(v_2j) * v_2j+1, then the pushes in order.
 *   y: [M, ldy] fp32 (ldy >= N, or >= N / 2 for epilogue 2). pushes: npush <= 64 records on the device (or NULL
 *   with npush 0); T: tokens per sequence row (the push row is min(m / T, 3)).
 *   Epilogue 1 with fewer than 256 blocks of 16 output rows splits K over several blocks that add their sums into
 *   y with fp32 atomics: the order of those additions, and so the last bits of y, may differ between calls.
 *   Epilogue 4 is epilogue 1 with every output summed in one fixed order (no split over K: a product with fewer
 *   than 256 blocks of 16 rows takes blocks of 4 rows instead), so that repeated calls give identical bits; it is
 *   the deterministic form of the decode step's residual adds (the engine's matvec sums in a fixed order).
 *   cap: the neuron activation capture of the MLP hook (engine/model.js:9, :451-453; the `cap` binding of
 *   engine/kernels_qwen35.js:251-279, its capOff folded into the pointer), NULL for none, epilogue 2 only: the
 *   activation of neuron j of row m (after the pushes, as y holds it) is also written to
 *   cap[(m / T) ld_cap_row + (m % T) ld_cap + j] in fp32 (ld_cap, ld_cap_row >= N / 2; 4-byte aligned), e.g.
 *   [sequence row][token][neuron] slices of a [layers, rows, tokens, neurons] buffer.
 */
int q35_gemv(const float* x, int64_t ldx, const void* W, int w_dtype, const float* w_scale, float* y, int64_t ldy,
             int64_t M, int64_t N, int64_t K, int epilogue, const q35_push* pushes, int64_t npush, int64_t T,
             float* cap, int64_t ld_cap, int64_t ld_cap_row, q35_stream_t stream);

/*
 * q35_gemv with the decoder layer's residual add + RMSNorm in front (HF:753-793 then HF:720-734; the engine's
 * addInto + rmsnorm, engine/kernels.js:226-246, fused into its matvec): s = x + x_add (x_add may be NULL), written to
 * x_out when x_out is not NULL, and the product takes h = s * rsqrt(mean(s^2) + eps) * (1 + norm_w) in place of x.
 *   x, x_add, x_out: [M, ldx] fp32, 16-byte aligned; x_out must not overlap x or x_add (Q35_EINVAL); norm_w: [K]
 *   fp32. Everything else as q35_gemv.
 */
int q35_gemv_norm(const float* x, const float* x_add, float* x_out, int64_t ldx, const float* norm_w, float eps,
                  const void* W, int w_dtype, const float* w_scale, float* y, int64_t ldy, int64_t M, int64_t N,
                  int64_t K, int epilogue, const q35_push* pushes, int64_t npush, int64_t T, float* cap,
                  int64_t ld_cap, int64_t ld_cap_row, q35_stream_t stream);

/*
 * q35_gemv_norm with the store epilogue (y = the logits, as that call writes them) and the argmax of each row of y
 * written to idx [M] int32: the lowest index among the largest values, as q35_argmax_rows (NaN never wins; a row with
 * no winner reports 0). The blocks fold their best (value, index) into slots [M] (uint64, 8-byte aligned) with one
 * atomic max each, and a one-block kernel then turns the slots into indices and clears them: slots must hold zeros
 * before the first call, and every call leaves them zero (calls sharing slots must not overlap).
 */
int q35_gemv_norm_argmax(const float* x, const float* x_add, float* x_out, int64_t ldx, const float* norm_w,
                         float eps, const void* W, int w_dtype, const float* w_scale, float* y, int64_t ldy,
                         int64_t M, int64_t N, int64_t K, uint64_t* slots, int32_t* idx, q35_stream_t stream);

/*
 * q35_gemv_norm (store epilogue) whose outputs 0 .. conv_channels - 1 go through the GDN layer's causal conv + SiLU
 * before they are stored: for output channel c of row m, silu(conv_bias[c] + sum_i conv_w[c, i] x_i) over the
 * channel's last conv_k inputs (the conv_k - 1 of conv_state[m, :, c], then this product), and conv_state[m, :, c]
 * advanced by one input. The same arithmetic as q35_gdn_conv at T = 1 (HF:454-475 causal_conv1d_update;
 * engine/kernels_qwen35.js:127-178). Each channel belongs to one block, so the state is updated in place.
 *   conv_w: [conv_channels, conv_k] fp32, conv_bias: [conv_channels] or NULL, conv_state: [M, conv_k - 1,
 *   conv_channels] fp32; 2 <= conv_k <= 8, N at most 16384 (8192 for M > 4). Everything else as q35_gemv_norm.
 */
int q35_gemv_norm_conv(const float* x, const float* x_add, float* x_out, int64_t ldx, const float* norm_w, float eps,
                       const void* W, int w_dtype, const float* w_scale, float* y, int64_t ldy, int64_t M, int64_t N,
                       int64_t K, const float* conv_w, const float* conv_bias, float* conv_state,
                       int64_t conv_channels, int64_t conv_k, q35_stream_t stream);

/*
 * q35_gemv of the gated RMSNorm of o (the GDN layer's output norm, HF:168-184; engine/kernels_qwen35.js:237-243),
 * computed per head of 128 inputs while x is staged: x = norm_w * (o * rsqrt(mean(o^2) + eps)) * silu(z) *
 * head_scale[h], in the order of q35_gdn_decode_fused's norm, then y (epilogue 0) = or (epilogue 1) += x W^T s.
 *   o: [M, ldo] fp32 (16-byte aligned), K = H 128 inputs; z: [M, ldz] fp32 (16-byte aligned, ldz a multiple of 4),
 *   head h's gate at columns 128 h .. 128 h + 127; norm_w: [128] fp32; head_scale: [H] or NULL. int8 weights only
 *   (Q35_I8 or Q35_I8_G128). epilogue 0, 1 or 4; everything else as q35_gemv (including the split-K accumulation
 *   of epilogue 1 and the fixed order of epilogue 4).
 */
int q35_gemv_gated_norm(const float* o, int64_t ldo, const float* z, int64_t ldz, const float* norm_w,
                        const float* head_scale, float eps, const void* W, int w_dtype, const float* w_scale,
                        float* y, int64_t ldy, int64_t M, int64_t N, int64_t K, int epilogue, q35_stream_t stream);

/*
 * Many-row int8 GEMM for the prefill projections: y[m, n] = sum_k x[m, k] W[n, k] s(n, k), s as for q35_gemv
 * (w_dtype Q35_I8: w_scale [N]; Q35_I8_G128: w_scale [N, K / 128], K a multiple of 128). Replaces the engine's int8
 * `matmul` (engine/kernels.js:97-151, used when M > 32) and, with the SwiGLU epilogue, its `swiglu` with the neuron
 * pushes (engine/kernels_qwen35.js:250-279); HF:704-717 and the mixers' projections in fp32.
 *   x: [M, ldx] fp32 (16-byte aligned, ldx a multiple of 4); W: [N, K] int8 row-major (16-byte aligned), K a multiple
 *   of 64; y: [M, ldy] fp32. fp32-accurate: bf16 MFMA products of W (exact in bf16) with a hi + lo split of x
 *   (relative error about 1e-5); with group scales each group's partial product is scaled in fp32.
 *   epilogue 0: y = v; 1: y += v; 2: SwiGLU over interleaved row pairs (row 2 j gate, 2 j + 1 up of neuron j):
 *   y[m, j] = silu(v_2j) * v_2j+1 then the pushes in order (N even, ldy >= N / 2); 3: as 2 with y written in the
 *   split layout of q35_gemm_q8_split's input (N / 2 a multiple of 8, ldy a multiple of 4, y 16-byte aligned), the
 *   down projection's input. pushes, npush <= 64 and T as for q35_gemv; cap, ld_cap, ld_cap_row (epilogues 2 and 3:
 *   the fp32 activations whatever the layout of y) as for q35_gemv.
 */
int q35_gemm_q8(const float* x, int64_t ldx, const int8_t* W, int w_dtype, const float* w_scale, float* y,
                int64_t ldy, int64_t M, int64_t N, int64_t K, int epilogue, const q35_push* pushes, int64_t npush,
                int64_t T, float* cap, int64_t ld_cap, int64_t ld_cap_row, q35_stream_t stream);

/*
 * q35_gemm_q8 on x already split by its producer (q35_add_rmsnorm_split): xs [M, ldx] 4-byte words in the split
 * layout (per row, each group of 8 inputs as 8 bf16 hi parts then 8 bf16 lo parts; ldx counted in inputs, a multiple
 * of 4). The product skips the split and is bitwise that of q35_gemm_q8 on the fp32 values hi + lo was made from.
 * Same reference lines as q35_gemm_q8.
 */
int q35_gemm_q8_split(const void* xs, int64_t ldx, const int8_t* W, int w_dtype, const float* w_scale, float* y,
                      int64_t ldy, int64_t M, int64_t N, int64_t K, int epilogue, const q35_push* pushes,
                      int64_t npush, int64_t T, float* cap, int64_t ld_cap, int64_t ld_cap_row,
                      q35_stream_t stream);

/*
 * q35_gemm_q8 on bf16 x (the attention output, read without a conversion to fp32): xb [M, ldx] bf16, 16-byte
 * aligned, ldx a multiple of 8. Runs on the register-staged kernel with only the hi products issued (the hi parts are
 * x, the lo parts zero): bitwise q35_gemm_q8 on the fp32 values of x where that also runs the register-staged kernel
 * (N < 2048 or K > 2048), equal to fp32 rounding elsewhere (the DMA kernel sums K in another grouping). Same
 * reference lines.
 */
int q35_gemm_q8_bf16(const void* xb, int64_t ldx, const int8_t* W, int w_dtype, const float* w_scale, float* y,
                     int64_t ldy, int64_t M, int64_t N, int64_t K, int epilogue, const q35_push* pushes,
                     int64_t npush, int64_t T, float* cap, int64_t ld_cap, int64_t ld_cap_row, q35_stream_t stream);

/*
 * a[m, n] = silu(gu[m, n]) * gu[m, I + n] with the pushes applied, gu: [M, 2 I] fp32 ([gate | up] per row),
 * a: [M, I] fp32; pushes, T and the capture (cap, ld_cap, ld_cap_row >= I) as for q35_gemv.
 */
int q35_swiglu_push(const float* gu, float* a, int64_t M, int64_t I, const q35_push* pushes, int64_t npush,
                    int64_t T, float* cap, int64_t ld_cap, int64_t ld_cap_row, q35_stream_t stream);

/*
 * Per-row argmax (greedy sampling): idx[r] = the lowest index of the largest value of x[r, 0:n] (the WGSL `argmax`,
 * engine/kernels.js:260-283; torch.argmax's rule), val[r] that value (val may be NULL). A row of -inf gives index 0.
 *   x: [rows, ldx] fp32 (rows need no alignment beyond 4 bytes). idx: [rows] int32.
 */
int q35_argmax_rows(const float* x, int64_t ldx, int64_t rows, int64_t n, int32_t* idx, float* val,
                    q35_stream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* Q35HIP_H */
