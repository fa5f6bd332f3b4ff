/*
 * qwen36_attn.h -- C ABI of libqwen36_attn.so, the MI355X (gfx950) attention
 * hot path of the Qwen3.6-35B-A3B engine.
 *
 * Conventions (as the reference's FMHA provider ABI,
 * benchmarks/shape-lab/native/src/qrt_ck_fmha_q8192_provider.cpp:134-325):
 *   - every entry point returns a hipError_t as int: 0 = success,
 *     1 (hipErrorInvalidValue) = rejected arguments, checked before any
 *     launch; nothing throws across the ABI;
 *   - the caller owns every device buffer (inputs, outputs, workspaces);
 *   - work is enqueued asynchronously on the caller's stream (a hipStream_t
 *     passed as void*; NULL = the default stream);
 *   - bf16 tensors are raw 16-bit storage; "stride" arguments are in
 *     elements; all layouts are row-major.
 * Geometry is fixed by the model: full attention Hq=16, Hkv=2, D=256
 * (query head h reads KV head h/8); Gated DeltaNet Hk=16, Hv=32, dk=dv=128,
 * conv kernel 4, conv_dim 8192.  Maximum sequence length 262144.
 */
#ifndef QWEN36_ATTN_H
#define QWEN36_ATTN_H

#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- FMHA prefill provider (drop-in) -------------------------------------
 * Replaces qrt_ck_fmha_{prepare,bf16_launch,bf16_launch_ex,release}
 * (qrt_ck_fmha_q8192_provider.cpp:240-325), bound by
 * NativeQ8192CkProvider::load/launch (native/src/native_full_prefill.hip.cpp
 * :140-266) and by Q8192CompoundProvider (q8192_compound_provider.py:120-202).
 * Q [q_tokens,16,256] bf16, K/V [kv_tokens,2,256] bf16, out fp32
 * [q_tokens,4096]; scale 1/16; top-left causal mask when
 * q_tokens == kv_tokens, bottom-right otherwise. */
/* prepare (0 < tokens <= 262144) allocates, once per device, the provider's
 * 132 MiB split-K scratch: launches with fewer than 16 query tiles of 256
 * rows split each tile's key range over several workgroups plus a combine
 * launch and use it (without it -- not prepared, or the allocation failed, in
 * which case prepare still returns 0 -- they run unsplit).  The first split
 * launch on a device claims the scratch for its stream: later launches on
 * that stream are ordered by it, launches on other streams run unsplit, so
 * launches on different streams never share it.  (Replaying a graph captured
 * on the owning stream concurrently with that stream's own launches is the
 * one way to race on it.)  The scratch is kept until the process ends
 * (graphs captured with a split launch hold its address), so release has
 * nothing to free; the provider's globals sit behind a mutex. */
int qrt_ck_fmha_prepare(unsigned tokens);
int qrt_ck_fmha_bf16_launch(const void* q, const void* k, const void* v,
                            float* out, unsigned tokens, void* stream);
int qrt_ck_fmha_bf16_launch_ex(const void* q, const void* k, const void* v,
                               float* out, unsigned query_tokens,
                               unsigned kv_tokens, void* stream);
int qrt_ck_fmha_release(void);
/* qwen36_fmha_prefill: the same attention with a caller-owned split-K
 * workspace (no counterpart in the reference's provider ABI), so short
 * prompts split on any stream: workspace of at least
 * qwen36_fmha_prefill_workspace_bytes(query_tokens, kv_tokens) bytes (0 =
 * this geometry runs unsplit and workspace may be NULL; also 0 for invalid
 * geometry, which the launch rejects).  Calls that overlap on one workspace
 * race. */
size_t qwen36_fmha_prefill_workspace_bytes(unsigned query_tokens, unsigned kv_tokens);
int qwen36_fmha_prefill(const void* q, const void* k, const void* v, float* out,
                        unsigned query_tokens, unsigned kv_tokens, void* workspace,
                        size_t workspace_bytes, void* stream);
/* qwen36_fmha_prefill_gated: the attention with the layer's sigmoid output
 * gate applied in the same launches (the FMHA epilogue, or the split-K
 * combine), writing bf16 rows instead of fp32 -- the reference runs the
 * FMHA provider (fp32 out) and then full_attention_gate_kernel's f32 form
 * (native_full_prefill.hip.cpp:140-266 then native_pointwise.hip.cpp:
 * 339-359); this is that pair fused, with the gate kernel's roundings
 * (attention -> bf16, sigmoid -> bf16, product -> bf16), so it equals
 * qwen36_fmha_prefill followed by qwen36_output_gate bit for bit (a NaN
 * gate gives a NaN in both).
 * q_gate: the fused q projection rows [query_tokens][q_gate_row_stride]
 * bf16 whose head h slice is [q (256) | gate (256)] at h*512 (stride >=
 * 8192, 8-byte aligned); out [query_tokens, 4096] bf16, 16-byte aligned.
 * Workspace as qwen36_fmha_prefill (same size function). */
int qwen36_fmha_prefill_gated(const void* q, const void* k, const void* v,
                              const void* q_gate, unsigned q_gate_row_stride, void* out,
                              unsigned query_tokens, unsigned kv_tokens, void* workspace,
                              size_t workspace_bytes, void* stream);
/* Legacy fixed-shape q8192 exports (qrt_ck_fmha_q8192_provider.cpp:214-300).
 * qrt_ck_fmha_q8192_f32_launch (:228-271): packed_qkv fp32 [8192, 9216] rows
 * of [q (4096) | 4096 more q_proj features, unused | k (512) | v (512)],
 * rounded to bf16 (nearest even) into provider staging -- 80 MiB per device,
 * allocated by q8192_prepare or the first f32 launch, freed by
 * q8192_release -- then the square causal attention into out fp32
 * [8192, 4096]. */
int qrt_ck_fmha_q8192_prepare(void);
int qrt_ck_fmha_q8192_f32_launch(const float* packed_qkv, float* out, void* stream);
int qrt_ck_fmha_q8192_bf16_launch(const void* q, const void* k, const void* v,
                                  float* out, void* stream);
int qrt_ck_fmha_q8192_release(void);

/* ---- GQA decode (split-K flash decode) -----------------------------------
 * Replaces launch_native_grouped_full_attention(layer, position, cache_end,
 * q, normalized_k, raw_v, state, stream)
 * (native/include/aima/native_full_attention.h:88-93,
 * native_full_attention.hip.cpp:681-765), whose invalid geometry throws
 * std::invalid_argument; here it returns 1.
 * q [16,256] bf16 (head-normed, roped); k_new/v_new [2,256] bf16 or both
 * NULL: when given they are written to cache row `position` first;
 * k_cache/v_cache [capacity,2,256] bf16; attention over rows [0,cache_end).
 * gate: NULL, or bf16 with gate[h*gate_head_stride + d] the gate of head h
 * (fused q-projection row: stride 512 from its gate half); then
 * out = bf16(bf16(attn) * bf16(sigmoid(gate))) as native_pointwise.hip.cpp
 * :207-222.  out [4096] bf16.  workspace (split partials) of at least
 * qwen36_decode_gqa_workspace_bytes(cache_end, split_tokens) bytes; calls
 * that overlap on one workspace race.
 * split_tokens 0 = automatic, else a multiple of 128 with at most 256 splits. */
size_t qwen36_decode_gqa_workspace_bytes(unsigned cache_end,
                                         unsigned split_tokens);
int qwen36_decode_gqa(const void* q, const void* k_new, const void* v_new,
                      void* k_cache, void* v_cache, unsigned position,
                      unsigned cache_end, unsigned capacity, const void* gate,
                      unsigned gate_head_stride, void* out, void* workspace,
                      size_t workspace_bytes, unsigned split_tokens,
                      void* stream);

/* qwen36_decode_gqa_noalloc: qwen36_decode_gqa without a workspace argument.
 * No counterpart in the reference: for callers that cannot allocate (code
 * under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc).  The split partials go to a library-owned device buffer of
 * 4,227,072 bytes (the workspace of 256 splits, the most any call uses),
 * one per GPU, held until the process ends; the call allocates nothing.
 * Arguments and results are those of qwen36_decode_gqa; a split count whose
 * workspace would exceed the buffer returns 1.  Every call on one GPU shares
 * that GPU's buffer: calls that overlap on one GPU (different streams, or
 * concurrently replayed graphs) race. */
int qwen36_decode_gqa_noalloc(const void* q, const void* k_new, const void* v_new,
                              void* k_cache, void* v_cache, unsigned position,
                              unsigned cache_end, unsigned capacity,
                              const void* gate, unsigned gate_head_stride,
                              void* out, unsigned split_tokens, void* stream);

/* qwen36_decode_step: the whole one-token decode of a gated full-attention
 * layer between its projections and o_proj, in one split launch plus the
 * combine: head RMSNorm (w + 1) and partial RoPE of the 16 query heads and of
 * the new key, the K (normalised) / V (raw) cache-row write at `position`,
 * split-K attention over rows [0, cache_end) and the sigmoid output gate.
 * Replaces the reference decode's norm/rope/KV-write launch plus its
 * attention core (four_layer_mini_engine.py:933
 * triton_full_attention_norm_rope_kv_write_kernel and :6614-6650;
 * native_full_attention.hip.cpp:58-69, :681-765).
 * q_gate: the q-projection row [16 x (256 query | 256 gate)] bf16; k_raw,
 * v_raw: [2 x 256] bf16 before the head norm; q/k_norm_weight [256] bf16;
 * caches [capacity, 2, 256] bf16; out [4096] bf16; workspace as for
 * qwen36_decode_gqa (same size function).  Rounding is identical to
 * qwen36_head_norm_rope followed by qwen36_decode_gqa. */
int qwen36_decode_step(const void* q_gate, const void* k_raw, const void* v_raw,
                       const void* q_norm_weight, const void* k_norm_weight,
                       void* k_cache, void* v_cache, unsigned position,
                       unsigned cache_end, unsigned capacity, void* out,
                       void* workspace, size_t workspace_bytes,
                       unsigned split_tokens, void* stream);

/* ---- full-attention pointwise ----------------------------------------------
 * qwen36_rotary_table: replaces prefill_rotary_table_kernel /
 *   decode_rotary_kernel (native_pointwise.hip.cpp:224-238,
 *   native_decode_runner.hip.cpp:52-59): cos/sin fp32 [tokens,32].
 * qwen36_head_norm_rope: replaces full_attention_head_norm_rope_prefill_kernel
 *   (native_pointwise.hip.cpp:242-337) + the KV write
 *   (four_layer_mini_engine.py:5980-5986): q_gate [T, >=8192 stride] fused
 *   [Q|Gate] rows, k/v [T, >=512 stride]; writes q_out [T,16,256] and cache
 *   rows [position_start, position_start+T) of k_cache/v_cache.
 * qwen36_output_gate: replaces full_attention_gate_kernel /
 *   full_attention_gate_f32_prefill_kernel (native_pointwise.hip.cpp:207-222,
 *   339-359): out[T,4096] = attn * sigmoid(gate), attn bf16 or fp32. */
int qwen36_rotary_table(float* cos_out, float* sin_out, unsigned tokens,
                        unsigned position_start, void* stream);
int qwen36_head_norm_rope(const void* q_gate, unsigned q_row_stride,
                          const void* k_raw, unsigned k_row_stride,
                          const void* v_raw, unsigned v_row_stride,
                          const void* q_weight, const void* k_weight,
                          unsigned tokens, unsigned position_start,
                          void* q_out, void* k_cache, void* v_cache,
                          void* stream);
int qwen36_output_gate(const void* attn, int attn_is_f32, const void* q_gate,
                       unsigned q_row_stride, void* out, unsigned tokens,
                       void* stream);

/* ---- Gated DeltaNet --------------------------------------------------------
 * qwen36_gdn_conv1d: replaces linear_causal_conv (four_layer_mini_engine.py
 *   :5293-5403) / the AOT _causal_conv1d_fwd_kernel: x [T, >=8192 stride],
 *   weight [8192,4], state_in/state_out [8192,3] bf16 (may alias),
 *   out [T,8192] = SiLU(conv).
 * qwen36_gdn_gating: the beta/g half of _fused_post_conv_kernel
 *   (four_layer_mini_engine.py:6507-6511): a, b [T, >=32 stride] bf16,
 *   A_log, dt_bias [32] fp32 -> g, beta [T,32] fp32.  flags 0: beta =
 *   sigmoid(b) rounded to bf16, as the torch layer evaluates it on the bf16
 *   projection output; QWEN36_GDN_BETA_FP32 (1): unrounded fp32 sigmoid, as
 *   vLLM's fused gating.  Other flag bits are rejected.
 * qwen36_gdn_recurrent: replaces torch_recurrent_gated_delta_rule
 *   (:5242-5276) / fused_sigmoid_gating_delta_rule_update's delta rule
 *   (native_linear_layer.hip.cpp:84-95).  q,k [T, qk_heads(16|32), 128]
 *   bf16 raw (l2-normalised in-kernel) with token stride qk_token_stride,
 *   v [T,32,128] with token stride v_token_stride, g/beta [T,32] fp32,
 *   state [32,128(k),128(v)] fp32 (state_out may alias state_in),
 *   out [T,32,128] bf16.  v_token_stride % 4 == 0; v and out 8-byte and
 *   the states 16-byte aligned.
 * qwen36_gdn_chunk_prefill: replaces torch_chunk_gated_delta_rule
 *   (:5167-5240, chunk 64) / the FLA chunk pipeline launched by
 *   native_linear_prefill.hip.cpp:474-836.  Same tensors as the recurrent
 *   step; state_in may be NULL (zeros).  Workspace of at least
 *   qwen36_gdn_chunk_prefill_workspace_bytes(tokens) bytes.  q, k and v
 *   16-byte aligned (their rows are read as 16-byte vectors).
 * qwen36_gdn_chunk_prefill_ex: the same with flags, for vLLM's
 *   chunk_gated_delta_rule(q, k, v, g, beta, initial_state,
 *   output_final_state, use_qk_l2norm_in_kernel) as the reference calls it
 *   (four_layer_mini_engine.py:6474-6483, state handoff :5482-5502):
 *   QWEN36_GDN_QK_NORMALIZED = use_qk_l2norm_in_kernel=False (q and k arrive
 *   l2-normalised and are used as given); QWEN36_GDN_STATE_VK = state_in and
 *   state_out in vLLM's [32, 128 (v), 128 (k)] orientation.  Flags 0 is
 *   qwen36_gdn_chunk_prefill.  Unknown flag bits are rejected.
 * qwen36_gdn_gated_norm: replaces linear_gated_norm_fused_kernel
 *   (native_pointwise.hip.cpp:376-430; :6531-6541): core [T,32,128],
 *   z [T, >=4096 stride], weight [128] bf16 -> out [T,4096]. */
int qwen36_gdn_conv1d(const void* x, unsigned x_row_stride, const void* weight,
                      const void* state_in, void* state_out, void* out,
                      unsigned tokens, void* stream);
#define QWEN36_GDN_BETA_FP32 1u
int qwen36_gdn_gating(const void* a, const void* b, unsigned ab_row_stride,
                      const void* a_log, const void* dt_bias, void* g,
                      void* beta, unsigned tokens, unsigned flags, void* stream);
int qwen36_gdn_recurrent(const void* q, const void* k, const void* v,
                         unsigned qk_heads, unsigned qk_token_stride,
                         unsigned v_token_stride, const void* g,
                         const void* beta, const void* state_in,
                         void* state_out, void* out, unsigned tokens,
                         void* stream);
size_t qwen36_gdn_chunk_prefill_workspace_bytes(unsigned tokens);
int qwen36_gdn_chunk_prefill(const void* q, const void* k, const void* v,
                             unsigned qk_heads, unsigned qk_token_stride,
                             unsigned v_token_stride, const void* g,
                             const void* beta, const void* state_in,
                             void* state_out, void* out, unsigned tokens,
                             void* workspace, size_t workspace_bytes,
                             void* stream);
#define QWEN36_GDN_QK_NORMALIZED 1u
#define QWEN36_GDN_STATE_VK 2u
int qwen36_gdn_chunk_prefill_ex(const void* q, const void* k, const void* v,
                                unsigned qk_heads, unsigned qk_token_stride,
                                unsigned v_token_stride, const void* g,
                                const void* beta, const void* state_in,
                                void* state_out, void* out, unsigned tokens,
                                unsigned flags, void* workspace,
                                size_t workspace_bytes, void* stream);
int qwen36_gdn_gated_norm(const void* core, const void* z,
                          unsigned z_row_stride, const void* weight, void* out,
                          unsigned tokens, void* stream);

/* qwen36_gdn_fused_gating_update: the decode update in vLLM's orientation
 *   with the gating fused -- replaces fused_sigmoid_gating_delta_rule_update
 *   as the reference's decode calls it (four_layer_mini_engine.py:6429-6440;
 *   native launch native_linear_layer.hip.cpp:84-95).  Per token: g =
 *   -exp(A_log) softplus(a + dt_bias) (linear above 20), beta = sigmoid(b)
 *   in fp32, q/k l2-normalised when flags bit 0 (use_qk_l2norm_in_kernel) is
 *   set, q *= scale (> 0), H <- H e^g, v' = (v - H k) beta, H <- H + v' k^T,
 *   o = H q.  A_log, dt_bias [32] fp32; a, b [T, >=32 stride] bf16; q, k
 *   [T, qk_heads (16|32), 128] bf16 (token stride a multiple of 8, 16-byte
 *   aligned); v [T, 32, 128] bf16 with token stride v_token_stride;
 *   state_in -> state_out [32, 128 (v), 128 (k)] fp32, 16-byte aligned (may
 *   alias); out [T, 32, 128] bf16. */
int qwen36_gdn_fused_gating_update(const void* a_log, const void* a, const void* b,
                                   unsigned ab_row_stride, const void* dt_bias,
                                   const void* q, const void* k, unsigned qk_heads,
                                   unsigned qk_token_stride, const void* v,
                                   unsigned v_token_stride, const void* state_in,
                                   void* state_out, void* out, unsigned tokens,
                                   float scale, unsigned flags, void* stream);
/* qwen36_gdn_fused_gating_update_varlen: the same update over N sequences,
 *   for vLLM's batched calls -- fused_sigmoid_gating_delta_rule_update with
 *   cu_seqlens / ssm_state_indices, and the packed decode
 *   fused_recurrent_gated_delta_rule_packed_decode
 *   (four_layer_mini_engine.py:6396-6417).  Sequence n covers tokens
 *   [cu_seqlens[n], cu_seqlens[n+1]) (int32 [N+1]; NULL: token n alone, then
 *   N == tokens) and carries state slot state_indices[n] (int32 [N]; NULL:
 *   slot n) of the pools state_in -> state_out [n_slots, 32, 128 (v), 128 (k)]
 *   fp32 (may alias).  A slot outside [0, n_slots), or an empty sequence, is
 *   padding: skipped, its outputs and state slot untouched.  1 <= N <= 65535;
 *   other arguments as qwen36_gdn_fused_gating_update. */
int qwen36_gdn_fused_gating_update_varlen(const void* a_log, const void* a, const void* b,
                                          unsigned ab_row_stride, const void* dt_bias,
                                          const void* q, const void* k, unsigned qk_heads,
                                          unsigned qk_token_stride, const void* v,
                                          unsigned v_token_stride, const void* state_in,
                                          void* state_out, void* out, unsigned tokens,
                                          const void* cu_seqlens, const void* state_indices,
                                          unsigned n_seqs, unsigned n_slots, float scale,
                                          unsigned flags, void* stream);

/* qwen36_gdn_decode_step: one launch for everything between the GDN input
 *   projections and out_proj -- conv1d + SiLU, gating, l2norm, the recurrent
 *   delta rule and the gated RMSNorm -- for `tokens` consecutive tokens.
 *   Replaces the reference decode's launch sequence for the linear layer
 *   (native_linear_layer.hip.cpp:84-157: fused input-projection/conv,
 *   fused_sigmoid_gating_delta_rule_update, gated norm; torch form
 *   four_layer_mini_engine.py:6378-6544 with mode == "decode").
 *   mixed_qkv [T, >=8192 stride] bf16 (before the conv), conv_weight
 *   [8192,4], conv_state_in -> conv_state_out [8192,3] bf16 (must not
 *   overlap: double-buffer them), a, b [T, >=32 stride] bf16, A_log, dt_bias
 *   [32] fp32, z [T, >=4096 stride] bf16, norm_weight [128] bf16,
 *   state_in -> state_out [32,128,128] fp32 (may alias), out [T,4096] bf16.
 *   Same error convention as the other entry points. */
int qwen36_gdn_decode_step(const void* mixed_qkv, unsigned x_row_stride,
                           const void* conv_weight, const void* conv_state_in,
                           void* conv_state_out, const void* a, const void* b,
                           unsigned ab_row_stride, const void* a_log,
                           const void* dt_bias, const void* z,
                           unsigned z_row_stride, const void* norm_weight,
                           const void* state_in, void* state_out, void* out,
                           unsigned tokens, void* stream);

/* ---- prefill projections ---------------------------------------------------
 * qwen36_prefill_gemm_bf16: y[m, n] = x[m, k] W[n, k]^T for a prompt of m
 * tokens, bf16 in and out with fp32 accumulation (one rounding); replaces
 * the reference's prefill projection GEMMs (hipBLASLt plans,
 * native_full_prefill.hip.cpp:552-560, native_prefill_gemm_plans.hip.cpp;
 * torch form `inp @ W.t()` in four_layer_mini_engine.py:6566-6573, :6386-6395,
 * :6653, :6544).  x row-major with row stride ldx (>= k, a multiple of 8), W
 * row-major [n, k] (out x in features), y row-major with row stride ldy
 * (>= n); x and W 16-byte aligned; k a multiple of 64 (<= 16384), n <= 65536,
 * m <= 262144. */
int qwen36_prefill_gemm_bf16(const void* x, unsigned ldx, const void* w, void* y,
                             unsigned ldy, unsigned m, unsigned n, unsigned k,
                             void* stream);

/* qwen36_prefill_gemm_workspace_bytes / qwen36_prefill_gemm_bf16_ws: the
 * same product with a caller workspace, which lets a short prompt with a long
 * k (e.g. the k = 4096 output projections at m = 1024, where whole-k tiles
 * fill half the GPU) split k into slices: each slice's fp32 partial products
 * go to the workspace and a second launch sums them in slice order and rounds
 * once, so the result is deterministic; it can differ from
 * qwen36_prefill_gemm_bf16's by the fp32 summation order (well inside one
 * bf16 rounding).  workspace_bytes returns 0 when the shape runs unsplit (ws
 * may then be NULL) and for a shape the launch rejects (m, n or k out of the
 * ranges above); otherwise ws is 16-byte aligned and holds at least that
 * many bytes, else the call returns the invalid-argument code.  Same
 * reference call sites as qwen36_prefill_gemm_bf16. */
size_t qwen36_prefill_gemm_workspace_bytes(unsigned m, unsigned n, unsigned k);
/* qwen36_prefill_gemm_bf16_lt: the same product (y = x W^T, bf16, fp32
 * accumulation, one rounding) run as a hipBLASLt GEMM -- the library the
 * reference's native prefill plans these projections with
 * (native_full_prefill.hip.cpp:552-560) -- for the shapes where its kernel
 * is faster than the MFMA kernel above.  Same arguments and limits as
 * qwen36_prefill_gemm_bf16_ws, except that the workspace (caller-owned,
 * qwen36_prefill_gemm_lt_workspace_bytes() bytes suffice for every shape)
 * is what hipBLASLt's algorithm needs.  The first call of a shape on a device
 * creates the library handle and queries the algorithm (host work only;
 * make it outside graph capture).  Returns hipErrorNotSupported when
 * hipBLASLt has no algorithm for the shape. */
size_t qwen36_prefill_gemm_lt_workspace_bytes(void);
int qwen36_prefill_gemm_bf16_lt(const void* x, unsigned ldx, const void* w, void* y,
                                unsigned ldy, unsigned m, unsigned n, unsigned k, void* ws,
                                size_t ws_bytes, void* stream);
int qwen36_prefill_gemm_bf16_ws(const void* x, unsigned ldx, const void* w, void* y,
                                unsigned ldy, unsigned m, unsigned n, unsigned k,
                                void* ws, size_t ws_bytes, void* stream);

/* ---- decode projections ----------------------------------------------------
 * qwen36_gemv_bf16: y[N] = W[N,K] x[K] for one token, bf16 in and out with
 * fp32 accumulation; replaces the decode projection GEMVs
 * (native_full_layer.hip.cpp:154-174 fused q/k/v and o_proj,
 * native_linear_layer.hip.cpp:151-157 in/out projections; torch form
 * `inp @ W.t()` in four_layer_mini_engine.py:6566-6573, :6386-6395).
 * W row-major [N, K] (out x in features), K = 2048 or 4096, W and x 16-byte
 * aligned. */
int qwen36_gemv_bf16(const void* w, unsigned n_rows, unsigned k, const void* x, void* y,
                     void* stream);

/* ---- MoE block (one decode token) --------------------------------------------
 * qwen36_moe_decode: the layer's step after attention for one token --
 * residual add, post-attention RMSNorm (w + 1), router top-8 with softmax
 * routing weights, the 8 routed experts (gate/up, SiLU, down) and the
 * sigmoid-gated shared expert, summed into the residual -- with the bf16
 * roundings of four_layer_mini_engine.py:8479-8650 (router :7775-7789,
 * experts :7791-7803, shared :8240-8300); replaces the decode's router top-k
 * kernels and native MoE consumer.  inp, attn_out, post_norm_w [2048] bf16;
 * w_in [E+1+1024, 2048] = rows [router | shared_gate | shared gate_proj |
 * shared up_proj]; expert_gate_up [E, 1024, 2048] (gate rows then up rows);
 * expert_down [E, 2048, 512]; shared_down [2048, 512]; out [2048] bf16;
 * 8 <= E <= 256, E % 4 == 0; all pointers 16-byte aligned; workspace of
 * qwen36_moe_decode_workspace_bytes() bytes (holds the selected expert ids
 * as int32 at byte offset 8192, their routing weights as fp32 at 8224 and
 * the router logits as bf16 at 17472). */
size_t qwen36_moe_decode_workspace_bytes(void);
int qwen36_moe_decode(const void* inp, const void* attn_out, const void* post_norm_w,
                      const void* w_in, const void* expert_gate_up, const void* expert_down,
                      const void* shared_down, unsigned n_experts, void* out, void* workspace,
                      size_t workspace_bytes, void* stream);

/* ---- MoE block (prefill, T tokens) ------------------------------------------
 * qwen36_moe_prefill: the same block for T = `tokens` rows (inp, attn_out,
 * out [T, 2048] bf16), weights as for qwen36_moe_decode; replaces the
 * reference's native MoE prefill (native_moe_prefill.hip.cpp: router GEMM and
 * router_topk8_softmax_256_kernel :234-323, moe_align_block32_256_kernel
 * :325-382, the two AOT fused_moe expert GEMMs with
 * expert_silu_multiply_kernel :384-402, the shared-expert GEMMs and kernels
 * :210-232, moe_sum8_kernel :404-430, the residual add) with the eager
 * arithmetic of four_layer_mini_engine.py:8479-8650.  1 <= T <= 262144;
 * workspace of qwen36_moe_prefill_workspace_bytes(T, E) bytes (0 = invalid
 * arguments), which starts with the expert ids (int32 [T, 8]) at offset 0,
 * the routing weights (fp32 [T, 8]) and the router logits (bf16 [T, ld],
 * ld = (E + 8) & ~7, column E = the shared gate), each region 256-byte
 * aligned. */
size_t qwen36_moe_prefill_workspace_bytes(unsigned tokens, unsigned n_experts);
int qwen36_moe_prefill(const void* inp, const void* attn_out, const void* post_norm_w,
                       const void* w_in, const void* expert_gate_up, const void* expert_down,
                       const void* shared_down, unsigned n_experts, unsigned tokens, void* out,
                       void* workspace, size_t workspace_bytes, void* stream);

/* ---- exact-prefix cache ----------------------------------------------------
 * Replaces NativeExactPrefixCache and the resident engine's entry pool
 * (native_resident_engine.hip.cpp:121-296, :553-560, :706-719, :826-836,
 * :1197-1214).  A pool owns `entries` snapshots (0 = the reference's rule:
 * 4 up to 32K tokens of capacity, 2 up to 128K, else 1).  Registered slices
 * are live device buffers: per-token (bytes_per_token > 0, capacity ==
 * max_tokens * bytes_per_token; a layer's K or V cache) or fixed (a GDN
 * layer's conv / recurrent state).  Capture and restore are one batched copy
 * launch each on the caller's stream; lookup is host-side (longest matching
 * token prefix); capture fills the first empty entry, else the least
 * recently used.  Pointers and sizes are 16-byte multiples.  create returns
 * NULL on bad arguments; the others return 0 or a hipError_t value. */
void* qwen36_prefix_cache_create(unsigned max_tokens, unsigned long long terminal_bytes,
                                 unsigned entries);
unsigned qwen36_prefix_cache_entries(void* pool);
int qwen36_prefix_cache_add_slice(void* pool, void* live, unsigned long long capacity_bytes,
                                  unsigned long long bytes_per_token);
int qwen36_prefix_cache_finalize(void* pool, unsigned long long* bytes_out);
int qwen36_prefix_cache_lookup(void* pool, const unsigned* tokens, unsigned n,
                               unsigned* matched, unsigned* index);
int qwen36_prefix_cache_restore(void* pool, unsigned index, void* stream,
                                unsigned long long* bytes_out);
int qwen36_prefix_cache_capture(void* pool, const unsigned* tokens, unsigned n,
                                const void* terminal, void* stream, unsigned* index_out,
                                unsigned long long* bytes_out);
int qwen36_prefix_cache_copy_terminal(void* pool, unsigned index, void* dst, void* stream);
int qwen36_prefix_cache_destroy(void* pool);

#ifdef __cplusplus
}
#endif

#endif /* QWEN36_ATTN_H */
