/*
 * rusty_hip.h — C ABI of librusty_hip.so, the MI355X (gfx950) backend for
 * RustyLLM's decode step.
 *
 * Every rusty_hip_* export below "Reference seam" mirrors one rusty_metal_*
 * declaration of the reference's src/metal.rs FFI block (lines cited), with
 * the same parameter order, types (usize -> uintptr_t) and return convention:
 * 1 = the full output was written, 0 = not handled (not initialised, null
 * pointer, zero or unsupported dimension, buffer too small, device error) and
 * the caller runs its CPU kernel instead (src/metal.rs:716-720).
 *
 * Weights passed by host pointer are uploaded once and cached by (pointer,
 * length) for the life of the process, as the Metal shim does
 * (src/metal_backend.m:788-842); row starts are padded to 16 bytes in the
 * device copy, block bytes are unchanged.  Calls are synchronous.  The per-op
 * exports share staging buffers and must be serialised by the caller, like
 * the reference's (src/runtime.rs:3167-3170); the library also holds an
 * internal mutex.
 *
 * Numerics follow the reference's x86 path: Q4_K, Q6_K and Q8_0 (K % 256 ==
 * 0) multiply against the Q8_K-quantized activation (src/simd.rs:944-959);
 * Q8_0 with other K and MXFP4 use f32 activations.
 */
#ifndef RUSTY_HIP_H
#define RUSTY_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ===== Reference seam (src/metal.rs:123-340) ============================== */

/* rusty_metal_available, src/metal.rs:127.  Initialises the device context. */
int rusty_hip_available(void);

/* rusty_metal_q4k_matvec / q6k_matvec, src/metal.rs:129-145. */
int rusty_hip_q4k_matvec(const uint8_t *weights, uintptr_t weights_len, const float *x, uintptr_t rows,
                         uintptr_t cols, float *out);
int rusty_hip_q6k_matvec(const uint8_t *weights, uintptr_t weights_len, const float *x, uintptr_t rows,
                         uintptr_t cols, float *out);

/* rusty_metal_q6k_matvec2 / 3, src/metal.rs:147-176. */
int rusty_hip_q6k_matvec2(const uint8_t *weights_a, uintptr_t weights_a_len, uintptr_t rows_a,
                          const uint8_t *weights_b, uintptr_t weights_b_len, uintptr_t rows_b, const float *x,
                          uintptr_t cols, float *out_a, float *out_b);
int rusty_hip_q6k_matvec3(const uint8_t *weights_a, uintptr_t weights_a_len, uintptr_t rows_a,
                          const uint8_t *weights_b, uintptr_t weights_b_len, uintptr_t rows_b,
                          const uint8_t *weights_c, uintptr_t weights_c_len, uintptr_t rows_c, const float *x,
                          uintptr_t cols, float *out_a, float *out_b, float *out_c);

/* rusty_metal_q4k_matvec2 / 3, src/metal.rs:177-206. */
int rusty_hip_q4k_matvec2(const uint8_t *weights_a, uintptr_t weights_a_len, uintptr_t rows_a,
                          const uint8_t *weights_b, uintptr_t weights_b_len, uintptr_t rows_b, const float *x,
                          uintptr_t cols, float *out_a, float *out_b);
int rusty_hip_q4k_matvec3(const uint8_t *weights_a, uintptr_t weights_a_len, uintptr_t rows_a,
                          const uint8_t *weights_b, uintptr_t weights_b_len, uintptr_t rows_b,
                          const uint8_t *weights_c, uintptr_t weights_c_len, uintptr_t rows_c, const float *x,
                          uintptr_t cols, float *out_a, float *out_b, float *out_c);

/* rusty_metal_q4k_q4k_q6k_matvec3, src/metal.rs:207-222. */
int rusty_hip_q4k_q4k_q6k_matvec3(const uint8_t *weights_a, uintptr_t weights_a_len, uintptr_t rows_a,
                                  const uint8_t *weights_b, uintptr_t weights_b_len, uintptr_t rows_b,
                                  const uint8_t *weights_c, uintptr_t weights_c_len, uintptr_t rows_c,
                                  const float *x, uintptr_t cols, float *out_a, float *out_b, float *out_c);

/* rusty_metal_q4k_q4k_q6k_ffn, src/metal.rs:224-237: out = down * (silu(gate*x) (.) up*x). */
int rusty_hip_q4k_q4k_q6k_ffn(const uint8_t *gate_weights, uintptr_t gate_weights_len, const uint8_t *up_weights,
                              uintptr_t up_weights_len, const uint8_t *down_weights, uintptr_t down_weights_len,
                              const float *x, uintptr_t input_cols, uintptr_t hidden_rows, uintptr_t down_rows,
                              uintptr_t down_cols, float *out);

/* rusty_metal_mistral_post_attention_ffn, src/metal.rs:239-257:
 * x += wo*attn_out; x += down * (silu(gate*n) (.) up*n), n = rmsnorm(x)*ffn_norm. */
int rusty_hip_mistral_post_attention_ffn(const uint8_t *wo_weights, uintptr_t wo_weights_len,
                                         const uint8_t *gate_weights, uintptr_t gate_weights_len,
                                         const uint8_t *up_weights, uintptr_t up_weights_len,
                                         const uint8_t *down_weights, uintptr_t down_weights_len, float *x,
                                         uintptr_t dim, const float *attn_out, uintptr_t attn_cols,
                                         const float *ffn_norm, float rms_eps, uintptr_t hidden_rows,
                                         uintptr_t down_rows, uintptr_t down_cols);

/* rusty_metal_q8_0_matvec, src/metal.rs:268-275 (int8 Q8_K path when cols % 256
 * == 0, f32 activations otherwise, as src/simd.rs dot_row). */
int rusty_hip_q8_0_matvec(const uint8_t *weights, uintptr_t weights_len, const float *x, uintptr_t rows,
                          uintptr_t cols, float *out);

/* rusty_metal_attention, src/metal.rs:277-299.  *_len are byte lengths;
 * keys/values are the whole layer cache (slot_count * stride floats). */
int rusty_hip_attention(const float *query, uintptr_t query_len, const float *keys, uintptr_t keys_len,
                        const float *values, uintptr_t values_len, const float *sinks, uintptr_t sinks_len,
                        float *out, uintptr_t out_len, uintptr_t heads, uintptr_t kv_mul, uintptr_t head_dim,
                        uintptr_t value_dim, uintptr_t key_stride, uintptr_t value_stride, uintptr_t slot_count,
                        uintptr_t start_t, uintptr_t end_t, float scale, int use_sink);

/* ResidentLayerDesc, src/metal.rs:347-360 (#[repr(C)]).  Weight order: wq,
 * wk, wv, wo, gate(w1), up(w3), down(w2).  w_dt: 0 = Q4_K, 1 = Q6_K as in the
 * reference; this library also accepts 2 = Q8_0, 3 = MXFP4, or the GGML type
 * id itself (8, 12, 14, 39). */
typedef struct {
    const uint8_t *w[7];
    uintptr_t w_len[7];
    uint32_t w_rows[7];
    uint32_t w_dt[7];
    const float *attn_norm;
    const float *ffn_norm;
    const float *bq;
    uint32_t bq_len;
    const float *bk;
    uint32_t bk_len;
    const float *bv;
    uint32_t bv_len;
} RustyResidentLayerDesc;

/* rusty_metal_resident_configure / set_layer / set_output / decode,
 * src/metal.rs:302-338.  The KV cache lives in HBM. */
int rusty_hip_resident_configure(uint32_t n_layers, uint32_t dim, uint32_t n_heads, uint32_t n_kv_heads,
                                 uint32_t head_dim, uint32_t value_dim, uint32_t hidden_dim, uint32_t vocab,
                                 uint32_t storage_len, float eps, uint32_t neox);
int rusty_hip_resident_set_layer(uint32_t l, const RustyResidentLayerDesc *desc);
int rusty_hip_resident_set_output(const float *output_norm, const uint8_t *output_w, uintptr_t output_w_len,
                                  uint32_t output_rows, uint32_t output_dt, const float *inv_freq,
                                  uint32_t inv_freq_len);
int rusty_hip_resident_decode(const float *x_embed, uint32_t pos, uint32_t start_t, int want_logits,
                              float *logits_out);

/* ===== Exports without a Metal counterpart ================================ */

/* MXFP4 has no Metal hook (src/simd.rs:4020-4024); these serve
 * matvec_mxfp4_into (src/simd.rs:4020) and the expert pair of
 * ExpertWeight::try_matvec_expert_pair_into (src/model.rs:962-1017). */
int rusty_hip_mxfp4_matvec(const uint8_t *weights, uintptr_t weights_len, const float *x, uintptr_t rows,
                           uintptr_t cols, float *out);
int rusty_hip_mxfp4_matvec2(const uint8_t *weights_a, uintptr_t weights_a_len, uintptr_t rows_a,
                            const uint8_t *weights_b, uintptr_t weights_b_len, uintptr_t rows_b, const float *x,
                            uintptr_t cols, float *out_a, float *out_b);

/* Routed MoE feed-forward block of gpt-oss decode (forward_gpt_oss_into,
 * src/model.rs:6846-6898; the reference has no GPU hook for it): router
 * logits = router_w x (+ router_bias), the top_k experts in f32 total order
 * (ties: lower index, select_top_logits_into :6659-6716), softmax over them
 * (softmax_selected_into :6639-6656), per expert h = swiglu_gpt_oss(gate x +
 * gate_bias, up x + up_bias), y = down h + down_bias, out = sum over the
 * selected experts in order of y * p.  x is the normalized input (xn2);
 * out (dim floats) receives the block's output before the residual add.
 * Expert tensors are expert-major [n_experts][rows] of GGML blocks
 * (ExpertWeight, src/model.rs:922-955) with f32 activations (MXFP4 = 39, or
 * Q8_0 = 8 when dim / hidden % 256 != 0); biases [n_experts][rows] f32, may be
 * null.  router_dt / expert_dt are GGML type ids.  selected / probs (top_k
 * entries each, may be null) receive the chosen experts and their weights.
 * n_experts <= 64, top_k <= 8.  Bit-identical to the reference. */
int rusty_hip_moe_ffn(const float *x, uintptr_t dim, const uint8_t *router_w, uintptr_t router_w_len,
                      uint32_t router_dt, const float *router_bias, uint32_t n_experts, uint32_t top_k,
                      const uint8_t *gate_w, uintptr_t gate_w_len, const uint8_t *up_w, uintptr_t up_w_len,
                      const uint8_t *down_w, uintptr_t down_w_len, uint32_t expert_dt, uintptr_t hidden,
                      const float *gate_bias, const float *up_bias, const float *down_bias, float *out,
                      int32_t *selected, float *probs);

/* Generic single matvec for any supported GGML type (8, 12, 14, 39): the
 * Weight::matvec_into dispatch of src/model.rs:218-257. */
int rusty_hip_matvec(uint32_t ggml_type, const uint8_t *weights, uintptr_t weights_len, const float *x,
                     uintptr_t rows, uintptr_t cols, float *out);

/* matvec_kquant_batch_into (src/simd.rs:3417-3435; the reference keeps the
 * batch on the CPU): one Q4_K / Q6_K matrix (kind 0/1 or GGML 12/14) against
 * a row-major batch of T = inputs_len / (4 cols) activation rows; out is
 * row-major [T][rows] (out_len >= 4 T rows bytes).  cols % 256 == 0, as the
 * reference gates.  Runs on the matrix cores; every out[t][r] is
 * bit-identical to the single-token matvec of row r with input row t. */
int rusty_hip_kquant_matvec_batch(uint32_t kind, const uint8_t *weights, uintptr_t weights_len, uintptr_t rows,
                                  uintptr_t cols, const float *inputs, uintptr_t inputs_len, float *out,
                                  uintptr_t out_len);

/* Resident decoder, device-token mode (no reference counterpart; the
 * Metal decoder takes the embedding from the host).  The embedding table is
 * held in HBM and the greedy pick (repeat penalty + first finite maximum,
 * src/sampling.rs:78-83, 321-356) runs on the device, so a whole token is one
 * graph replay with no host round trip. */
int rusty_hip_resident_set_embedding(const uint8_t *embd, uintptr_t embd_len, uint32_t ggml_type);
/* Prefills `prompt` at positions start_pos.., then greedily generates n_gen
 * tokens into out_tokens (recent-token window of 64, src/runtime.rs:493-521).
 * logits_out (vocab floats, may be null) receives the logits of the last
 * forward.  As prefill_prompt_tokens (src/runtime.rs:3368-3420), a prompt of
 * more than two tokens on a batchable model has all but its last token
 * prefilled in batched chunks (rusty_hip_resident_prefill); environment
 * RUSTY_HIP_PREFILL=0 runs them one decode step at a time instead.  Both give
 * the same bits. */
int rusty_hip_resident_generate(const int32_t *prompt, uint32_t n_prompt, uint32_t start_pos, uint32_t n_gen,
                                float repeat_penalty, int32_t *out_tokens, float *logits_out);
/* forward_prefill_batch (src/model.rs:9917-10090): advances the KV cache over
 * tokens[0..n_tokens) at positions start_pos.. without computing logits, in
 * chunks (512 tokens; RUSTY_HIP_PREFILL_CHUNK, 64..2048) that run each weight matrix once per chunk on
 * the matrix cores.  Needs the device embedding (set_embedding) and a model
 * that standard_prefill_batchable (:9869-9887) accepts: every projection
 * Q4_K or Q6_K, widths multiples of 256; start_pos + n_tokens <= storage_len.
 * A gpt-oss decoder (resident_configure_moe) with Q8_0 attention and router,
 * MXFP4 experts and f32 KV is batched too (the reference prefills gpt-oss one
 * forward_prefill_gpt_oss step per token, src/model.rs:10286): each token's
 * arithmetic is its decode step's, every ring layer's token reads the ring as
 * it stood at its own step, and start_pos + n_tokens <= max_len.  Returns 0
 * for other models (the caller then decodes token by token).  Every cached
 * K/V value is bit-identical to decoding the tokens in turn with the
 * reference-order attention. */
int rusty_hip_resident_prefill(const int32_t *tokens, uint32_t n_tokens, uint32_t start_pos);
/* Chooses the expert product of the batched gpt-oss prefill (no counterpart
 * in the reference, which prefills gpt-oss token by token): 0 (the default,
 * or environment RUSTY_HIP_EXPERT_MFMA=1 for 1) keeps every expert row the
 * reference's serial dot_mxfp4_f32_scalar sum, bit for bit; 1 runs the
 * products on the matrix cores (f32 MFMA over the exact f32 weights
 * lut * 2^(e-127) and the f32 activations), whose sums differ from the serial
 * ones in rounding only (within 1e-4 of sum |w x| per product).  Returns the
 * previous setting. */
int rusty_hip_set_expert_mfma(int on);
/* The batched expert product on DEVICE buffers (no counterpart in the
 * reference; the product the gpt-oss prefill runs per layer, for tests and
 * callers that route tokens themselves): for every pair p < n_pairs with
 * expert e = sel[p] (0 <= e < n_exp; other values select nothing),
 * y[p * ldy + r] = sum over c of row r of expert e's MXFP4 matrix times
 * x[(x_per_pair ? p : p / top_k) * ldx + c], r < rows, c < cols.  Expert e's
 * row r starts at w + e * exp_stride + r * row_stride (row_stride a multiple
 * of 16 holding cols / 32 blocks of 17 bytes).  mfma = 0: the serial sums
 * (bit-exact with dot_mxfp4_f32_scalar, src/simd.rs:5886-5902); 1: the
 * matrix cores.  n_pairs <= 1024.  Waits for all device work first
 * and returns once y is written; returns 0 on bad arguments. */
int rusty_hip_mxfp4_experts(const uint8_t *w, int64_t row_stride, int64_t exp_stride, uint32_t n_exp, uint32_t rows,
                            uint32_t cols, const float *x, int64_t ldx, int x_per_pair, uint32_t top_k,
                            const int32_t *sel, uint32_t n_pairs, float *y, int64_t ldy, int mfma);
/* Copies slots [slot0, slot0+n_slots) of layer l's K (which = 0) or V
 * (which = 1) cache to / from host memory. */
int rusty_hip_resident_kv_read(uint32_t l, uint32_t which, uint32_t slot0, uint32_t n_slots, float *host_out);
int rusty_hip_resident_kv_write(uint32_t l, uint32_t which, uint32_t slot0, uint32_t n_slots, const float *host_in);

/* KVCache::enable_bf16 (src/model.rs:1406-1421) for the standard resident
 * decoder (no reference GPU counterpart; the reference's bf16 cache is a CPU
 * path): on = 1 switches the cache to bf16 elements, narrowed as
 * KVCache::write_k / write_v do (f32_to_bf16, round to nearest even), and
 * attention becomes attention_over_kv_heads_bf16 (src/model.rs:6205-6580):
 * the same recurrence over widened rows, with every head's scores in
 * dot_bf16_f32's single-accumulator order.  Call after configure; the cache
 * is cleared by the switch.  kv_read / kv_write then move uint16 elements
 * (n_slots * width * 2 bytes).  Split-K attention has no bf16 form: with a
 * bf16 cache the reference order runs in both attention modes.  Returns 0
 * in gpt-oss mode (the reference keeps bf16 KV to the standard
 * architecture). */
int rusty_hip_resident_enable_bf16(int on);

/* gpt-oss mode of the resident decoder: the whole forward_gpt_oss_into step
 * (src/model.rs:6733-6908) on the device, one graph per token.  The reference
 * runs this model on the CPU with per-op GPU hooks; this path has no Metal
 * counterpart.  Per layer: RMSNorm, Q/K/V (+ biases), RoPE with the YaRN
 * concentration, KV store, attention with per-head sinks (sliding window on
 * even layers), wo (+ bo) into the residual, RMSNorm, the routed MoE block
 * (as rusty_hip_moe_ffn) into the residual.  Configure with this call, then
 * set every layer with rusty_hip_resident_set_moe_layer, then
 * rusty_hip_resident_set_output / _set_embedding; decode, generate, kv_read
 * and time_decode work as for the standard decoder.  value_dim = head_dim.
 * storage_len is the cache's max_len (positions accepted).  With
 * sliding_window > 0 the KV cache is the reference's ring of
 * min(sliding_window, max_len) slots, position p in slot p % slots
 * (KVCache::with_sliding_window / slot_for_pos, src/model.rs:1363-1464), and
 * every layer reads it with slot_count = slots: the even layers over the
 * window, the odd layers from position 0 (src/model.rs:6786-6810), which
 * revisits slots once pos >= slots exactly as the reference's slot walk
 * does.  kv_read / kv_write address ring slots.  forward_gpt_oss_into has no
 * start position, so resident_decode ignores start_t in this mode. */
typedef struct {
    const uint8_t *w[4];       /* wq, wk, wv, wo */
    uintptr_t w_len[4];
    uint32_t w_dt[4];          /* GGML type ids */
    const float *bq, *bk, *bv, *bo;
    const float *sinks;        /* n_heads */
    const float *attn_norm, *post_attn_norm;
    const uint8_t *router;     /* [n_experts][dim] */
    uintptr_t router_len;
    uint32_t router_dt;
    const float *router_bias;  /* n_experts */
    const uint8_t *exps[3];    /* gate, up [n_experts*hidden][dim]; down [n_experts*dim][hidden] */
    uintptr_t exps_len[3];
    uint32_t exps_dt;
    const float *exps_bias[3]; /* [n_experts][hidden] x 2, [n_experts][dim] */
} RustyMoeLayerDesc;
int rusty_hip_resident_configure_moe(uint32_t n_layers, uint32_t dim, uint32_t n_heads, uint32_t n_kv_heads,
                                     uint32_t head_dim, uint32_t hidden_dim, uint32_t n_experts, uint32_t top_k,
                                     uint32_t vocab, uint32_t storage_len, uint32_t sliding_window, float eps,
                                     float rope_concentration);
int rusty_hip_resident_set_moe_layer(uint32_t l, const RustyMoeLayerDesc *desc);

/* No reference counterpart: rusty_hip_attention for callers that cannot
 * allocate device memory (tight serving loops, harnesses that forbid
 * hipMalloc).  Same arguments, checks, numerics and attention mode as
 * rusty_hip_attention, but query, keys, values, sinks and out are DEVICE
 * pointers, and the call makes no allocation: its scratch (the exact order's
 * scores, coefficients and masks, or the split-K partials) is one fixed
 * 16 MiB device array per GPU, held until the process ends.  Returns 0, with
 * a message on stderr, when a call needs more than that (exact order: about
 * 8.2 bytes per query head per attended position, so heads x positions up to
 * ~2 M, e.g. 40 heads over 49152 positions).  Ordering: the call first waits
 * for all work already submitted to the device (so inputs written on any of
 * the caller's streams are complete), then runs on the library's own stream
 * and returns once out is written.  It is synchronous and therefore cannot be
 * recorded into a caller's HIP graph.  Calls that overlap on one GPU share
 * the scratch array and race. */
int rusty_hip_attention_noalloc(const float *query, uintptr_t query_len, const float *keys, uintptr_t keys_len,
                                const float *values, uintptr_t values_len, const float *sinks, uintptr_t sinks_len,
                                float *out, uintptr_t out_len, uintptr_t heads, uintptr_t kv_mul, uintptr_t head_dim,
                                uintptr_t value_dim, uintptr_t key_stride, uintptr_t value_stride,
                                uintptr_t slot_count, uintptr_t start_t, uintptr_t end_t, float scale, int use_sink);

/* ===== GGUF on-disk path (src/gguf.rs; src/model.rs:40-120, 3573-3860,
 * 5180-5420) ============================================================== */

/* What the reference's parser and loaders read from a GGUF v3 file
 * (GGUFFile::parse, Config::from_gguf and load_model's head/value dim
 * override from the attn_q / attn_v shapes).  Host only: needs no GPU. */
typedef struct {
    char arch[32];              /* general.architecture (default "llama") */
    uint32_t version, n_tensors;
    uint64_t data_offset;       /* start of tensor data (general.alignment, default 32) */
    uint32_t n_layers, dim, n_heads, n_kv_heads, head_dim, value_dim, hidden_dim, vocab;
    uint32_t context_length, sliding_window, n_experts, top_k, rope_orig_ctx;
    float rope_theta, rms_eps, rope_scaling;
    uint32_t tied_output;       /* no output.weight: the head reuses token_embd (src/model.rs:3653-3667) */
    uint32_t fused_qkv;         /* blk.N.attn_qkv.weight instead of attn_q/k/v (:3795-3859) */
    uint32_t qkv_bias;
} RustyGgufSummary;
int rusty_hip_gguf_summary(const char *path, RustyGgufSummary *out);

/* Configures the resident decoder from a GGUF file (no reference
 * counterpart: the reference's Rust loader would call the resident exports
 * itself).  llama / qwen2 / qwen3 files go through rusty_hip_resident_configure
 * and set_layer as load_model maps them (tied output, fused attn_qkv split by
 * rows, the shape override of head/value dim); gpt-oss files through
 * configure_moe / set_moe_layer as load_gpt_oss_model maps them.  RoPE
 * tables are built as the reference's DecodeBuffer does (build_rope_inv_freq,
 * or the YaRN table for gpt-oss).  max_len is the cache length.  The file is
 * mapped read-only and unmapped before the call returns; weights are copied
 * through pinned staging buffers into the decoder's own device copies.
 * Returns 0 for an unreadable file, a missing tensor or a shape the decoder
 * does not take (RUSTY_HIP_DEBUG=1 prints which). */
int rusty_hip_resident_load_gguf(const char *path, uint32_t max_len);

/* Attention order for every later call (no reference counterpart).
 * 0 (default): the reference's serial online-softmax order with glibc's expf,
 * bit for bit (src/model.rs:5739-6198); 1: split-K flash decode, within
 * 1e-4 x row norm but not bit-exact.  RUSTY_HIP_ATTN=fast picks 1 at start.
 * Returns the previous mode; other values only query. */
int rusty_hip_attention_mode(int mode);

/* Frees every device weight copy cached for the per-op exports (no reference
 * counterpart: the Metal cache lives as long as the process because the
 * reference's weights are mmap'd and never freed).  Call it before freeing
 * host weight memory whose addresses may be reused.  The resident decoder
 * holds copies of its own, uploaded by set_layer / set_moe_layer /
 * set_output / set_embedding and freed by the next configure, so this call
 * leaves a configured decoder working. */
int rusty_hip_weight_cache_clear(void);

/* Timing on the library's stream (the stream every kernel is launched on). */
int rusty_hip_sync(void);
/* Per-kernel-family timing: while enabled, graphs are bypassed and each
 * family's launch is timed by a HIP event pair that the dispatch itself
 * stamps (hipExtLaunchKernel start/stop events) on the library stream. */
int rusty_hip_profile_enable(int on);
/* Family i: returns 0 past the last one; fills name (<= 63 chars), total
 * milliseconds and launch count accumulated since enable. */
int rusty_hip_profile_get(int i, char *name, double *total_ms, int64_t *count);
/* Times n_tokens decode steps (graph replays in device-token mode) between
 * two HIP events on the library stream; returns elapsed ms via *ms. */
int rusty_hip_resident_time_decode(uint32_t n_tokens, float repeat_penalty, double *ms);

/* Kernel sweep (bench only; no reference counterpart: the reference's own
 * kernel bench, runtime.rs:2639 and :5448-5474, times its CPU kernels).
 * Each runs `iters` launches on device-resident inputs rotated over `copies`
 * device copies (so launches stream from HBM, not from caches), recording
 * kernel durations in the profile families when profiling is on, and returns
 * the last launch's output.  bench_matvec: y = W x for one GGML type
 * (x quantized on the device as the reference does).  bench_attention:
 * decode attention over ctx linear slots of pseudo-normal K/V (head_dim =
 * value_dim, scale 1/sqrt(head_dim)); mode 0 exact, 1 split-K. */
int rusty_hip_bench_matvec(uint32_t ggml_type, const uint8_t *weights, uintptr_t weights_len, const float *x,
                           uintptr_t rows, uintptr_t cols, uint32_t copies, uint32_t iters, float *out);
int rusty_hip_bench_attention(uint32_t heads, uint32_t kv_mul, uint32_t head_dim, uint32_t ctx, uint32_t copies,
                              uint32_t iters, uint32_t seed, int mode, float *out);

/* Test hooks (device results of single stages, for bit-exactness checks). */
int rusty_hip_debug_quantize_q8k(const float *x, uintptr_t n, int8_t *qs, float *d, int16_t *bsums);
int rusty_hip_debug_dequant(uint32_t ggml_type, const uint8_t *weights, uintptr_t weights_len, uintptr_t rows,
                            uintptr_t cols, float *out);
int rusty_hip_debug_block_ints(uint32_t ggml_type, const uint8_t *weights, uintptr_t weights_len, uintptr_t rows,
                               uintptr_t cols, const float *x, int32_t *out);
int rusty_hip_debug_rmsnorm(const float *x, const float *w, float eps, uintptr_t n, float *out);
int rusty_hip_debug_silu_mul(const float *gate, const float *up, uintptr_t n, float *out);
int rusty_hip_debug_rope(float *q, float *k, uint32_t pos, uint32_t head_dim, uint32_t n_heads, uint32_t n_kv_heads,
                         const float *inv_freq, uint32_t neox);
int rusty_hip_debug_greedy(const float *logits, uintptr_t n, const int32_t *recent, uint32_t n_recent, float penalty,
                           int32_t *token);
int rusty_hip_debug_f16(const uint16_t *h, uintptr_t n, float *out);
int rusty_hip_debug_expf(const float *x, uintptr_t n, float *out);
/* Marks the resident decoder's next streamed attention launch as timed out
 * (what a bounded wait that ran out records): its waits return at once, it
 * ends normally with invalid values, and the decode call that ran it returns
 * 0.  Test hook for that failure path; 0 when no streamed launch exists. */
int rusty_hip_debug_stream_mark(void);

#ifdef __cplusplus
}
#endif
#endif
