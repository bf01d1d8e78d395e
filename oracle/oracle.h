/*
 * oracle.h — CPU restatement of RustyLLM's x86-64 decode-step numerics.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the parity checker for the HIP
 * path and the in-run CPU baseline of bench.py.  Only tests/, the smoke()
 * check in __graft_entry__.py and bench.py's cpu_baseline leg may load it.
 * Nothing in rustyllm_amd/ links, imports or calls it.
 *
 * Every function restates one reference function (Rust, src/simd.rs and
 * src/model.rs of SimonWaldherr/RustyLLM) with the same operation order; the
 * citation is on each definition in oracle.c.  The library is built with
 * -ffp-contract=off so a*b+c is never fused unless the reference calls an FMA
 * intrinsic (_mm256_fmadd_ps) at that point.
 */
#ifndef RUSTY_ORACLE_H
#define RUSTY_ORACLE_H

#include <stdint.h>
#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

/* GGML type ids (reference src/gguf.rs:12-30). */
enum {
    ORC_F32 = 0,
    ORC_Q8_0 = 8,
    ORC_Q4_K = 12,
    ORC_Q6_K = 14,
    ORC_MXFP4 = 39,
};

/* ---- scalar helpers ---------------------------------------------------- */
float orc_f16_to_f32(uint16_t h);
float orc_mxfp4_scale(uint8_t e);

/* ---- Q8_K activation quantizer ---------------------------------------- */
void orc_quantize_row_q8k_scalar(const float *x, int64_t n, int8_t *qs, float *d, int16_t *bsums);
void orc_quantize_row_q8k_avx2(const float *x, int64_t n, int8_t *qs, float *d, int16_t *bsums);

/* ---- dequantization ----------------------------------------------------- */
void orc_dequant_row(int dtype, const uint8_t *q, float *out, int64_t n);

/* ---- fused dots (one row) ---------------------------------------------- */
float orc_dot_q4_k_q8k_avx2(const uint8_t *w, const int8_t *qs, const float *d, const int16_t *bsums, int64_t n);
float orc_dot_q6_k_q8k_avx2(const uint8_t *w, const int8_t *qs, const float *d, const int16_t *bsums, int64_t n);
float orc_dot_q8_0_q8k_avx2(const uint8_t *w, const int8_t *qs, const float *d, const int16_t *bsums, int64_t n);
float orc_dot_q8_0_f32_avx2(const uint8_t *w, const float *x, int64_t n);
float orc_dot_mxfp4_f32_scalar(const uint8_t *w, const float *x, int64_t n);
float orc_dot_f32_avx2(const float *a, const float *b, int64_t n);

/* scalar integer emulations from the reference's own tests */
float orc_emulate_q4_k_q8k(const uint8_t *w, const int8_t *qs, const float *d, const int16_t *bsums, int64_t n);
float orc_emulate_q6_k_q8k(const uint8_t *w, const int8_t *qs, const float *d, int64_t n);
float orc_emulate_q8_0_q8k(const uint8_t *w, const int8_t *qs, const float *d, int64_t n);

/* per-block integer parts: Q4_K -> (isum, imin) per 256; Q6_K -> isum per 256;
 * Q8_0 -> s per 32-block. */
void orc_q4k_block_ints(const uint8_t *w, const int8_t *qs, const int16_t *bsums, int64_t n, int32_t *isum, int32_t *imin);
void orc_q6k_block_ints(const uint8_t *w, const int8_t *qs, int64_t n, int32_t *isum);
void orc_q8_0_block_ints(const uint8_t *w, const int8_t *qs, int64_t n, int32_t *s);

/* ---- matvec (reference Weight::matvec_into dispatch) -------------------- */
int64_t orc_row_bytes(int dtype, int64_t cols);
void orc_matvec(int dtype, const uint8_t *w, const float *x, int64_t rows, int64_t cols, float *out, int threads);
void orc_set_threads(int threads);
void orc_set_fast_schedule(int on);

/* ---- attention ---------------------------------------------------------- */
void orc_online_attention(const float *q, const float *keys, const float *values,
                          int64_t key_stride, int64_t value_stride, int64_t slot_count,
                          int64_t hd, int64_t vd, int64_t start_t, int64_t end_t,
                          float scale, float *out);
void orc_online_attention_with_sink(const float *q, const float *keys, const float *values,
                                    int64_t key_stride, int64_t value_stride, int64_t slot_count,
                                    int64_t hd, int64_t vd, int64_t start_t, int64_t end_t,
                                    float scale, float sink, float *out);
void orc_online_attention_grouped(const float *q, const float *keys, const float *values,
                                  int64_t key_stride, int64_t value_stride, int64_t slot_count,
                                  int64_t hd, int64_t vd, int64_t kv_mul, int64_t start_t,
                                  int64_t end_t, float scale, float *out);
void orc_attention_over_kv_heads(const float *q, const float *keys, const float *values,
                                 int64_t key_stride, int64_t value_stride, int64_t slot_count,
                                 int64_t hd, int64_t vd, int64_t n_kv, int64_t kv_mul,
                                 int64_t start_t, int64_t end_t, float scale, float *out);
/* gpt-oss per-head sink attention over all heads (reference model.rs:6815-6833) */
void orc_attention_sink_heads(const float *q, const float *keys, const float *values,
                              const float *sinks, int64_t key_stride, int64_t value_stride,
                              int64_t slot_count, int64_t hd, int64_t vd, int64_t n_heads,
                              int64_t kv_mul, int64_t start_t, int64_t end_t, float scale,
                              float *out);
int64_t orc_attention_start_pos(int64_t pos, int64_t window);

/* ---- small ops ------------------------------------------------------------ */
void orc_rms_norm(const float *x, const float *w, float eps, int64_t n, float *out);
void orc_build_rope_inv_freq(float theta, int64_t head_dim, float scaling, float *inv);
void orc_build_rope_inv_freq_gpt_oss(float theta, int64_t head_dim, float scaling, int64_t orig_ctx, float *inv,
                                     float *concentration);
void orc_rope_qk(float *q, float *k, int64_t pos, int64_t hd, int64_t nh, int64_t nkv, const float *inv_freq);
void orc_rope_qk_neox(float *q, float *k, int64_t pos, int64_t hd, int64_t nh, int64_t nkv, const float *inv_freq);
void orc_rope_gpt_oss(float *q, float *k, int64_t pos, int64_t hd, int64_t nh, int64_t nkv, float concentration,
                      const float *inv_freq);
void orc_silu_mul_avx2(const float *gate, const float *up, float *out, int64_t n);
void orc_silu_mul_scalar(const float *gate, const float *up, float *out, int64_t n);
float orc_swiglu_gpt_oss(float g, float u);
void orc_select_top_logits(const float *logits, int64_t n, int64_t k, int32_t *idx, float *val);
void orc_softmax_selected(const float *val, int64_t k, float *out);
void orc_apply_repeat_penalty(float *logits, int64_t n, const uint32_t *recent, int64_t nrecent, float penalty);
uint32_t orc_argmax_finite(const float *logits, int64_t n);
void orc_expf_array(const float *x, int64_t n, float *out);
uint32_t orc_greedy(float *logits, int64_t n, const uint32_t *recent, int64_t nrecent, float penalty);

/* ---- standard (llama / qwen2) decode model ------------------------------- */
typedef struct {
    int32_t n_layers, dim, n_heads, n_kv_heads, head_dim, value_dim, hidden_dim, vocab;
    int32_t storage_len;      /* KV slots per layer */
    int32_t sliding_window;   /* 0 = none */
    int32_t neox;             /* 1 = rotate-half RoPE (qwen2/qwen3) */
    float eps;
    int32_t kv_bf16;          /* 1 = bf16 KV cache (KVCache::enable_bf16) */
} orc_config;

/* weight order: wq, wk, wv, wo, gate(w1), up(w3), down(w2); types are GGML ids */
typedef struct {
    const uint8_t *w[7];
    uint64_t w_len[7];
    uint32_t w_rows[7];
    uint32_t w_type[7];
    const float *attn_norm;
    const float *ffn_norm;
    const float *bq; uint32_t bq_len;
    const float *bk; uint32_t bk_len;
    const float *bv; uint32_t bv_len;
} orc_layer;

typedef struct orc_model orc_model;
orc_model *orc_model_create(const orc_config *cfg);
void orc_model_free(orc_model *m);
int orc_model_set_layer(orc_model *m, int32_t l, const orc_layer *layer);
int orc_model_set_output(orc_model *m, const float *output_norm, const uint8_t *output_w,
                         uint32_t output_type, const uint8_t *embd, uint32_t embd_type,
                         const float *inv_freq);
void orc_model_forward_from(orc_model *m, uint32_t token, int64_t pos, int64_t start_t, float *logits,
                            int want_logits);
void orc_model_forward(orc_model *m, uint32_t token, int64_t pos, float *logits, int want_logits);
/* the layer's K (which = 0) or V cache: float, or uint16 bf16 with kv_bf16 */
float *orc_model_kv(orc_model *m, int32_t layer, int32_t which);
uint16_t orc_f32_to_bf16(float x);
float orc_bf16_to_f32(uint16_t h);
float orc_dot_bf16_f32_avx2(const float *a, const float *bw, int64_t n);
void orc_online_attention_grouped_bf16(const float *queries, const uint16_t *keys, const uint16_t *values, int64_t ks,
                                       int64_t vs, int64_t slots, int64_t hd, int64_t vd, int64_t kv_mul,
                                       int64_t start_t, int64_t end_t, float scale, float *out);
void orc_attention_over_kv_heads_bf16(const float *q, const uint16_t *keys, const uint16_t *values, int64_t ks,
                                      int64_t vs, int64_t slots, int64_t hd, int64_t vd, int64_t n_kv,
                                      int64_t kv_mul, int64_t start_t, int64_t end_t, float scale, float *out);
/* prefill prompt (per token) then greedy-decode n_gen tokens. Returns count. */
int64_t orc_model_generate(orc_model *m, const uint32_t *prompt, int64_t n_prompt, int64_t start_pos,
                           int64_t n_gen, float penalty, uint32_t *out_tokens, float *last_logits);

/* ---- gpt-oss decode model (forward_gpt_oss_into, model.rs:6733-6908) ---- */
typedef struct {
    int32_t n_layers, dim, n_heads, n_kv_heads, head_dim, value_dim, hidden_dim, n_experts, top_k, vocab;
    int32_t max_len;          /* positions; the ring holds min(window, max_len) of them */
    int32_t sliding_window;   /* even layers attend the last `window` positions */
    float eps, concentration; /* RMSNorm eps; YaRN concentration of the RoPE table */
} orc_gptoss_config;

typedef struct {
    const uint8_t *wq, *wk, *wv, *wo;
    uint32_t wq_type, wk_type, wv_type, wo_type;
    const float *bq, *bk, *bv, *bo, *sinks, *attn_norm, *post_attn_norm;
    const uint8_t *router;
    uint32_t router_type;
    const float *router_bias;
    const uint8_t *gate_exps, *up_exps, *down_exps; /* expert-major [n_experts][rows] */
    uint32_t exps_type;
    const float *gate_exps_bias, *up_exps_bias, *down_exps_bias; /* [n_experts][hidden|dim] */
} orc_gptoss_layer;

typedef struct orc_gptoss orc_gptoss;
orc_gptoss *orc_gptoss_create(const orc_gptoss_config *cfg);
void orc_gptoss_free(orc_gptoss *m);
int orc_gptoss_set_layer(orc_gptoss *m, int32_t l, const orc_gptoss_layer *layer);
int orc_gptoss_set_output(orc_gptoss *m, const float *output_norm, const uint8_t *output_w, uint32_t output_type,
                          const uint8_t *embd, uint32_t embd_type, const float *inv_freq);
int64_t orc_gptoss_storage(const orc_gptoss *m);
float *orc_gptoss_kv(orc_gptoss *m, int32_t layer, int32_t which);
void orc_gptoss_forward(orc_gptoss *m, uint32_t token, int64_t pos, float *logits, int want_logits);

/* ---- reference test fixtures (src/simd.rs tests) ------------------------- */
void orc_make_q4k_weights(int64_t rows, int64_t cols, uint8_t seed, uint8_t *out);
void orc_make_q4k_weights_dmin(int64_t rows, int64_t cols, uint8_t seed, uint8_t *out);
void orc_make_q6k_weights(int64_t rows, int64_t cols, uint8_t seed, uint8_t *out);
void orc_make_q8_0_row_scaled(int64_t cols, uint8_t seed, uint8_t *out);
void orc_make_mxfp4_test_row(int64_t blocks, uint8_t *out);
void orc_test_activation(int64_t cols, float *out);
void orc_mxfp4_test_activation(int64_t n, float *out);

#ifdef __cplusplus
}
#endif
#endif
