/*
 * mri_llama.h — C ABI of the GPU LlamaModelInt8 (decoder layers, output
 * head and greedy decoding) built on the quantized-matmul entry points of
 * mri_qmatmul.h.
 *
 * Drop-in for src/model/llama/forward_int8.rs: LlamaModelInt8 (:416-546)
 * and TransformerBlockInt8 (:148-402), with the KvCache of
 * src/cache/kv_cache.rs.  All seven projections of every layer and the
 * output projection run through mri_matmul_int8_from_f32 (per-channel
 * INT8, as the reference), mri_matmul_q8_0_direct or
 * mri_matmul_q4_0_dequant, chosen per weight.
 *
 * Activations, logits, the KV cache and the embedding table live in device
 * memory; token ids passed to the forward calls are host values.  Calls are
 * asynchronous on `stream` (hipStream_t; NULL = default stream).  A model
 * handle keeps per-handle activation buffers: calls on one handle must be
 * ordered (one stream, or synchronized), like the reference's &mut self of
 * the cache they update.
 *
 * Numerics: projections as documented in mri_qmatmul.h; RoPE is bit-exact
 * given the reference's table (computed here on the host with the same
 * libm calls as RopeTable::new); RMSNorm, softmax, the attention value sum
 * and SwiGLU's exp agree with the reference to f32 rounding.
 */
#ifndef MRI_LLAMA_H
#define MRI_LLAMA_H

#include "mri_qmatmul.h"

#ifdef __cplusplus
extern "C" {
#endif

/* LlamaConfig fields the forward pass uses (src/model/llama/config.rs):
 * embedding_length, head_count, head_count_kv, feed_forward_length,
 * vocab_size, context_length (the RoPE table and cache length),
 * rms_norm_eps, rope_freq_base, block_count. */
typedef struct mri_llama_config {
    size_t dim;
    size_t n_heads;
    size_t n_kv_heads;
    size_t ffn_dim;
    size_t vocab;
    size_t max_seq;
    float eps;
    float rope_base;
    size_t n_layers;
} mri_llama_config;

typedef enum mri_weight_format {
    MRI_WEIGHT_INT8 = 0, /* const mri_qmatrix *       */
    MRI_WEIGHT_Q8_0 = 1, /* const mri_q8_0_matrix *   */
    MRI_WEIGHT_Q4_0 = 2, /* device pointer to raw Q4_0 blocks, n_out x k_in */
    /* const mri_q4_0_matrix *: Q4_0 weights projected with int8 activations
     * (mri_matmul_q4_0_w4a8, an extension without a reference counterpart) */
    MRI_WEIGHT_Q4_0_W4A8 = 3
} mri_weight_format;

/* A projection weight [n_out, k_in] (GGUF "out, in" layout).  The handle or
 * buffer is borrowed: it must outlive the model.  n_out / k_in are checked
 * against the role's shape. */
typedef struct mri_weight_ref {
    int format; /* mri_weight_format */
    const void *ptr;
    size_t n_out;
    size_t k_in;
} mri_weight_ref;

typedef struct mri_llama mri_llama;
typedef struct mri_kv_cache mri_kv_cache;

/* LlamaModelInt8::new, forward_int8.rs:430-444: token_embd [vocab, dim] and
 * output_norm [dim] are host f32 arrays (copied to the device); `output` is
 * the [vocab, dim] unembedding projection.  Layers are set with
 * mri_llama_set_layer before the first forward call.  InvalidShape for
 * inconsistent dimensions (n_heads % n_kv_heads, dim % n_heads, odd head
 * dim); Unsupported for a head dim other than 64 or 128. */
mri_status mri_llama_create(const mri_llama_config *cfg, const float *token_embd,
                            const float *output_norm, mri_weight_ref output,
                            mri_llama **out);
/* TransformerBlockInt8::new, forward_int8.rs:168-198: norms are host f32
 * [dim]; w[0..6] = wq [n_heads*hd, dim], wk, wv [n_kv*hd, dim],
 * wo [dim, n_heads*hd], wgate, wup [ffn, dim], wdown [dim, ffn].  When wq,
 * wk, wv (and wgate, wup) are handles of one format (INT8, Q8_0 or W4A8)
 * whose n_out are multiples of 16, the model builds owned row
 * concatenations of them here and projects once per group; outputs equal
 * the separate projections'.  Setting a layer again replaces them. */
mri_status mri_llama_set_layer(mri_llama *model, size_t layer, const float *attn_norm,
                               const float *ffn_norm, const mri_weight_ref w[7]);
void mri_llama_destroy(mri_llama *model);

/* KvCache::new, src/cache/kv_cache.rs:65: [n_layers][max_seq][n_kv*hd] f32
 * for K and V, zero-filled, on the device. */
mri_status mri_kv_cache_create(size_t n_layers, size_t max_seq, size_t n_kv_heads,
                               size_t head_dim, mri_kv_cache **out);
void mri_kv_cache_destroy(mri_kv_cache *cache);

/* Prefill of n tokens at positions start_pos .. start_pos + n - 1:
 * embed (forward_int8.rs:125-140), TransformerBlockInt8::forward_cached per
 * layer (:207-216, writing the cache), rmsnorm and the output projection
 * (:526-528).  logits: device [n, vocab].  InvalidShape for n == 0, a token
 * id >= vocab, or start_pos + n beyond the cache / RoPE table. */
mri_status mri_llama_forward_cached(mri_llama *model, const uint32_t *tokens, size_t n,
                                    size_t start_pos, mri_kv_cache *cache, float *logits,
                                    void *stream);
/* LlamaModelInt8::forward_decode, forward_int8.rs:538-546: one token at
 * position pos.  logits: device [vocab]. */
mri_status mri_llama_forward_decode(mri_llama *model, uint32_t token, size_t pos,
                                    mri_kv_cache *cache, float *logits, void *stream);
/* Greedy generation: forward_cached over the prompt (positions 0 ..), then
 * n_steps decode steps (positions n_prompt ..), each fed the argmax
 * (sampling/mod.rs:144-151, last of equal maxima) of the previous logits.
 * Token ids stay on the device between steps.  tokens_out (host,
 * n_steps + 1): the argmax of the prompt's last row, then of each step; it
 * is written when the call returns (the call synchronizes `stream`).
 * logits_out (device, nullable, [n_steps + 1, vocab]) receives the rows of
 * logits that chose them.  InvalidShape unless 1 <= n_prompt and
 * n_prompt + n_steps <= the cache / RoPE length. */
mri_status mri_llama_generate_greedy(mri_llama *model, const uint32_t *prompt, size_t n_prompt,
                                     size_t n_steps, mri_kv_cache *cache, uint32_t *tokens_out,
                                     float *logits_out, void *stream);

/* argmax of each of `rows` rows of n f32 values (device), as
 * sampling/mod.rs:144-151; idx: device [rows]. */
mri_status mri_argmax(const float *v, size_t rows, size_t n, uint32_t *idx, void *stream);

#ifdef __cplusplus
}
#endif
#endif
