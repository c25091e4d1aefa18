/*
 * llama.c — CPU restatement of the non-matmul steps of one LlamaModelInt8
 * decoder layer and of greedy sampling (TEST INFRASTRUCTURE ONLY: the
 * checker for the GPU decoder layer, never linked into the product).
 *
 * Every step follows the reference's f32 evaluation order: sequential sums
 * from 0.0, no fused multiply-add (built with -ffp-contract=off), and the C
 * library's expf / powf / cosf / sinf, which are the functions Rust's f32
 * exp / powf / cos / sin call on x86-64 Linux.
 */
#include "oracle.h"

#include <math.h>
#include <stdio.h>
#include <string.h>

/* rmsnorm, ops/norm/rmsnorm.rs (the row loop of `rmsnorm`):
 *   mean_sq = (sum_i x_i*x_i) / d     (sequential f32)
 *   rms_inv = 1 / sqrt(mean_sq + eps)
 *   out_i   = w_i * (x_i * rms_inv)                                      */
void orc_rmsnorm(const float *x, size_t rows, size_t d, const float *w, float eps, float *out) {
    for (size_t r = 0; r < rows; r++) {
        const float *xr = x + r * d;
        float sum = 0.0f;
        for (size_t i = 0; i < d; i++) {
            float sq = xr[i] * xr[i];
            sum = sum + sq;
        }
        float mean_sq = sum / (float)d;
        float rms_inv = 1.0f / sqrtf(mean_sq + eps);
        for (size_t i = 0; i < d; i++) {
            float t = xr[i] * rms_inv;
            out[r * d + i] = w[i] * t;
        }
    }
}

/* RopeTable::new, ops/rope.rs: theta_i = 1 / base^(2i / head_dim),
 * angle = pos * theta_i, tables [max_seq][head_dim/2] of cos and sin.   */
void orc_rope_table(size_t max_seq, size_t head_dim, float base, float *cos_out, float *sin_out) {
    const size_t half = head_dim / 2;
    for (size_t pos = 0; pos < max_seq; pos++) {
        for (size_t i = 0; i < half; i++) {
            float e = (2.0f * (float)i) / (float)head_dim;
            float theta = 1.0f / powf(base, e);
            float angle = (float)pos * theta;
            cos_out[pos * half + i] = cosf(angle);
            sin_out[pos * half + i] = sinf(angle);
        }
    }
}

/* rope_apply, ops/rope.rs: x [seq, n_heads, head_dim] in place, pairs
 * (2i, 2i+1) rotated by the table row start_pos + s:
 *   x0' = x0*c - x1*s,   x1' = x1*c + x0*s                                */
int orc_rope_apply(float *x, size_t seq, size_t n_heads, size_t head_dim, const float *cos_t,
                   const float *sin_t, size_t max_seq, size_t start_pos) {
    if (head_dim % 2 != 0) return ORC_INVALID_SHAPE;
    if (start_pos + seq > max_seq) return ORC_INVALID_SHAPE;
    const size_t half = head_dim / 2;
    for (size_t s = 0; s < seq; s++) {
        const size_t pos = start_pos + s;
        for (size_t h = 0; h < n_heads; h++) {
            float *b = x + (s * n_heads + h) * head_dim;
            for (size_t i = 0; i < half; i++) {
                float c = cos_t[pos * half + i], sn = sin_t[pos * half + i];
                float x0 = b[2 * i], x1 = b[2 * i + 1];
                float a0 = x0 * c, a1 = x1 * sn;
                float b0 = x1 * c, b1 = x0 * sn;
                b[2 * i] = a0 - a1;
                b[2 * i + 1] = b0 + b1;
            }
        }
    }
    return ORC_OK;
}

/* grouped_query_attention_causal_with_offset, attention/gqa.rs:217-240,
 * for every head h (kv head h / (n_heads / n_kv_heads)):
 *   scores = q_h @ k_kv^T             matmul_naive (ops/matmul/naive.rs:82-90):
 *                                     sequential sum over the head dim
 *   scores *= 1 / sqrt(d_k)           attention/sdpa.rs:226-227
 *   scores += causal mask             attention/mask.rs:77-115 (-inf for
 *                                     key j > start_pos + i)
 *   softmax per row                   ops/softmax.rs:36-57 (max, exp(v - max)
 *                                     summed sequentially, times 1/sum)
 *   out_h = weights @ v_kv            matmul_naive: sequential over keys
 * and the heads concatenated (concat_heads): out [seq_q, n_heads*head_dim].
 * Masked keys contribute exp(-inf) = 0 to the sum and 0 * v to the output,
 * so the loops stop at the last visible key (same values, fewer steps).
 * q: [seq_q, n_heads*head_dim]; k, v: [seq_k, n_kv_heads*head_dim].
 * scratch: seq_k floats.                                                  */
int orc_gqa_causal(const float *q, size_t seq_q, const float *k, const float *v, size_t seq_k,
                   size_t n_heads, size_t n_kv_heads, size_t head_dim, size_t start_pos,
                   float *out, float *scratch) {
    if (n_kv_heads == 0 || n_heads % n_kv_heads != 0) return ORC_INVALID_SHAPE;
    if (seq_q == 0 || seq_k == 0 || start_pos + seq_q > seq_k) return ORC_INVALID_SHAPE;
    const size_t groups = n_heads / n_kv_heads;
    const size_t qd = n_heads * head_dim, kvd = n_kv_heads * head_dim;
    const float scale = 1.0f / sqrtf((float)head_dim);
    for (size_t h = 0; h < n_heads; h++) {
        const size_t kh = h / groups;
        for (size_t i = 0; i < seq_q; i++) {
            const float *qi = q + i * qd + h * head_dim;
            const size_t nvis = start_pos + i + 1;  // keys 0 .. start_pos + i
            float mx = -INFINITY;
            for (size_t j = 0; j < nvis; j++) {
                const float *kj = k + j * kvd + kh * head_dim;
                float acc = 0.0f;
                for (size_t p = 0; p < head_dim; p++) {
                    float t = qi[p] * kj[p];
                    acc = acc + t;
                }
                float sc = acc * scale;
                sc = sc + 0.0f;  // the mask's 0 for a visible key
                scratch[j] = sc;
                mx = fmaxf(mx, sc);
            }
            float sum = 0.0f;
            for (size_t j = 0; j < nvis; j++) {
                scratch[j] = expf(scratch[j] - mx);
                sum = sum + scratch[j];
            }
            const float inv = 1.0f / sum;
            for (size_t j = 0; j < nvis; j++) scratch[j] = scratch[j] * inv;
            float *oi = out + i * qd + h * head_dim;
            for (size_t p = 0; p < head_dim; p++) oi[p] = 0.0f;
            for (size_t j = 0; j < nvis; j++) {
                const float *vj = v + j * kvd + kh * head_dim;
                const float wj = scratch[j];
                for (size_t p = 0; p < head_dim; p++) {
                    float t = wj * vj[p];
                    oi[p] = oi[p] + t;
                }
            }
        }
    }
    return ORC_OK;
}

/* swiglu, ops/activation/swiglu.rs: out = silu(gate) * up with
 * silu_scalar(x) = x / (1 + exp(-x)) (ops/activation/silu.rs:23-26).   */
void orc_swiglu(const float *gate, const float *up, size_t n, float *out) {
    for (size_t i = 0; i < n; i++) {
        float g = gate[i];
        float den = 1.0f + expf(-g);
        float s = g / den;
        out[i] = s * up[i];
    }
}

/* argmax, sampling/mod.rs:144-151: Iterator::max_by over partial_cmp, which
 * keeps the LAST of equal maxima; 0 for an empty slice.  (The reference
 * panics on NaN; NaN never compares greater here.)                       */
uint32_t orc_argmax(const float *v, size_t n) {
    if (n == 0) return 0;
    size_t best = 0;
    for (size_t i = 1; i < n; i++)
        if (v[i] >= v[best]) best = i;
    return (uint32_t)best;
}
