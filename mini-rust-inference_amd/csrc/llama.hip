// llama.hip — the non-matmul steps of one LlamaModelInt8 decoder layer
// (model/llama/forward_int8.rs:291-357) and greedy sampling, on gfx950.
//
// Every step works on f32 rows in HBM laid out as the reference's tensors
// ([rows, features], row-major).  Evaluation orders follow the reference
// where that costs nothing (built with -ffp-contract=off, so no implicit
// FMA): RoPE is bit-exact given the same table, every attention score is
// the reference's sequential dot product; sums over a row (RMSNorm, the
// softmax denominator, the attention-weighted values) are tree or
// multi-wave sums and therefore agree to rounding only.
#include <hip/hip_runtime.h>

#include <cfloat>

#include "common.hpp"

namespace mri {
namespace {

constexpr int kWave = 64;

__device__ inline float wave_sum(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, kWave);
    return v;
}
__device__ inline float wave_max(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, kWave));
    return v;
}

// ---- embedding lookup (forward_int8.rs:125-140) ------------------------------
// x[r, :] = table[tokens[r], :].  Token ids are checked against the vocabulary
// on the host, or come from the argmax kernel (always < vocab).
__global__ __launch_bounds__(256) void k_embed(const float *__restrict__ table,
                                               const uint32_t *__restrict__ tokens, int d,
                                               float *__restrict__ x) {
    const size_t src = (size_t)tokens[blockIdx.x] * d, dst = (size_t)blockIdx.x * d;
    for (int i = threadIdx.x; i < d; i += 256) x[dst + i] = table[src + i];
}

// ---- RMSNorm (ops/norm/rmsnorm.rs) ------------------------------------------------
// One workgroup per row: mean_sq = sum(x*x) / d, rms_inv = 1 / sqrt(mean_sq +
// eps) (correctly rounded divide and sqrt), out = w * (x * rms_inv).
__global__ __launch_bounds__(256) void k_rmsnorm(const float *__restrict__ x,
                                                 const float *__restrict__ w, int d, float eps,
                                                 float *__restrict__ out) {
    __shared__ float s_part[4];
    const float *xr = x + (size_t)blockIdx.x * d;
    float *orow = out + (size_t)blockIdx.x * d;
    float acc = 0.0f;
    for (int i = threadIdx.x; i < d; i += 256) {
        const float sq = xr[i] * xr[i];
        acc = acc + sq;
    }
    acc = wave_sum(acc);
    if ((threadIdx.x & 63) == 0) s_part[threadIdx.x >> 6] = acc;
    __syncthreads();
    const float sum = ((s_part[0] + s_part[1]) + s_part[2]) + s_part[3];
    const float mean_sq = sum / (float)d;
    const float rms_inv = 1.0f / sqrtf(mean_sq + eps);
    for (int i = threadIdx.x; i < d; i += 256) {
        const float t = xr[i] * rms_inv;
        orow[i] = w[i] * t;
    }
}

// ---- RoPE + KV-cache write (ops/rope.rs, attention/cached.rs) --------------------------
// Row s of q (n_heads heads) and k (n_kv heads) is rotated with table row
// start_pos + s: pair (2i, 2i+1) -> (x0*c - x1*s, x1*c + x0*s).  q is
// rotated in place; the rotated k row and the v row are written to the
// cache at position start_pos + s (write_k / write_v).
__global__ __launch_bounds__(256) void k_rope_qkv(float *__restrict__ q,
                                                  const float *__restrict__ k,
                                                  const float *__restrict__ v, int qd, int kvd,
                                                  int half, const float *__restrict__ cos_t,
                                                  const float *__restrict__ sin_t, int start_pos,
                                                  float *__restrict__ kc,
                                                  float *__restrict__ vc) {
    const int s = blockIdx.x, pos = start_pos + s;
    const float *ct = cos_t + (size_t)pos * half, *st = sin_t + (size_t)pos * half;
    float *qr = q + (size_t)s * qd;
    for (int p = threadIdx.x; p < qd / 2; p += 256) {
        const int i = p % half;
        const float c = ct[i], sn = st[i];
        const float x0 = qr[2 * p], x1 = qr[2 * p + 1];
        const float a0 = x0 * c, a1 = x1 * sn, b0 = x1 * c, b1 = x0 * sn;
        qr[2 * p] = a0 - a1;
        qr[2 * p + 1] = b0 + b1;
    }
    const float *kr = k + (size_t)s * kvd;
    float *kd = kc + (size_t)pos * kvd;
    for (int p = threadIdx.x; p < kvd / 2; p += 256) {
        const int i = p % half;
        const float c = ct[i], sn = st[i];
        const float x0 = kr[2 * p], x1 = kr[2 * p + 1];
        const float a0 = x0 * c, a1 = x1 * sn, b0 = x1 * c, b1 = x0 * sn;
        kd[2 * p] = a0 - a1;
        kd[2 * p + 1] = b0 + b1;
    }
    const float *vr = v + (size_t)s * kvd;
    float *vd = vc + (size_t)pos * kvd;
    for (int i = threadIdx.x; i < kvd; i += 256) vd[i] = vr[i];
}

// ---- causal grouped-query attention (attention/gqa.rs:217-240) --------------------------
// Workgroup (query block b, head h): QB query rows i (absolute positions
// start_pos + i) against the keys 0 .. L-1 of kv head h / groups in the
// cache, L = start_pos + last row + 1.  Same three passes as the reference:
//  1. scores: lane j of the workgroup owns key j and computes its dot product
//     with each of the QB queries sequentially over the head dimension
//     (matmul_naive's order), times 1/sqrt(head_dim); keys after a row's
//     position get -inf (causal mask).  The queries sit in LDS and are read
//     as broadcasts; each key row is read once per workgroup.
//  2. softmax per row: max, exp(s - max), sum, times 1/sum.
//  3. values: wave w sums its quarter of the keys, lane l owning dims
//     HD/64 * l ..; the four partial rows are added in wave order.
// LDS: queries [QB][HD], weights [QB][Lcap], partials [4][QB][HD].
template <int HD, int QB>
__global__ __launch_bounds__(256) void k_attention(
    const float *__restrict__ q, int qd, const float *__restrict__ kc,
    const float *__restrict__ vc, int kvd, int seq_q, int start_pos, int groups, int lcap,
    float scale, float *__restrict__ out) {
    constexpr int E = HD / kWave;  // dims per lane in the value pass
    extern __shared__ float s_mem[];
    float *s_q = s_mem;                    // [QB][HD]
    float *s_p = s_q + QB * HD;            // [QB][lcap]
    float *s_o = s_p + (size_t)QB * lcap;  // [4][QB][HD]
    const int t = threadIdx.x, lane = t & 63, wv = t >> 6;
    const int h = blockIdx.y, kh = h / groups;
    const int i0 = blockIdx.x * QB;
    const int nq = min(QB, seq_q - i0);
    const int L = start_pos + i0 + nq;  // keys the block's last row sees
    for (int e = t; e < QB * HD; e += 256) {
        const int qq = e / HD, p = e % HD;
        s_q[e] = qq < nq ? q[(size_t)(i0 + qq) * qd + h * HD + p] : 0.0f;
    }
    __syncthreads();
    // 1. scores
    for (int j = t; j < L; j += 256) {
        float acc[QB];
#pragma unroll
        for (int qq = 0; qq < QB; ++qq) acc[qq] = 0.0f;
        const float4 *kr = reinterpret_cast<const float4 *>(kc + (size_t)j * kvd + kh * HD);
#pragma unroll 4
        for (int p4 = 0; p4 < HD / 4; ++p4) {
            const float4 kv = kr[p4];
#pragma unroll
            for (int qq = 0; qq < QB; ++qq) {
                const float4 qv = reinterpret_cast<const float4 *>(s_q + qq * HD)[p4];
                float m0 = qv.x * kv.x;
                acc[qq] = acc[qq] + m0;
                m0 = qv.y * kv.y;
                acc[qq] = acc[qq] + m0;
                m0 = qv.z * kv.z;
                acc[qq] = acc[qq] + m0;
                m0 = qv.w * kv.w;
                acc[qq] = acc[qq] + m0;
            }
        }
#pragma unroll
        for (int qq = 0; qq < QB; ++qq) {
            const float sc = acc[qq] * scale;
            s_p[qq * lcap + j] = j <= start_pos + i0 + qq ? sc + 0.0f : -INFINITY;
        }
    }
    __syncthreads();
    // 2. softmax of each row (wave wv takes rows wv, wv + 4, ...)
    for (int qq = wv; qq < nq; qq += 4) {
        float *row = s_p + qq * lcap;
        float m = -INFINITY;
        for (int j = lane; j < L; j += kWave) m = fmaxf(m, row[j]);
        m = wave_max(m);
        float sum = 0.0f;
        for (int j = lane; j < L; j += kWave) {
            const float e = expf(row[j] - m);
            row[j] = e;
            sum = sum + e;
        }
        sum = wave_sum(sum);
        const float inv = 1.0f / sum;
        for (int j = lane; j < L; j += kWave) row[j] = row[j] * inv;
    }
    __syncthreads();
    // 3. weighted values: wave wv sums keys [j0, j1)
    const int j0 = (int)((long long)L * wv / 4), j1 = (int)((long long)L * (wv + 1) / 4);
    float o[QB][E];
#pragma unroll
    for (int qq = 0; qq < QB; ++qq)
#pragma unroll
        for (int e = 0; e < E; ++e) o[qq][e] = 0.0f;
    for (int j = j0; j < j1; ++j) {
        const float *vr = vc + (size_t)j * kvd + kh * HD + lane * E;
        float vv[E];
#pragma unroll
        for (int e = 0; e < E; ++e) vv[e] = vr[e];
#pragma unroll
        for (int qq = 0; qq < QB; ++qq) {
            const float w = s_p[qq * lcap + j];
#pragma unroll
            for (int e = 0; e < E; ++e) {
                const float m0 = w * vv[e];
                o[qq][e] = o[qq][e] + m0;
            }
        }
    }
#pragma unroll
    for (int qq = 0; qq < QB; ++qq)
#pragma unroll
        for (int e = 0; e < E; ++e) s_o[(wv * QB + qq) * HD + lane * E + e] = o[qq][e];
    __syncthreads();
    for (int e = t; e < nq * HD; e += 256) {
        const int qq = e / HD, p = e % HD;
        const float r = ((s_o[(0 * QB + qq) * HD + p] + s_o[(1 * QB + qq) * HD + p]) +
                         s_o[(2 * QB + qq) * HD + p]) +
                        s_o[(3 * QB + qq) * HD + p];
        out[(size_t)(i0 + qq) * qd + h * HD + p] = r;
    }
}

// ---- SwiGLU (ops/activation/swiglu.rs): out = gate / (1 + exp(-gate)) * up ----
__global__ __launch_bounds__(256) void k_swiglu(const float *__restrict__ gate,
                                                const float *__restrict__ up, size_t n,
                                                float *__restrict__ out) {
    for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (size_t)gridDim.x * 256) {
        const float g = gate[i];
        const float den = 1.0f + expf(-g);
        const float s = g / den;
        out[i] = s * up[i];
    }
}

// ---- residual add (forward_int8.rs:100-121): out = a + b -------------------------------
__global__ __launch_bounds__(256) void k_add(const float *__restrict__ a,
                                             const float *__restrict__ b, size_t n,
                                             float *__restrict__ out) {
    for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (size_t)gridDim.x * 256)
        out[i] = a[i] + b[i];
}

// ---- greedy argmax (sampling/mod.rs:144-151) ----------------------------------------
// Last index of the maximum (Iterator::max_by keeps the last of equal
// maxima); NaN never wins.  One workgroup of 1024 threads per row.
__global__ __launch_bounds__(1024) void k_argmax(const float *__restrict__ v, int n,
                                                 uint32_t *__restrict__ idx) {
    __shared__ float s_v[16];
    __shared__ int s_i[16];
    const float *row = v + (size_t)blockIdx.x * n;
    float bv = -INFINITY;
    int bi = -1;
    for (int i = threadIdx.x; i < n; i += 1024) {
        const float x = row[i];
        if (bi < 0 || x >= bv) {
            if (!(x != x)) {
                bv = x;
                bi = i;
            }
        }
    }
    // (value, index) reduction: larger value, then larger index
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        const float ov = __shfl_xor(bv, o, kWave);
        const int oi = __shfl_xor(bi, o, kWave);
        if (oi >= 0 && (bi < 0 || ov > bv || (ov == bv && oi > bi))) {
            bv = ov;
            bi = oi;
        }
    }
    if ((threadIdx.x & 63) == 0) {
        s_v[threadIdx.x >> 6] = bv;
        s_i[threadIdx.x >> 6] = bi;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        float rv = s_v[0];
        int ri = s_i[0];
        for (int w = 1; w < 16; ++w)
            if (s_i[w] >= 0 && (ri < 0 || s_v[w] > rv || (s_v[w] == rv && s_i[w] > ri))) {
                rv = s_v[w];
                ri = s_i[w];
            }
        idx[blockIdx.x] = ri < 0 ? 0u : (uint32_t)ri;
    }
}

// query rows per attention workgroup: the largest of 16, 4, 1 whose LDS fits
template <int HD, int QB>
size_t attn_lds(int lcap) {
    return (size_t)(QB * HD + (size_t)QB * lcap + 4 * QB * HD) * sizeof(float);
}

template <int HD, int QB>
mri_status attn_launch(const float *q, int qd, const float *kc, const float *vc, int kvd,
                       int seq_q, int start_pos, int groups, int n_heads, float *out,
                       hipStream_t s) {
    const int L = start_pos + seq_q;
    const int lcap = (L + 3) / 4 * 4;
    const size_t lds = attn_lds<HD, QB>(lcap);
    static bool attr_set = false;
    if (!attr_set) {
        MRI_HIP(hipFuncSetAttribute(reinterpret_cast<const void *>(&k_attention<HD, QB>),
                                    hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024));
        attr_set = true;
    }
    const float scale = 1.0f / sqrtf((float)HD);
    hipLaunchKernelGGL((k_attention<HD, QB>), dim3((seq_q + QB - 1) / QB, n_heads), dim3(256),
                       lds, s, q, qd, kc, vc, kvd, seq_q, start_pos, groups, lcap, scale, out);
    MRI_LAUNCHED("k_attention");
    return MRI_OK;
}

template <int HD>
mri_status attn_dispatch(const float *q, int qd, const float *kc, const float *vc, int kvd,
                         int seq_q, int start_pos, int groups, int n_heads, float *out,
                         hipStream_t s) {
    const int lcap = (start_pos + seq_q + 3) / 4 * 4;
    constexpr size_t kMax = 160 * 1024;
    if (seq_q > 1 && attn_lds<HD, 16>(lcap) <= kMax)
        return attn_launch<HD, 16>(q, qd, kc, vc, kvd, seq_q, start_pos, groups, n_heads, out,
                                   s);
    if (seq_q > 1 && attn_lds<HD, 4>(lcap) <= kMax)
        return attn_launch<HD, 4>(q, qd, kc, vc, kvd, seq_q, start_pos, groups, n_heads, out,
                                  s);
    if (attn_lds<HD, 1>(lcap) <= kMax)
        return attn_launch<HD, 1>(q, qd, kc, vc, kvd, seq_q, start_pos, groups, n_heads, out,
                                  s);
    return set_error(MRI_ERR_UNSUPPORTED, "attention: context too long for one workgroup");
}

inline unsigned grid_for(size_t n) {
    const size_t g = (n + 255) / 256;
    return (unsigned)(g < 8192 ? (g ? g : 1) : 8192);
}

}  // namespace

mri_status launch_embed(const float *table, const uint32_t *tokens, size_t rows, size_t d,
                        float *x, hipStream_t s) {
    if (!rows) return MRI_OK;
    hipLaunchKernelGGL(k_embed, dim3((unsigned)rows), dim3(256), 0, s, table, tokens, (int)d, x);
    MRI_LAUNCHED("k_embed");
    return MRI_OK;
}

mri_status launch_rmsnorm(const float *x, const float *w, size_t rows, size_t d, float eps,
                          float *out, hipStream_t s) {
    if (!rows) return MRI_OK;
    hipLaunchKernelGGL(k_rmsnorm, dim3((unsigned)rows), dim3(256), 0, s, x, w, (int)d, eps, out);
    MRI_LAUNCHED("k_rmsnorm");
    return MRI_OK;
}

mri_status launch_rope_qkv(float *q, const float *k, const float *v, size_t seq, size_t qd,
                           size_t kvd, size_t head_dim, const float *cos_t, const float *sin_t,
                           size_t start_pos, float *kc, float *vc, hipStream_t s) {
    if (!seq) return MRI_OK;
    hipLaunchKernelGGL(k_rope_qkv, dim3((unsigned)seq), dim3(256), 0, s, q, k, v, (int)qd,
                       (int)kvd, (int)(head_dim / 2), cos_t, sin_t, (int)start_pos, kc, vc);
    MRI_LAUNCHED("k_rope_qkv");
    return MRI_OK;
}

bool attention_supported(size_t head_dim) { return head_dim == 64 || head_dim == 128; }

mri_status launch_attention(const float *q, size_t seq_q, const float *kc, const float *vc,
                            size_t n_heads, size_t n_kv_heads, size_t head_dim,
                            size_t start_pos, float *out, hipStream_t s) {
    if (!seq_q) return MRI_OK;
    const int qd = (int)(n_heads * head_dim), kvd = (int)(n_kv_heads * head_dim);
    const int groups = (int)(n_heads / n_kv_heads);
    if (head_dim == 128)
        return attn_dispatch<128>(q, qd, kc, vc, kvd, (int)seq_q, (int)start_pos, groups,
                                  (int)n_heads, out, s);
    if (head_dim == 64)
        return attn_dispatch<64>(q, qd, kc, vc, kvd, (int)seq_q, (int)start_pos, groups,
                                 (int)n_heads, out, s);
    return set_error(MRI_ERR_UNSUPPORTED, "attention: head_dim must be 64 or 128");
}

mri_status launch_swiglu(const float *gate, const float *up, size_t n, float *out,
                         hipStream_t s) {
    if (!n) return MRI_OK;
    hipLaunchKernelGGL(k_swiglu, dim3(grid_for(n)), dim3(256), 0, s, gate, up, n, out);
    MRI_LAUNCHED("k_swiglu");
    return MRI_OK;
}

mri_status launch_add(const float *a, const float *b, size_t n, float *out, hipStream_t s) {
    if (!n) return MRI_OK;
    hipLaunchKernelGGL(k_add, dim3(grid_for(n)), dim3(256), 0, s, a, b, n, out);
    MRI_LAUNCHED("k_add");
    return MRI_OK;
}

mri_status launch_argmax(const float *v, size_t rows, size_t n, uint32_t *idx, hipStream_t s) {
    if (!rows) return MRI_OK;
    hipLaunchKernelGGL(k_argmax, dim3((unsigned)rows), dim3(1024), 0, s, v, (int)n, idx);
    MRI_LAUNCHED("k_argmax");
    return MRI_OK;
}

}  // namespace mri
