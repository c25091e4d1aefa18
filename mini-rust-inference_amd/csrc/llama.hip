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
#include <type_traits>

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
// x[r, :] = table[tokens[r], :], 1024 floats per workgroup.  Token ids are
// checked against the vocabulary on the host, or come from the argmax
// kernel (always < vocab).  d % 4 == 0 (the float4 path) or any d.
template <bool V4>
__global__ __launch_bounds__(256) void k_embed(const float *__restrict__ table,
                                               const uint32_t *__restrict__ tokens, int d,
                                               float *__restrict__ x) {
    const size_t src = (size_t)tokens[blockIdx.x] * d, dst = (size_t)blockIdx.x * d;
    const int i = (blockIdx.y * 256 + threadIdx.x) * 4;
    if constexpr (V4) {
        if (i < d)
            *reinterpret_cast<float4 *>(x + dst + i) =
                *reinterpret_cast<const float4 *>(table + src + i);
    } else {
        for (int e = i; e < min(i + 4, d); ++e) x[dst + e] = table[src + e];
    }
}

// ---- RMSNorm (ops/norm/rmsnorm.rs) ------------------------------------------------
// One workgroup per row: mean_sq = sum(x*x) / d, rms_inv = 1 / sqrt(mean_sq +
// eps) (correctly rounded divide and sqrt), out = w * (x * rms_inv).  NV > 0:
// the row is read once into registers, NV float4 per thread (d % 4 == 0,
// d <= 1024 * NV); NV == 0: any d, two passes.
// MODE 1 (NV > 0): the row is first gathered from an embedding table,
// table[tokens[row]], and also stored to x_out (embed + the first norm).
// MODE 2 (NV > 0): the row is first x + delta (the residual add,
// forward_int8.rs:100-121), stored back to x_out (= x) before the norm.
// STATS (NV > 0): instead of the normalized row, out[2*row] = rms_inv and
// out[2*row + 1] = max |w * (x * rms_inv)| over the row (the values the
// quantizer that consumes the row needs; k_norm_quant recomputes the row
// from x with the same operations, so the normalized rows never go to
// memory).
template <int NV, int MODE = 0, bool STATS = false>
// (x and x_out are the same buffer in MODE 2: neither is restrict.)
__global__ __launch_bounds__(256) void k_rmsnorm(const float *x, const float *__restrict__ w,
                                                 int d, float eps, float *__restrict__ out,
                                                 const uint32_t *__restrict__ tokens = nullptr,
                                                 const float *__restrict__ delta = nullptr,
                                                 float *x_out = nullptr) {
    static_assert(!STATS || NV > 0, "row statistics need the register-resident row");
    __shared__ float s_part[4];
    __shared__ float s_max[4];
    const float *xr = MODE == 1 ? x + (size_t)tokens[blockIdx.x] * d : x + (size_t)blockIdx.x * d;
    float *orow = out + (size_t)blockIdx.x * d;
    float acc = 0.0f;
    float4 xv[NV > 0 ? NV : 1];
    if constexpr (NV > 0) {
#pragma unroll
        for (int c = 0; c < NV; ++c) {
            const int i = (c * 256 + threadIdx.x) * 4;
            xv[c] = i < d ? *reinterpret_cast<const float4 *>(xr + i) : float4{0, 0, 0, 0};
        }
        if constexpr (MODE == 2) {
#pragma unroll
            for (int c = 0; c < NV; ++c) {
                const int i = (c * 256 + threadIdx.x) * 4;
                if (i < d) {
                    const float4 dv =
                        *reinterpret_cast<const float4 *>(delta + (size_t)blockIdx.x * d + i);
                    xv[c] = float4{xv[c].x + dv.x, xv[c].y + dv.y, xv[c].z + dv.z, xv[c].w + dv.w};
                }
            }
        }
        if constexpr (MODE != 0) {
#pragma unroll
            for (int c = 0; c < NV; ++c) {
                const int i = (c * 256 + threadIdx.x) * 4;
                if (i < d) *reinterpret_cast<float4 *>(x_out + (size_t)blockIdx.x * d + i) = xv[c];
            }
        }
#pragma unroll
        for (int c = 0; c < NV; ++c) {
            float sq = xv[c].x * xv[c].x;
            acc = acc + sq;
            sq = xv[c].y * xv[c].y;
            acc = acc + sq;
            sq = xv[c].z * xv[c].z;
            acc = acc + sq;
            sq = xv[c].w * xv[c].w;
            acc = acc + sq;
        }
    } else {
        for (int i = threadIdx.x; i < d; i += 256) {
            const float sq = xr[i] * xr[i];
            acc = acc + sq;
        }
    }
    acc = wave_sum(acc);
    if ((threadIdx.x & 63) == 0) s_part[threadIdx.x >> 6] = acc;
    __syncthreads();
    const float sum = ((s_part[0] + s_part[1]) + s_part[2]) + s_part[3];
    const float mean_sq = sum / (float)d;
    const float rms_inv = 1.0f / sqrtf(mean_sq + eps);
    if constexpr (STATS) {
        float mx = 0.0f;
#pragma unroll
        for (int c = 0; c < NV; ++c) {
            const int i = (c * 256 + threadIdx.x) * 4;
            if (i < d) {
                const float4 wv = *reinterpret_cast<const float4 *>(w + i);
                mx = fmaxf(mx, fabsf(wv.x * (xv[c].x * rms_inv)));
                mx = fmaxf(mx, fabsf(wv.y * (xv[c].y * rms_inv)));
                mx = fmaxf(mx, fabsf(wv.z * (xv[c].z * rms_inv)));
                mx = fmaxf(mx, fabsf(wv.w * (xv[c].w * rms_inv)));
            }
        }
        mx = wave_max(mx);
        if ((threadIdx.x & 63) == 0) s_max[threadIdx.x >> 6] = mx;
        __syncthreads();
        if (threadIdx.x == 0) {
            out[2 * (size_t)blockIdx.x] = rms_inv;
            out[2 * (size_t)blockIdx.x + 1] = fmaxf(fmaxf(s_max[0], s_max[1]), fmaxf(s_max[2], s_max[3]));
        }
    } else if constexpr (NV > 0) {
#pragma unroll
        for (int c = 0; c < NV; ++c) {
            const int i = (c * 256 + threadIdx.x) * 4;
            if (i < d) {
                const float4 wv = *reinterpret_cast<const float4 *>(w + i);
                float4 o;
                o.x = wv.x * (xv[c].x * rms_inv);
                o.y = wv.y * (xv[c].y * rms_inv);
                o.z = wv.z * (xv[c].z * rms_inv);
                o.w = wv.w * (xv[c].w * rms_inv);
                *reinterpret_cast<float4 *>(orow + i) = o;
            }
        }
    } else {
        for (int i = threadIdx.x; i < d; i += 256) {
            const float t = xr[i] * rms_inv;
            orow[i] = w[i] * t;
        }
    }
}

// ---- RoPE + KV-cache write (ops/rope.rs, attention/cached.rs) --------------------------
// Row s of q (n_heads heads) and k (n_kv heads) is rotated with table row
// start_pos + s: pair (2i, 2i+1) -> (x0*c - x1*s, x1*c + x0*s).  q is
// rotated in place; the rotated k row and the v row are written to the
// cache at position start_pos + s (write_k / write_v).  Workgroup (s, y):
// one head of row s, y < n_heads a q head, then the k heads, then the v
// heads; thread i owns pair i (half = head_dim / 2 <= 64 threads).
__global__ __launch_bounds__(64) void k_rope_qkv(float *__restrict__ q,
                                                 const float *__restrict__ k,
                                                 const float *__restrict__ v, int qs, int kvs,
                                                 int kvd, int half, int n_heads, int n_kv,
                                                 const float *__restrict__ cos_t,
                                                 const float *__restrict__ sin_t, int start_pos,
                                                 float *__restrict__ kc,
                                                 float *__restrict__ vc) {
    const int s = blockIdx.x, pos = start_pos + s, y = blockIdx.y, i = threadIdx.x;
    if (i >= half) return;
    const int hd = 2 * half;
    if (y >= n_heads + n_kv) {  // v head: copy
        const int off = (y - n_heads - n_kv) * hd + 2 * i;
        const float2 vv = *reinterpret_cast<const float2 *>(v + (size_t)s * kvs + off);
        *reinterpret_cast<float2 *>(vc + (size_t)pos * kvd + off) = vv;
        return;
    }
    const float c = cos_t[(size_t)pos * half + i], sn = sin_t[(size_t)pos * half + i];
    const float *src;
    float *dst;
    if (y < n_heads) {
        src = dst = q + (size_t)s * qs + y * hd + 2 * i;
    } else {
        src = k + (size_t)s * kvs + (y - n_heads) * hd + 2 * i;
        dst = kc + (size_t)pos * kvd + (y - n_heads) * hd + 2 * i;
    }
    const float2 xv = *reinterpret_cast<const float2 *>(src);
    const float a0 = xv.x * c, a1 = xv.y * sn, b0 = xv.y * c, b1 = xv.x * sn;
    *reinterpret_cast<float2 *>(dst) = float2{a0 - a1, b0 + b1};
}

// ---- causal grouped-query attention (attention/gqa.rs:217-240) --------------------------
// Prefill form.  Workgroup (query block, head h): QB query rows i (absolute
// positions start_pos + i) against the keys 0 .. L-1 of kv head
// h / groups in the cache, L = start_pos + the block's last row + 1.  The
// reference's three passes:
//  1. scores, one 64-key tile at a time: the tile is loaded by the whole
//     workgroup at once (one load latency per tile) and stored transposed,
//     kT[p][key] with a row pitch of 65 floats, so that lane `key` reading
//     kT[p][key] and the loading lanes writing it hit distinct banks.  Lane
//     `key` of wave w computes the dot products of its key with queries w,
//     w + 4, ... sequentially over the head dimension (matmul_naive's order),
//     times 1/sqrt(head_dim); keys past a row's position get -inf.
//  2. softmax per row: max, exp(s - max), sum, times 1/sum.
//  3. values, one 64-key tile at a time (row-major in LDS): lane l of wave w
//     owns dims HD/64 * l .. of queries w, w + 4, ... and sums the keys in
//     order, as the reference.
// LDS: queries [QB][HD], one tile [max(HD*65, 64*HD)], weights [QB][lcap].
template <int HD>
constexpr int attn_tile_floats() { return HD * 65 > 64 * HD ? HD * 65 : 64 * HD; }

template <int HD, int QB>
__global__ __launch_bounds__(256) void k_attention(
    const float *__restrict__ q, int qs, int qd, const float *__restrict__ kc,
    const float *__restrict__ vc, int kvd, int seq_q, int start_pos, int groups, int lcap,
    float scale, float *__restrict__ out) {
    constexpr int E = HD / kWave;  // dims per lane in the value pass
    constexpr int R = QB / 4;      // queries per wave
    constexpr int KT = 64;         // keys per tile
    constexpr int P4 = HD / 4;     // float4 per key row
    static_assert(QB % 4 == 0, "query block");
    extern __shared__ __attribute__((aligned(16))) float s_mem[];  // read and written as float4
    float *s_q = s_mem;                          // [QB][HD]
    float *s_t = s_q + QB * HD;                  // tile
    float *s_p = s_t + attn_tile_floats<HD>();   // [QB][lcap]
    const int t = threadIdx.x, lane = t & 63, wv = t >> 6;
    const int h = blockIdx.y, kh = h / groups;
    const int i0 = blockIdx.x * QB;
    const int nq = min(QB, seq_q - i0);
    const int L = start_pos + i0 + nq;  // keys the block's last row sees
    for (int e = t; e < QB * HD; e += 256) {
        const int qq = e / HD, p = e % HD;
        s_q[e] = qq < nq ? q[(size_t)(i0 + qq) * qs + h * HD + p] : 0.0f;
    }
    // 1. scores
    for (int j0 = 0; j0 < L; j0 += KT) {
        __syncthreads();  // the previous tile is consumed (and s_q written)
#pragma unroll
        for (int u = 0; u < KT * P4 / 256; ++u) {
            const int idx = t + 256 * u, key = idx / P4, p4 = idx % P4;
            float4 kv = float4{0, 0, 0, 0};
            if (j0 + key < L)
                kv = *reinterpret_cast<const float4 *>(kc + (size_t)(j0 + key) * kvd + kh * HD +
                                                       4 * p4);
            s_t[(4 * p4 + 0) * 65 + key] = kv.x;
            s_t[(4 * p4 + 1) * 65 + key] = kv.y;
            s_t[(4 * p4 + 2) * 65 + key] = kv.z;
            s_t[(4 * p4 + 3) * 65 + key] = kv.w;
        }
        __syncthreads();
        float acc[R];
#pragma unroll
        for (int r = 0; r < R; ++r) acc[r] = 0.0f;
        for (int p4 = 0; p4 < P4; ++p4) {
            float kk[4];
#pragma unroll
            for (int c = 0; c < 4; ++c) kk[c] = s_t[(4 * p4 + c) * 65 + lane];
#pragma unroll
            for (int r = 0; r < R; ++r) {
                const float4 qv = reinterpret_cast<const float4 *>(s_q + (wv + 4 * r) * HD)[p4];
                float m0 = qv.x * kk[0];
                acc[r] = acc[r] + m0;
                m0 = qv.y * kk[1];
                acc[r] = acc[r] + m0;
                m0 = qv.z * kk[2];
                acc[r] = acc[r] + m0;
                m0 = qv.w * kk[3];
                acc[r] = acc[r] + m0;
            }
        }
        const int j = j0 + lane;
        if (j < L) {
#pragma unroll
            for (int r = 0; r < R; ++r) {
                const int qq = wv + 4 * r;
                const float sc = acc[r] * scale;
                s_p[qq * lcap + j] = j <= start_pos + i0 + qq ? sc + 0.0f : -INFINITY;
            }
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
    // 3. weighted values
    float o[R][E];
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
        for (int e = 0; e < E; ++e) o[r][e] = 0.0f;
    for (int j0 = 0; j0 < L; j0 += KT) {
        __syncthreads();  // softmax done / the previous tile consumed
#pragma unroll
        for (int u = 0; u < KT * P4 / 256; ++u) {
            const int idx = t + 256 * u, key = idx / P4, p4 = idx % P4;
            float4 vv = float4{0, 0, 0, 0};
            if (j0 + key < L)
                vv = *reinterpret_cast<const float4 *>(vc + (size_t)(j0 + key) * kvd + kh * HD +
                                                       4 * p4);
            reinterpret_cast<float4 *>(s_t)[idx] = vv;  // [key][HD]
        }
        __syncthreads();
        const int jn = min(KT, L - j0);
        for (int j = 0; j < jn; ++j) {
            float vv[E];
#pragma unroll
            for (int e = 0; e < E; ++e) vv[e] = s_t[j * HD + lane * E + e];
#pragma unroll
            for (int r = 0; r < R; ++r) {
                const float w = s_p[(wv + 4 * r) * lcap + j0 + j];
#pragma unroll
                for (int e = 0; e < E; ++e) {
                    const float m0 = w * vv[e];
                    o[r][e] = o[r][e] + m0;
                }
            }
        }
    }
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const int qq = wv + 4 * r;
        if (qq < nq)
#pragma unroll
            for (int e = 0; e < E; ++e) out[(size_t)(i0 + qq) * qd + h * HD + lane * E + e] = o[r][e];
    }
}

// Decode form (one query row), split over the keys.  Workgroup (chunk c,
// head h) takes keys [CK c, CK c + CK) of the L = start_pos + 1 visible ones,
// CK = 16 NW, 16 per wave (NW = 8: 128 keys; in the 7B layer's decode step
// at 512-640 keys, 64-key chunks of four waves took 0.2-0.7 us a token
// longer, twice as many chunks to publish and combine, and 256-key chunks
// of 16 waves 1.3-2.4 us longer).  Each load instruction
// of a wave reads whole key (and value) rows, HD/4 lanes of 16 bytes per
// row, so a chunk arrives as contiguous 512-byte rows (with one lane per
// key, each instruction read 16
// bytes of 64 different rows: 10.0 against 9.3 us a call at 512-640 keys,
// 32 heads of 128); all of a thread's key and value loads are issued before
// the first use.  The rest of a call is its tail: the partial stores, the
// count and the combine, three memory round trips in sequence.  A key's dot is four products per
// lane, then the HD/4 lanes added by a butterfly; then the chunk's max m_c,
// weights e_j = exp(s_j - m_c) and their sum l_c (every wave computes them
// from the CK scores in LDS, CK / 64 a lane), and the chunk's weighted
// value sum o_c (per lane in key order, then the lane groups and the NW
// waves added in order).  The chunk's (m_c, l_c, o_c) go to part ([heads][chunks][HD+2])
// through device-scope (sc1) stores, complete before the workgroup counts
// itself on its head's counter (relaxed, device scope); the workgroup that
// counts last for a head combines the chunks (attn_combine) and resets the
// counter, so no workgroup waits for another and no second launch is needed.
// The partials reach the point of coherence of all XCDs before the count
// (vmcnt(0) and a barrier), and the combining workgroup reads them with sc1
// loads, which do not hit lines its XCD's L2 cached before.  (A release /
// acquire count at device scope writes back and invalidates the XCD's L2 in
// every workgroup: 14.4 against 10.5 us a call at 512-575 keys.)
// cnt: one word per head, zero between calls.
__device__ inline float attn_part_load(const float *p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// Output element d of a head from its nch chunk partials at ph: m = max_c m_c,
// then l = sum_c l_c exp(m_c - m) and o = sum_c o_c[d] exp(m_c - m) in chunk
// order, out[d] = o / l.  The first 16 chunks' (m_c, l_c, o_c[d]) are loaded
// together, before the first use, so the combine costs one memory round trip
// up to 16 chunks (1024 keys).
template <int HD>
__device__ inline void attn_combine(const float *ph, int nch, int d, float *out) {
    if (d >= HD) return;
    constexpr int B = 16;
    float mv[B], lv[B], ov[B];
    auto batch = [&](int c0) __attribute__((always_inline)) {
#pragma unroll
        for (int u = 0; u < B; ++u) {
            const float *pc = ph + (size_t)min(c0 + u, nch - 1) * (HD + 2);
            mv[u] = attn_part_load(pc);
            lv[u] = attn_part_load(pc + 1);
            ov[u] = attn_part_load(pc + 2 + d);
        }
    };
    batch(0);
    float m = -INFINITY;
#pragma unroll
    for (int u = 0; u < B; ++u)
        if (u < nch) m = fmaxf(m, mv[u]);
    for (int c = B; c < nch; ++c) m = fmaxf(m, attn_part_load(ph + (size_t)c * (HD + 2)));
    float l = 0.0f, o = 0.0f;
    for (int c0 = 0; c0 < nch; c0 += B) {
        if (c0 > 0) batch(c0);
#pragma unroll
        for (int u = 0; u < B; ++u) {
            if (c0 + u < nch) {
                const float f = expf(mv[u] - m);
                l = l + lv[u] * f;
                o = o + ov[u] * f;
            }
        }
    }
    out[d] = o / l;
}

template <int HD, int NW>
__global__ __launch_bounds__(NW * 64) void k_attn_decode_part(
    const float *__restrict__ q, const float *__restrict__ kc, const float *__restrict__ vc,
    int kvd, int L, int groups, float scale, float *__restrict__ part, int *__restrict__ cnt,
    float *__restrict__ out) {
    // A key (or value) row is R4 float4; one wave load instruction covers
    // KPI whole rows (R4 lanes each), so every load is KPI contiguous rows.
    // Wave wv holds keys 16 wv .. 16 wv + 15 of the chunk: key 16 wv + KPI i
    // + sub in load i, lane (sub, d4) with float4 d4 of the row.
    constexpr int R4 = HD / 4, KPI = kWave / R4, NI = 16 / KPI;
    constexpr int CK = 16 * NW, NS = CK / kWave;  // keys of a chunk, scores a lane
    static_assert(HD % 64 == 0 && HD <= 256 && NW % 4 == 0, "head dim, waves");
    __shared__ float s_s[CK];
    __shared__ __attribute__((aligned(16))) float s_o[NW][HD];  // written as float4
    __shared__ int s_last;
    const int t = threadIdx.x, lane = t & 63, wv = t >> 6;
    const int sub = lane / R4, d4 = lane % R4;
    const int c = blockIdx.x, h = blockIdx.y, kh = h / groups, nch = gridDim.x;
    const int j0 = CK * c + 16 * wv + sub;
    float4 kr[NI], vr[NI];
#pragma unroll
    for (int i = 0; i < NI; ++i) {
        const int j = j0 + KPI * i;
        const size_t off = (size_t)j * kvd + kh * HD;
        kr[i] = j < L ? reinterpret_cast<const float4 *>(kc + off)[d4] : float4{0, 0, 0, 0};
        vr[i] = j < L ? reinterpret_cast<const float4 *>(vc + off)[d4] : float4{0, 0, 0, 0};
    }
    const float4 qv = reinterpret_cast<const float4 *>(q + (size_t)h * HD)[d4];
    // dots: four products per lane in dim order, then the R4 lanes of a key
    // added by a butterfly
    float sc[NI];
#pragma unroll
    for (int i = 0; i < NI; ++i) {
        float a = qv.x * kr[i].x;
        float m0 = qv.y * kr[i].y;
        a = a + m0;
        m0 = qv.z * kr[i].z;
        a = a + m0;
        m0 = qv.w * kr[i].w;
        sc[i] = a + m0;
    }
#pragma unroll
    for (int o = R4 / 2; o > 0; o >>= 1)
#pragma unroll
        for (int i = 0; i < NI; ++i) sc[i] = sc[i] + __shfl_xor(sc[i], o, kWave);
    if (d4 == 0) {
#pragma unroll
        for (int i = 0; i < NI; ++i) {
            const int j = j0 + KPI * i;
            s_s[j - CK * c] = j < L ? sc[i] * scale : -INFINITY;
        }
    }
    __syncthreads();
    // every wave: the chunk's max m_c, weights e_j = exp(s_j - m_c), sum l_c
    // (lane l holds keys l, l + 64, ..)
    float sv[NS], e[NS];
    float mm = -INFINITY;
#pragma unroll
    for (int u = 0; u < NS; ++u) {
        sv[u] = s_s[lane + kWave * u];
        mm = fmaxf(mm, sv[u]);
    }
    const float m = wave_max(mm);
    float es = 0.0f;
#pragma unroll
    for (int u = 0; u < NS; ++u) {
        e[u] = CK * c + kWave * u + lane < L ? expf(sv[u] - m) : 0.0f;
        es = es + e[u];
    }
    const float lsum = wave_sum(es);
    float *pc = part + ((size_t)h * nch + c) * (HD + 2);
    if (t == 0) {
        __hip_atomic_store(pc, m, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_store(pc + 1, lsum, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    // weighted values of this wave's keys, in key order per lane; the KPI
    // lane groups, then the NW waves, added in order
    float4 o = float4{0, 0, 0, 0};
#pragma unroll
    for (int i = 0; i < NI; ++i) {
        const int kx = 16 * wv + KPI * i + sub;  // key of the chunk
        float w = __shfl(e[0], kx % kWave, kWave);
#pragma unroll
        for (int u = 1; u < NS; ++u) {
            const float wu = __shfl(e[u], kx % kWave, kWave);
            w = kx / kWave == u ? wu : w;
        }
        float m0 = w * vr[i].x;
        o.x = o.x + m0;
        m0 = w * vr[i].y;
        o.y = o.y + m0;
        m0 = w * vr[i].z;
        o.z = o.z + m0;
        m0 = w * vr[i].w;
        o.w = o.w + m0;
    }
#pragma unroll
    for (int g = 1; g < KPI; g <<= 1) {
        o.x = o.x + __shfl_xor(o.x, g * R4, kWave);
        o.y = o.y + __shfl_xor(o.y, g * R4, kWave);
        o.z = o.z + __shfl_xor(o.z, g * R4, kWave);
        o.w = o.w + __shfl_xor(o.w, g * R4, kWave);
    }
    if (sub == 0) reinterpret_cast<float4 *>(s_o[wv])[d4] = o;
    __syncthreads();
    for (int d = t; d < HD; d += NW * kWave) {
        float a = s_o[0][d];
#pragma unroll
        for (int u = 1; u < NW; ++u) a = a + s_o[u][d];
        __hip_atomic_store(pc + 2 + d, a, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): this thread's partials are at the device
    __syncthreads();
    if (t == 0)
        s_last = __hip_atomic_fetch_add(&cnt[h], 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
                 nch - 1;
    __syncthreads();
    if (!s_last) return;
    attn_combine<HD>(part + (size_t)h * nch * (HD + 2), nch, t, out + (size_t)h * HD);
    if (t == 0) __hip_atomic_store(&cnt[h], 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Decode form with one workgroup per head, for contexts up to
// kDecHeadMaxL keys: no partials leave the workgroup, so the partial
// stores, counter and combine of the split form are gone (5.7 against
// 7.1 us at contexts of 9-72 keys, 32 heads of 128).  A head's keys then
// stream through one CU, which at 512-575 keys is slower than the split
// form (11.6 against 10.3 us), so longer contexts split.  The 8 waves
// hold 32 groups of 16 lanes; in step s group G takes keys 128 s + 4 G ..
// + 3, each lane 8 dims of each (float4 loads, 512 contiguous bytes per key
// row).  A group keeps its own online softmax over its keys (max m, sum l,
// output o; four keys per update), and the 32 group states are combined
// through LDS at the end.  The next step's rows, if any, are loaded while
// the current step is computed.  Differs from the reference's sequential
// sums only in f32 rounding.
constexpr int kDecHeadMaxL = 128;
template <int HD>
__global__ __launch_bounds__(512) void k_attn_decode_head(
    const float *__restrict__ q, const float *__restrict__ kc, const float *__restrict__ vc,
    int kvd, int L, int groups, float scale, float *__restrict__ out) {
    constexpr int DPL = HD / 16;  // dims per lane
    constexpr int V4 = DPL / 4;   // float4 per lane and key row
    constexpr int KPG = 4;        // keys per group and step
    constexpr int NG = 32;        // groups
    constexpr int KPS = NG * KPG; // keys per step
    static_assert(HD % 64 == 0 && HD <= 256, "16 lanes of float4 per key row");
    __shared__ float s_m[NG], s_l[NG];
    __shared__ float s_o[NG][HD + 4];
    const int t = threadIdx.x, l = t & 63, li = l & 15;
    const int grp = (t >> 6) * 4 + (l >> 4);
    const int h = blockIdx.x, kh = h / groups;
    float4 qv[V4];
#pragma unroll
    for (int v = 0; v < V4; ++v)
        qv[v] = reinterpret_cast<const float4 *>(q + (size_t)h * HD + li * DPL)[v];
    const float *kb = kc + (size_t)kh * HD + li * DPL, *vb = vc + (size_t)kh * HD + li * DPL;
    const int nsteps = (L + KPS - 1) / KPS;
    float4 kr[2][KPG][V4], vr[2][KPG][V4];
    auto load = [&](auto buf, int st) __attribute__((always_inline)) {
        constexpr int B = decltype(buf)::value;
#pragma unroll
        for (int k = 0; k < KPG; ++k) {
            const size_t j = (size_t)min(st * KPS + grp * KPG + k, L - 1);
#pragma unroll
            for (int v = 0; v < V4; ++v) {
                kr[B][k][v] = reinterpret_cast<const float4 *>(kb + j * kvd)[v];
                vr[B][k][v] = reinterpret_cast<const float4 *>(vb + j * kvd)[v];
            }
        }
    };
    float m = -INFINITY, lsum = 0.0f, o[DPL];
#pragma unroll
    for (int d = 0; d < DPL; ++d) o[d] = 0.0f;
    auto step = [&](auto cur, int st) __attribute__((always_inline)) {
        constexpr int C = decltype(cur)::value;
        if (st + 1 < nsteps) load(std::integral_constant<int, 1 - C>{}, st + 1);
        float sc[KPG];
#pragma unroll
        for (int k = 0; k < KPG; ++k) {
            float d = 0.0f;
#pragma unroll
            for (int v = 0; v < V4; ++v) {
                d = d + qv[v].x * kr[C][k][v].x;
                d = d + qv[v].y * kr[C][k][v].y;
                d = d + qv[v].z * kr[C][k][v].z;
                d = d + qv[v].w * kr[C][k][v].w;
            }
#pragma unroll
            for (int x = 8; x > 0; x >>= 1) d = d + __shfl_xor(d, x);
            sc[k] = st * KPS + grp * KPG + k < L ? d * scale : -INFINITY;
        }
        const float m_new = fmaxf(fmaxf(m, fmaxf(sc[0], sc[1])), fmaxf(sc[2], sc[3]));
        const float m_use = m_new == -INFINITY ? 0.0f : m_new;  // then every score is -inf
        const float alpha = expf(m - m_use);
        float p[KPG];
#pragma unroll
        for (int k = 0; k < KPG; ++k) p[k] = expf(sc[k] - m_use);
        lsum = lsum * alpha + ((p[0] + p[1]) + (p[2] + p[3]));
#pragma unroll
        for (int v = 0; v < V4; ++v) {
            float4 a = {o[4 * v] * alpha, o[4 * v + 1] * alpha, o[4 * v + 2] * alpha,
                        o[4 * v + 3] * alpha};
#pragma unroll
            for (int k = 0; k < KPG; ++k) {
                a.x = a.x + p[k] * vr[C][k][v].x;
                a.y = a.y + p[k] * vr[C][k][v].y;
                a.z = a.z + p[k] * vr[C][k][v].z;
                a.w = a.w + p[k] * vr[C][k][v].w;
            }
            o[4 * v] = a.x;
            o[4 * v + 1] = a.y;
            o[4 * v + 2] = a.z;
            o[4 * v + 3] = a.w;
        }
        m = m_new;
    };
    using I0 = std::integral_constant<int, 0>;
    using I1 = std::integral_constant<int, 1>;
    load(I0{}, 0);
    int st = 0;
    for (; st + 1 < nsteps; st += 2) {
        step(I0{}, st);
        step(I1{}, st + 1);
    }
    if (st < nsteps) step(I0{}, st);
    // combine the groups: out = sum_G c_G o_G / sum_G c_G l_G, c_G = e^(m_G - max m)
    // (a group that saw no key has m = -inf, l = 0, o = 0; key 0 is always seen)
    if (li == 0) {
        s_m[grp] = m;
        s_l[grp] = lsum;
    }
#pragma unroll
    for (int d = 0; d < DPL; ++d) s_o[grp][li * DPL + d] = o[d];
    __syncthreads();
    if (t >= HD) return;
    float M = -INFINITY;
    for (int G = 0; G < NG; ++G) M = fmaxf(M, s_m[G]);
    float den = 0.0f, num = 0.0f;
    for (int G = 0; G < NG; ++G) {
        const float c = expf(s_m[G] - M);
        den = den + c * s_l[G];
        num = num + c * s_o[G][t];
    }
    out[(size_t)h * HD + t] = num / den;
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
// The same, 4 elements per thread (n % 4 == 0, 16-byte aligned rows).
__global__ __launch_bounds__(256) void k_swiglu4(const float4 *__restrict__ gate,
                                                 const float4 *__restrict__ up, size_t n4,
                                                 float4 *__restrict__ out) {
    for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n4; i += (size_t)gridDim.x * 256) {
        const float4 g = gate[i], u = up[i];
        float4 o;
        o.x = g.x / (1.0f + expf(-g.x)) * u.x;
        o.y = g.y / (1.0f + expf(-g.y)) * u.y;
        o.z = g.z / (1.0f + expf(-g.z)) * u.z;
        o.w = g.w / (1.0f + expf(-g.w)) * u.w;
        out[i] = o;
    }
}

// Rows of [gate | up] (the fused gate/up projection, 2*ffn floats a row)
// into rows of ffn: the same function, 4 elements per thread (ffn % 4 == 0).
__global__ __launch_bounds__(256) void k_swiglu_rows4(const float4 *__restrict__ gu, int ffn4,
                                                      size_t n4, float4 *__restrict__ out) {
    for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n4; i += (size_t)gridDim.x * 256) {
        const size_t r = i / ffn4, j = i - r * ffn4;
        const float4 g = gu[r * 2 * ffn4 + j], u = gu[r * 2 * ffn4 + ffn4 + j];
        float4 o;
        o.x = g.x / (1.0f + expf(-g.x)) * u.x;
        o.y = g.y / (1.0f + expf(-g.y)) * u.y;
        o.z = g.z / (1.0f + expf(-g.z)) * u.z;
        o.w = g.w / (1.0f + expf(-g.w)) * u.w;
        out[i] = o;
    }
}

// ---- residual add (forward_int8.rs:100-121): out = a + b -------------------------------
__global__ __launch_bounds__(256) void k_add(const float *__restrict__ a,
                                             const float *__restrict__ b, size_t n,
                                             float *__restrict__ out) {
    for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (size_t)gridDim.x * 256)
        out[i] = a[i] + b[i];
}
__global__ __launch_bounds__(256) void k_add4(const float4 *__restrict__ a,
                                              const float4 *__restrict__ b, size_t n4,
                                              float4 *__restrict__ out) {
    for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n4; i += (size_t)gridDim.x * 256) {
        const float4 x = a[i], y = b[i];
        out[i] = float4{x.x + y.x, x.y + y.y, x.z + y.z, x.w + y.w};
    }
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
    // 32 loads in flight per thread (one pass up to 32768 values); within a
    // thread indices only grow, so ">=" keeps the last of equal values
    for (int i0 = threadIdx.x; i0 < n; i0 += 32 * 1024) {
        float xs[32];
#pragma unroll
        for (int u = 0; u < 32; ++u) xs[u] = row[min(i0 + u * 1024, n - 1)];
#pragma unroll
        for (int u = 0; u < 32; ++u) {
            const int i = i0 + u * 1024;
            const float x = xs[u];
            if (i < n && !(x != x) && (bi < 0 || x >= bv)) {
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

// (value, index) order of the argmax: a larger value, then a larger index
// (the last of equal values); oi < 0 is no candidate.
__device__ inline bool arg_better(float ov, int oi, float bv, int bi) {
    return oi >= 0 && (bi < 0 || ov > bv || (ov == bv && oi > bi));
}

// The second half of the fused greedy argmax: the largest of n keys
// (argmax_key, one per 16-channel tile of the output projection) in one
// workgroup; writes its index (0 when every key is 0, i.e. every value
// NaN) and, with table, copies that row of table to x_out.
__global__ __launch_bounds__(256) void k_argmax_keys(const unsigned long long *__restrict__ keys,
                                                     int n, uint32_t *__restrict__ idx,
                                                     const float *__restrict__ table, int d,
                                                     float *__restrict__ x_out) {
    __shared__ unsigned long long s_k[4];
    unsigned long long k = 0;
    for (int i = threadIdx.x; i < n; i += 256) k = keys[i] > k ? keys[i] : k;
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        const unsigned lo = __shfl_xor((unsigned)k, o), hi = __shfl_xor((unsigned)(k >> 32), o);
        const unsigned long long ok = ((unsigned long long)hi << 32) | lo;
        k = ok > k ? ok : k;
    }
    if ((threadIdx.x & 63) == 0) s_k[threadIdx.x >> 6] = k;
    __syncthreads();
    k = s_k[0];
#pragma unroll
    for (int w = 1; w < 4; ++w) k = s_k[w] > k ? s_k[w] : k;
    const uint32_t id = k ? (uint32_t)k : 0u;
    if (threadIdx.x == 0) idx[0] = id;
    if (!table) return;
    const float4 *src = reinterpret_cast<const float4 *>(table + (size_t)id * d);
    for (int i = threadIdx.x; i < d / 4; i += 256) reinterpret_cast<float4 *>(x_out)[i] = src[i];
}

// One row split over the blocks: block b reduces its slice, stores its
// (value, index) and counts itself; the block that counts last combines
// the gridDim.x <= 64 candidates, writes idx[0], resets the counter, and
// with table copies row idx of table ([*][d] f32) to x_out.  ws: the
// counter at word 0, candidate values at words 4.., indices at 68...
// The candidates are stored and loaded with device-scope (sc1) accesses,
// which reach the point of coherence of all XCDs, and each block waits for
// its stores to complete before it counts.  The count is an acquire-release
// read-modify-write at agent (device) scope, which covers every XCD of the
// device, so the candidates happen-before the last block's reads in the
// memory model too.
constexpr int kArgSplit = 64;
__global__ __launch_bounds__(256) void k_argmax_split(const float *__restrict__ v, int n,
                                                      uint32_t *__restrict__ idx,
                                                      const float *__restrict__ table, int d,
                                                      float *__restrict__ x_out,
                                                      unsigned *__restrict__ ws) {
    __shared__ float s_v[4];
    __shared__ int s_i[4];
    __shared__ int s_last, s_tok;
    unsigned *count = ws;
    int *part_v = reinterpret_cast<int *>(ws + 4);
    int *part_i = reinterpret_cast<int *>(ws + 4 + kArgSplit);
    const int per = (n + (int)gridDim.x - 1) / (int)gridDim.x;
    const int lo = (int)blockIdx.x * per, hi = min(n, lo + per);
    float bv = -INFINITY;
    int bi = -1;
    // four loads in flight per thread; within a thread indices only grow,
    // so ">=" keeps the last of equal values
    for (int i0 = lo + (int)threadIdx.x; i0 < hi; i0 += 4 * 256) {
        float xs[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) xs[u] = v[min(i0 + u * 256, hi - 1)];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const int i = i0 + u * 256;
            const float x = xs[u];
            if (i < hi && !(x != x) && (bi < 0 || x >= bv)) {
                bv = x;
                bi = i;
            }
        }
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        const float ov = __shfl_xor(bv, o, kWave);
        const int oi = __shfl_xor(bi, o, kWave);
        if (arg_better(ov, oi, bv, bi)) {
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
        for (int w = 1; w < 4; ++w)
            if (arg_better(s_v[w], s_i[w], bv, bi)) {
                bv = s_v[w];
                bi = s_i[w];
            }
        __hip_atomic_store(&part_v[blockIdx.x], __float_as_int(bv), __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_store(&part_i[blockIdx.x], bi, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        // release: publishes this block's candidate; acquire: the last block
        // reads every candidate after it (device scope: all XCDs)
        s_last = __hip_atomic_fetch_add(count, 1u, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT) ==
                 gridDim.x - 1;
    }
    __syncthreads();
    if (!s_last) return;
    if (threadIdx.x < 64) {
        const int b = threadIdx.x;
        float cv = -INFINITY;
        int ci = -1;
        if (b < (int)gridDim.x) {
            cv = __int_as_float(
                __hip_atomic_load(&part_v[b], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
            ci = __hip_atomic_load(&part_i[b], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) {
            const float ov = __shfl_xor(cv, o, kWave);
            const int oi = __shfl_xor(ci, o, kWave);
            if (arg_better(ov, oi, cv, ci)) {
                cv = ov;
                ci = oi;
            }
        }
        if (b == 0) {
            idx[0] = ci < 0 ? 0u : (uint32_t)ci;
            s_tok = ci < 0 ? 0 : ci;
            __hip_atomic_store(count, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    }
    if (!table) return;
    __syncthreads();
    const float *src = table + (size_t)s_tok * d;
    for (int i = threadIdx.x; i < d; i += 256) x_out[i] = src[i];
}

// Prefill form on the fp32 matrix cores (head dim 128): the same causal
// attention as k_attention, in the flash-attention order.  Workgroup =
// (block of 32 query rows, head h), heaviest blocks first; its 4 waves take
// the visible key tiles of 32 round-robin (wave w: tiles w, w + 4, ...), each
// with its own running max, sum and output, and the four partials are
// combined through LDS at the end.  Per tile, with v_mfma_f32_32x32x2_f32:
//   S^T (32 keys x 32 queries) = K_tile . Q^T   (64 MFMAs over the 128 dims)
//   online softmax per query in base 2: P = 2^(S log2(e) / sqrt(128) - m),
//     with m (and l, O^T) moved to the running max only when that grows by
//     more than 12
//   O^T (128 dims x 32 queries) += V_tile^T . P^T   (4 x 16 MFMAs)
// A wave's vector work (softmax) does not overlap its own matrix-core work,
// only another wave's: two workgroups share each CU (80 KiB of LDS and at
// most 256 registers per wave each), so every SIMD runs two waves whose
// softmax, load waits and products interleave.  Each wave stages its tiles
// in its own 16 KiB of LDS with direct global->LDS loads (16 bytes per lane)
// in two 8 KiB halves: dims 0-63 and 64-127 of the K tile, then keys 0-15
// and 16-31 of the V tile, each half loaded while the other half's products
// run.  The layout is the order the lanes read it, so every operand read is
// one conflict-free ds_read_b128 per lane.  The matrix cores sum over k in
// any order, so the dims are permuted to suit that: k-step 4j + c of S pairs
// dims 8j + c (lanes 0-31) and 8j + 4 + c (lanes 32-63) of K row "key" and
// Q row "query"; dim tile dt of O^T holds dims 4i + dt, so V row key's dims
// 4i .. 4i + 3 are one read of lane i.  Each lane holds one query (column
// l % 32), so the softmax's reductions are over its own registers and the
// other half-wave (one shuffle), and P^T feeds the second product from
// registers: in k-step r, lane half u contributes the key of its output
// register r, 8(r/4) + 4u + r%4.  The result differs from the reference's
// sequential sums only in f32 rounding (and v_exp_f32's 1 ulp).
typedef float v16f __attribute__((ext_vector_type(16)));
constexpr int kAmQ = 32;         // query rows per workgroup
constexpr int kAmK = 32;         // keys per tile
constexpr int kAmP = 132;        // combine pitch in floats: [wave][query][dim]
constexpr int kAmHalf = 8192;    // bytes of half a staged tile
constexpr int kAmTile = 2 * kAmHalf;
constexpr int kAmQOff = 4 * kAmTile;                  // Q block after the 4 waves' tiles
constexpr size_t kAmLds = (size_t)kAmQOff + kAmTile;  // 80 KiB: two workgroups per CU
constexpr int kAmMlOff = 4 * kAmQ * kAmP * 4;         // m [4][32], l [4][32] after the partials
constexpr float kAmMove = 12.0f;                      // P <= 2^12 between moves of m
static_assert((size_t)kAmMlOff + 2 * 4 * kAmQ * sizeof(float) <= kAmLds,
              "combine partials, m and l alias the staged tiles and the queries");

// The loads below write M0 themselves; no code of this file keeps a value
// in M0 across them (gfx9 LDS instructions do not use it, and the generated
// code has no other M0 write), so clobbering the reserved register is safe
// here.  s_nop 0 covers the M0 -> LDS DMA hazard.
#pragma clang diagnostic ignored "-Winline-asm"

// 16 bytes per lane from a per-lane address into LDS at lds + 16 * lane
__device__ inline void am_dma16(const void *g, unsigned lds) {
    asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off"
                 :
                 : "v"(g), "s"(lds)
                 : "memory", "m0");
}
// the same from a uniform base plus a per-lane 32-bit offset
__device__ inline void am_dma16_s(const void *base, unsigned voff, unsigned lds) {
    asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, %1"
                 :
                 : "v"(voff), "s"(base), "s"(lds)
                 : "memory", "m0");
}
template <int N>
__device__ inline void am_wait_vm() {
    asm volatile("s_waitcnt vmcnt(%0)" : : "n"(N) : "memory");
}
__device__ inline void am_wait_lds_reads() { asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory"); }

__global__ __launch_bounds__(256, 2) void k_attention_mfma(
    const float *__restrict__ q, int qs, const float *__restrict__ kc,
    const float *__restrict__ vc, int kvd, int seq_q, int start_pos, int groups, int n_heads,
    float scale_log2, float *__restrict__ out, int qd) {
    constexpr int HD = 128;
    extern __shared__ __align__(16) char s_amb[];
    const int t = threadIdx.x, l = t & 63, lq = l & 31, hf = l >> 5;
    const int w = __builtin_amdgcn_readfirstlane(t >> 6);
    const int nqb = (seq_q + kAmQ - 1) / kAmQ;
    const int h = blockIdx.x % n_heads, qb = nqb - 1 - blockIdx.x / n_heads;
    const int kh = h / groups;
    const int i0 = qb * kAmQ;
    const int qi = i0 + lq;           // this lane's query row
    const bool qvalid = qi < seq_q;
    const int pq = start_pos + qi;    // its absolute position: keys 0 .. pq
    const int last_row = min(i0 + kAmQ, seq_q) - 1;
    const int Lw = start_pos + last_row + 1;  // keys the block sees
    const int nt = (Lw + kAmK - 1) / kAmK;

    const unsigned lds0 = __builtin_amdgcn_readfirstlane((unsigned)(size_t)s_amb);
    const unsigned kv_lds = lds0 + w * kAmTile;  // this wave's K, then V tile
    const unsigned q_lds = lds0 + kAmQOff;
    // reader offsets: step j (r) of lane l reads bytes 1024 j + 16 l
    const char *kv_rd = s_amb + w * kAmTile + 16 * l;
    const char *q_rd = s_amb + kAmQOff + 16 * l;

    // Staging: a tile whose 32 rows all lie before the block's last visible
    // key uses uniform row addresses and a fixed per-lane offset; the
    // block's last tile clamps every row to that key (finite values; their
    // scores are masked).
    const size_t row_bytes = (size_t)kvd * 4;
    const char *k_head = reinterpret_cast<const char *>(kc + (size_t)kh * HD);
    const char *v_head = reinterpret_cast<const char *>(vc + (size_t)kh * HD);
    const unsigned k_voff = (unsigned)(lq * row_bytes) + 16 * hf;       // K row lq, dims 4hf ..
    const unsigned v_voff = (unsigned)(4 * hf * row_bytes) + 16 * lq;   // V row 4hf, dims 4lq ..
    auto dma_k = [&](int kt, int half) __attribute__((always_inline)) {
        const unsigned lds = kv_lds + half * kAmHalf;
        if ((kt + 1) * kAmK <= Lw) {
            const char *b = k_head + (size_t)kt * kAmK * row_bytes + 256 * half;
#pragma unroll
            for (int j = 0; j < 8; ++j) am_dma16_s(b + 32 * j, k_voff, lds + 1024 * j);
        } else {
            const float *src = kc + (size_t)min(kt * kAmK + lq, Lw - 1) * kvd + (size_t)kh * HD +
                               4 * hf + 64 * half;
#pragma unroll
            for (int j = 0; j < 8; ++j) am_dma16(src + 8 * j, lds + 1024 * j);
        }
    };
    auto dma_v = [&](int kt, int half) __attribute__((always_inline)) {
        const unsigned lds = kv_lds + half * kAmHalf;
        if ((kt + 1) * kAmK <= Lw) {
#pragma unroll
            for (int rr = 0; rr < 8; ++rr) {
                const int r = 8 * half + rr;
                am_dma16_s(v_head + (size_t)(kt * kAmK + 8 * (r >> 2) + (r & 3)) * row_bytes,
                           v_voff, lds + 1024 * rr);
            }
        } else {
#pragma unroll
            for (int rr = 0; rr < 8; ++rr) {
                const int r = 8 * half + rr;
                const int key = min(kt * kAmK + 8 * (r >> 2) + 4 * hf + (r & 3), Lw - 1);
                am_dma16(vc + (size_t)key * kvd + (size_t)kh * HD + 4 * lq, lds + 1024 * rr);
            }
        }
    };
    // the query block, in the K tile's order (rows past seq_q repeat the last
    // row; their scores are masked): wave w stages steps 4w .. 4w + 3
    {
        const float *src = q + (size_t)min(qi, seq_q - 1) * qs + (size_t)h * HD + 4 * hf;
#pragma unroll
        for (int u = 0; u < 4; ++u) am_dma16(src + 8 * (4 * w + u), q_lds + 1024 * (4 * w + u));
    }

    auto s_half = [&](int half, v16f &x0, v16f &x1) __attribute__((always_inline)) {
#pragma unroll
        for (int jj = 0; jj < 8; ++jj) {
            const int j = 8 * half + jj;
            const float4 kv = *reinterpret_cast<const float4 *>(kv_rd + 1024 * j);
            const float4 qv = *reinterpret_cast<const float4 *>(q_rd + 1024 * j);
            x0 = __builtin_amdgcn_mfma_f32_32x32x2f32(kv.x, qv.x, x0, 0, 0, 0);
            x1 = __builtin_amdgcn_mfma_f32_32x32x2f32(kv.y, qv.y, x1, 0, 0, 0);
            x0 = __builtin_amdgcn_mfma_f32_32x32x2f32(kv.z, qv.z, x0, 0, 0, 0);
            x1 = __builtin_amdgcn_mfma_f32_32x32x2f32(kv.w, qv.w, x1, 0, 0, 0);
        }
    };
    // Online softmax with a lazily moved reference m: P = 2^(y - m), and m
    // (with l and O) moves to the tile max only when that exceeds it by more
    // than kAmMove.  A query with no visible key yet keeps m = -inf, l = 0,
    // O = 0.  Only tiles that reach past the block's first query, or a block
    // with rows past seq_q, need the mask.
    float m_ref = -INFINITY, l_run = 0.0f;
    v16f o[4];
#pragma unroll
    for (int dt = 0; dt < 4; ++dt) o[dt] = v16f{};
    float p[16];
    const bool rows_short = i0 + kAmQ > seq_q;
    auto softmax = [&](const v16f &x, int kt) __attribute__((always_inline)) {
        float y[16];
        if (rows_short || kt * kAmK + kAmK - 1 > start_pos + i0) {
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int key = kt * kAmK + 8 * (r >> 2) + 4 * hf + (r & 3);
                y[r] = (qvalid && key <= pq) ? x[r] * scale_log2 : -INFINITY;
            }
        } else {
#pragma unroll
            for (int r = 0; r < 16; ++r) y[r] = x[r] * scale_log2;
        }
        float mt = y[0];
#pragma unroll
        for (int r = 1; r < 16; ++r) mt = fmaxf(mt, y[r]);
        mt = fmaxf(mt, __shfl_xor(mt, 32));
        const bool move = mt > m_ref + kAmMove;
        const float alpha = move ? __builtin_amdgcn_exp2f(m_ref - mt) : 1.0f;  // 0 from -inf
        m_ref = move ? mt : m_ref;
        const float m_use = m_ref == -INFINITY ? 0.0f : m_ref;  // then every y is -inf
        float ps = 0.0f;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            p[r] = __builtin_amdgcn_exp2f(y[r] - m_use);
            ps = ps + p[r];
        }
        ps = ps + __shfl_xor(ps, 32);
        l_run = l_run * alpha + ps;
        if (__any(move)) {
#pragma unroll
            for (int dt = 0; dt < 4; ++dt) o[dt] = o[dt] * alpha;
        }
    };
    auto pv_half = [&](int half) __attribute__((always_inline)) {
#pragma unroll
        for (int rr = 0; rr < 8; ++rr) {
            const int r = 8 * half + rr;
            const float4 vv = *reinterpret_cast<const float4 *>(kv_rd + 1024 * r);
            o[0] = __builtin_amdgcn_mfma_f32_32x32x2f32(vv.x, p[r], o[0], 0, 0, 0);
            o[1] = __builtin_amdgcn_mfma_f32_32x32x2f32(vv.y, p[r], o[1], 0, 0, 0);
            o[2] = __builtin_amdgcn_mfma_f32_32x32x2f32(vv.z, p[r], o[2], 0, 0, 0);
            o[3] = __builtin_amdgcn_mfma_f32_32x32x2f32(vv.w, p[r], o[3], 0, 0, 0);
        }
    };
    // This wave's tiles kt = w, w + 4, ...  Each half is staged once the
    // reads of what its LDS held before have returned; every wait leaves
    // exactly the other half's 8 loads in flight, in this order:
    //   K lo, K hi | S lo | V lo | S hi | V hi | softmax | PV lo | next K lo
    //   | PV hi | next K hi
    if (w < nt) {
        dma_k(w, 0);
        dma_k(w, 1);
        am_wait_vm<8>();  // this wave's share of the queries, K lo
        __syncthreads();  // every wave's share of the queries
        for (int kt = w; kt < nt; kt += 4) {
            const bool more = kt + 4 < nt;
            am_wait_vm<8>();  // K lo
            v16f x0 = v16f{}, x1 = v16f{};
            s_half(0, x0, x1);
            am_wait_lds_reads();
            dma_v(kt, 0);
            am_wait_vm<8>();  // K hi
            s_half(1, x0, x1);
            am_wait_lds_reads();
            dma_v(kt, 1);
            softmax(x0 + x1, kt);
            am_wait_vm<8>();  // V lo
            pv_half(0);
            am_wait_lds_reads();
            if (more) {
                dma_k(kt + 4, 0);
                am_wait_vm<8>();  // V hi
            } else {
                am_wait_vm<0>();  // V hi
            }
            pv_half(1);
            am_wait_lds_reads();
            if (more) dma_k(kt + 4, 1);
        }
    } else {
        am_wait_vm<0>();
        __syncthreads();
    }
    const float m_run = m_ref;
    // combine: O = sum_w c_w O_w / sum_w c_w l_w, c_w = 2^(m_w - max_w m_w)
    // (a wave that saw no key of a query has m_w = -inf, l_w = 0, O_w = 0);
    // the partials overwrite the staged tiles once every wave is done
    __syncthreads();
    {
        float *s_am = reinterpret_cast<float *>(s_amb);
        float *pw = s_am + (size_t)(w * kAmQ + lq) * kAmP;
#pragma unroll
        for (int r = 0; r < 16; ++r)
            *reinterpret_cast<float4 *>(pw + 4 * (8 * (r >> 2) + 4 * hf + (r & 3))) =
                make_float4(o[0][r], o[1][r], o[2][r], o[3][r]);
        float *sm = reinterpret_cast<float *>(s_amb + kAmMlOff), *sl = sm + 4 * kAmQ;
        if (hf == 0) {
            sm[w * kAmQ + lq] = m_run;
            sl[w * kAmQ + lq] = l_run;
        }
        __syncthreads();
        const int qq = t >> 3, seg = t & 7;  // query, 16-dim segment
        if (i0 + qq >= seq_q) return;
        float mw[4], M = -INFINITY;
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            mw[u] = sm[u * kAmQ + qq];
            M = fmaxf(M, mw[u]);
        }
        float c[4], L = 0.0f;
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            c[u] = __builtin_amdgcn_exp2f(mw[u] - M);  // 0 for m_w = -inf (M is finite)
            L = L + c[u] * sl[u * kAmQ + qq];
        }
        const float inv = 1.0f / L;
        float *op = out + (size_t)(i0 + qq) * qd + (size_t)h * HD + 16 * seg;
#pragma unroll
        for (int d4 = 0; d4 < 4; ++d4) {
            float4 acc = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const float4 v = *reinterpret_cast<const float4 *>(
                    s_am + (size_t)(u * kAmQ + qq) * kAmP + 16 * seg + 4 * d4);
                acc.x = acc.x + c[u] * v.x;
                acc.y = acc.y + c[u] * v.y;
                acc.z = acc.z + c[u] * v.z;
                acc.w = acc.w + c[u] * v.w;
            }
            *reinterpret_cast<float4 *>(op + 4 * d4) =
                make_float4(acc.x * inv, acc.y * inv, acc.z * inv, acc.w * inv);
        }
    }
}

mri_status attn_mfma_launch(const float *q, int qs, int qd, const float *kc, const float *vc,
                            int kvd, int seq_q, int start_pos, int groups, int n_heads,
                            float *out, hipStream_t s) {
    static DeviceOnce attr;
    MRI_HIP(attr.run([](int) {
        return hipFuncSetAttribute(reinterpret_cast<const void *>(&k_attention_mfma),
                                   hipFuncAttributeMaxDynamicSharedMemorySize, (int)kAmLds);
    }));
    const float scale_log2 = (float)(1.4426950408889634 / sqrt(128.0));  // log2(e) / sqrt(128)
    const int nqb = (seq_q + kAmQ - 1) / kAmQ;
    hipLaunchKernelGGL(k_attention_mfma, dim3(nqb * n_heads), dim3(256), kAmLds, s, q, qs, kc, vc,
                       kvd, seq_q, start_pos, groups, n_heads, scale_log2, out, qd);
    MRI_LAUNCHED("k_attention_mfma");
    return MRI_OK;
}

// query rows per prefill workgroup: 16, else 4 when the weight rows do not fit
template <int HD, int QB>
size_t attn_lds(int lcap) {
    return (size_t)(QB * HD + attn_tile_floats<HD>() + (size_t)QB * lcap) * sizeof(float);
}

template <int HD, int QB>
mri_status attn_launch(const float *q, int qs, int qd, const float *kc, const float *vc, int kvd,
                       int seq_q, int start_pos, int groups, int n_heads, float *out,
                       hipStream_t s) {
    const int L = start_pos + seq_q;
    const int lcap = (L + 3) / 4 * 4;
    const size_t lds = attn_lds<HD, QB>(lcap);
    static DeviceOnce attr;
    MRI_HIP(attr.run([](int) {
        return hipFuncSetAttribute(reinterpret_cast<const void *>(&k_attention<HD, QB>),
                                   hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);
    }));
    const float scale = 1.0f / sqrtf((float)HD);
    hipLaunchKernelGGL((k_attention<HD, QB>), dim3((seq_q + QB - 1) / QB, n_heads), dim3(256),
                       lds, s, q, qs, qd, kc, vc, kvd, seq_q, start_pos, groups, lcap, scale, out);
    MRI_LAUNCHED("k_attention");
    return MRI_OK;
}

// Words of the per-head counters at the start of the partials buffer.
inline size_t attn_cnt_words(size_t n_heads) { return (n_heads + 63) / 64 * 64; }

template <int HD>
mri_status attn_dispatch(const float *q, int qs, int qd, const float *kc, const float *vc, int kvd,
                         int seq_q, int start_pos, int groups, int n_heads, float *out,
                         float *part, hipStream_t s) {
    const int L = start_pos + seq_q;
    const bool rows16 =
        (((uintptr_t)q | (uintptr_t)kc | (uintptr_t)vc) & 15) == 0 && kvd % 4 == 0;
    if (seq_q == 1 && HD % 64 == 0 && L <= kDecHeadMaxL && rows16) {
        hipLaunchKernelGGL(k_attn_decode_head<HD>, dim3(n_heads), dim3(512), 0, s, q, kc, vc, kvd,
                           L, groups, 1.0f / sqrtf((float)HD), out);
        MRI_LAUNCHED("k_attn_decode_head");
        return MRI_OK;
    }
    if (seq_q == 1 && part && L <= 1024 * 64 && rows16) {  // the combine holds <= 1024 chunks
        constexpr int NW = 8;  // waves of a chunk, 16 keys each
        const int nch = (L + 16 * NW - 1) / (16 * NW);
        const float scale = 1.0f / sqrtf((float)HD);
        // [head counters, padded to 64 words][partials]
        int *cnt = reinterpret_cast<int *>(part);
        hipLaunchKernelGGL((k_attn_decode_part<HD, NW>), dim3(nch, n_heads), dim3(NW * kWave), 0, s, q, kc,
                           vc, kvd, L, groups, scale, part + attn_cnt_words(n_heads), cnt, out);
        MRI_LAUNCHED("k_attn_decode_part");
        return MRI_OK;
    }
    if (HD == 128 && seq_q >= 32)
        return attn_mfma_launch(q, qs, qd, kc, vc, kvd, seq_q, start_pos, groups, n_heads, out, s);
    const int lcap = (L + 3) / 4 * 4;
    constexpr size_t kMax = 160 * 1024;
    if (attn_lds<HD, 16>(lcap) <= kMax)
        return attn_launch<HD, 16>(q, qs, qd, kc, vc, kvd, seq_q, start_pos, groups, n_heads,
                                   out, s);
    if (attn_lds<HD, 4>(lcap) <= kMax)
        return attn_launch<HD, 4>(q, qs, qd, kc, vc, kvd, seq_q, start_pos, groups, n_heads,
                                  out, s);
    return set_error(MRI_ERR_UNSUPPORTED, "attention: context too long for one workgroup");
}

inline unsigned grid_for(size_t n) {
    const size_t g = (n + 255) / 256;
    return (unsigned)(g < 8192 ? (g ? g : 1) : 8192);
}

}  // namespace

inline bool al16(const void *p) { return ((uintptr_t)p & 15) == 0; }

mri_status launch_embed(const float *table, const uint32_t *tokens, size_t rows, size_t d,
                        float *x, hipStream_t s) {
    if (!rows) return MRI_OK;
    const dim3 grid((unsigned)rows, (unsigned)((d + 1023) / 1024));
    if (d % 4 == 0 && al16(table) && al16(x))
        hipLaunchKernelGGL(k_embed<true>, grid, dim3(256), 0, s, table, tokens, (int)d, x);
    else
        hipLaunchKernelGGL(k_embed<false>, grid, dim3(256), 0, s, table, tokens, (int)d, x);
    MRI_LAUNCHED("k_embed");
    return MRI_OK;
}

mri_status launch_rmsnorm(const float *x, const float *w, size_t rows, size_t d, float eps,
                          float *out, hipStream_t s) {
    if (!rows) return MRI_OK;
    const dim3 g((unsigned)rows), b(256);
    const bool v4 = d % 4 == 0 && al16(x) && al16(w) && al16(out);
    if (v4 && d <= 1024)
        hipLaunchKernelGGL(k_rmsnorm<1>, g, b, 0, s, x, w, (int)d, eps, out);
    else if (v4 && d <= 2048)
        hipLaunchKernelGGL(k_rmsnorm<2>, g, b, 0, s, x, w, (int)d, eps, out);
    else if (v4 && d <= 4096)
        hipLaunchKernelGGL(k_rmsnorm<4>, g, b, 0, s, x, w, (int)d, eps, out);
    else if (v4 && d <= 8192)
        hipLaunchKernelGGL(k_rmsnorm<8>, g, b, 0, s, x, w, (int)d, eps, out);
    else
        hipLaunchKernelGGL(k_rmsnorm<0>, g, b, 0, s, x, w, (int)d, eps, out);
    MRI_LAUNCHED("k_rmsnorm");
    return MRI_OK;
}

// Embedding gather + RMSNorm (x_out = table[tokens], out = rmsnorm(x_out)),
// or residual add + RMSNorm (x += delta, out = rmsnorm(x)).  Falls back to
// the separate kernels for shapes the one-pass form does not take.
mri_status launch_embed_rmsnorm(const float *table, const uint32_t *tokens, size_t rows,
                                size_t d, const float *w, float eps, float *x_out, float *out,
                                hipStream_t s) {
    if (!rows) return MRI_OK;
    if (d % 4 || d > 8192 || !al16(table) || !al16(w) || !al16(out) || !al16(x_out)) {
        mri_status st = launch_embed(table, tokens, rows, d, x_out, s);
        if (st) return st;
        return launch_rmsnorm(x_out, w, rows, d, eps, out, s);
    }
    const dim3 g((unsigned)rows), b(256);
    if (d <= 1024)
        hipLaunchKernelGGL((k_rmsnorm<1, 1>), g, b, 0, s, table, w, (int)d, eps, out, tokens,
                           nullptr, x_out);
    else if (d <= 2048)
        hipLaunchKernelGGL((k_rmsnorm<2, 1>), g, b, 0, s, table, w, (int)d, eps, out, tokens,
                           nullptr, x_out);
    else if (d <= 4096)
        hipLaunchKernelGGL((k_rmsnorm<4, 1>), g, b, 0, s, table, w, (int)d, eps, out, tokens,
                           nullptr, x_out);
    else
        hipLaunchKernelGGL((k_rmsnorm<8, 1>), g, b, 0, s, table, w, (int)d, eps, out, tokens,
                           nullptr, x_out);
    MRI_LAUNCHED("k_rmsnorm");
    return MRI_OK;
}

mri_status launch_add_rmsnorm(float *x, const float *delta, size_t rows, size_t d,
                              const float *w, float eps, float *out, hipStream_t s) {
    if (!rows) return MRI_OK;
    if (d % 4 || d > 8192 || !al16(x) || !al16(delta) || !al16(w) || !al16(out)) {
        mri_status st = launch_add(x, delta, rows * d, x, s);
        if (st) return st;
        return launch_rmsnorm(x, w, rows, d, eps, out, s);
    }
    const dim3 g((unsigned)rows), b(256);
    if (d <= 1024)
        hipLaunchKernelGGL((k_rmsnorm<1, 2>), g, b, 0, s, x, w, (int)d, eps, out, nullptr,
                           delta, x);
    else if (d <= 2048)
        hipLaunchKernelGGL((k_rmsnorm<2, 2>), g, b, 0, s, x, w, (int)d, eps, out, nullptr,
                           delta, x);
    else if (d <= 4096)
        hipLaunchKernelGGL((k_rmsnorm<4, 2>), g, b, 0, s, x, w, (int)d, eps, out, nullptr,
                           delta, x);
    else
        hipLaunchKernelGGL((k_rmsnorm<8, 2>), g, b, 0, s, x, w, (int)d, eps, out, nullptr,
                           delta, x);
    MRI_LAUNCHED("k_rmsnorm");
    return MRI_OK;
}

bool rmsnorm_stats_supported(size_t d) { return d % 4 == 0 && d <= 8192; }

// The statistics of RMSNorm rows (STATS above): mode 0 norm x as is, mode 1
// gather the rows from `table` by `tokens` into x_out first, mode 2 add
// delta into x first.  d % 4 == 0, d <= 8192, 16-byte aligned rows.
mri_status launch_rmsnorm_stats(int mode, const float *x, const float *delta,
                                const uint32_t *tokens, float *x_out, size_t rows, size_t d,
                                const float *w, float eps, float *stats, hipStream_t s) {
    if (!rows) return MRI_OK;
    if (!rmsnorm_stats_supported(d) || !al16(x) || !al16(w) || (delta && !al16(delta)) ||
        (x_out && !al16(x_out)))
        return set_error(MRI_ERR_INVALID_ARGUMENT, "rmsnorm stats: unsupported row shape");
    const dim3 g((unsigned)rows), b(256);
    auto go = [&](auto nv) {
        constexpr int NV = decltype(nv)::value;
        if (mode == 1)
            hipLaunchKernelGGL((k_rmsnorm<NV, 1, true>), g, b, 0, s, x, w, (int)d, eps, stats,
                               tokens, nullptr, x_out);
        else if (mode == 2)
            hipLaunchKernelGGL((k_rmsnorm<NV, 2, true>), g, b, 0, s, x, w, (int)d, eps, stats,
                               nullptr, delta, x_out);
        else
            hipLaunchKernelGGL((k_rmsnorm<NV, 0, true>), g, b, 0, s, x, w, (int)d, eps, stats);
    };
    if (d <= 1024) go(std::integral_constant<int, 1>{});
    else if (d <= 2048) go(std::integral_constant<int, 2>{});
    else if (d <= 4096) go(std::integral_constant<int, 4>{});
    else go(std::integral_constant<int, 8>{});
    MRI_LAUNCHED("k_rmsnorm(stats)");
    return MRI_OK;
}

mri_status launch_rope_qkv(float *q, const float *k, const float *v, size_t seq, size_t n_heads,
                           size_t n_kv, size_t head_dim, size_t q_stride, size_t kv_stride,
                           const float *cos_t, const float *sin_t, size_t start_pos, float *kc,
                           float *vc, hipStream_t s) {
    if (!seq) return MRI_OK;
    if (head_dim % 2 || head_dim > 128)
        return set_error(MRI_ERR_UNSUPPORTED, "rope: head_dim must be even and <= 128");
    const int kvd = (int)(n_kv * head_dim);
    hipLaunchKernelGGL(k_rope_qkv, dim3((unsigned)seq, (unsigned)(n_heads + 2 * n_kv)), dim3(64),
                       0, s, q, k, v, (int)q_stride, (int)kv_stride, kvd, (int)(head_dim / 2),
                       (int)n_heads, (int)n_kv, cos_t, sin_t, (int)start_pos, kc, vc);
    MRI_LAUNCHED("k_rope_qkv");
    return MRI_OK;
}

bool attention_supported(size_t head_dim) { return head_dim == 64 || head_dim == 128; }

size_t attention_part_floats(size_t n_heads, size_t head_dim, size_t max_seq) {
    return attn_cnt_words(n_heads) + n_heads * ((max_seq + 63) / 64) * (head_dim + 2);
}

mri_status launch_attention(const float *q, size_t q_stride, size_t seq_q, const float *kc,
                            const float *vc, size_t n_heads, size_t n_kv_heads, size_t head_dim,
                            size_t start_pos, float *out, float *part, hipStream_t s) {
    if (!seq_q) return MRI_OK;
    const int qd = (int)(n_heads * head_dim), kvd = (int)(n_kv_heads * head_dim);
    const int groups = (int)(n_heads / n_kv_heads), qs = (int)q_stride;
    if (head_dim == 128)
        return attn_dispatch<128>(q, qs, qd, kc, vc, kvd, (int)seq_q, (int)start_pos, groups,
                                  (int)n_heads, out, part, s);
    if (head_dim == 64)
        return attn_dispatch<64>(q, qs, qd, kc, vc, kvd, (int)seq_q, (int)start_pos, groups,
                                 (int)n_heads, out, part, s);
    return set_error(MRI_ERR_UNSUPPORTED, "attention: head_dim must be 64 or 128");
}

mri_status launch_swiglu(const float *gate, const float *up, size_t n, float *out,
                         hipStream_t s) {
    if (!n) return MRI_OK;
    if (n % 4 == 0 && al16(gate) && al16(up) && al16(out))
        hipLaunchKernelGGL(k_swiglu4, dim3(grid_for(n / 4)), dim3(256), 0, s,
                           reinterpret_cast<const float4 *>(gate),
                           reinterpret_cast<const float4 *>(up), n / 4,
                           reinterpret_cast<float4 *>(out));
    else
        hipLaunchKernelGGL(k_swiglu, dim3(grid_for(n)), dim3(256), 0, s, gate, up, n, out);
    MRI_LAUNCHED("k_swiglu");
    return MRI_OK;
}

mri_status launch_swiglu_rows(const float *gu, size_t rows, size_t ffn, float *out,
                              hipStream_t s) {
    if (!rows || !ffn) return MRI_OK;
    if (ffn % 4 || !al16(gu) || !al16(out)) {
        for (size_t r = 0; r < rows; ++r) {
            mri_status st = launch_swiglu(gu + r * 2 * ffn, gu + r * 2 * ffn + ffn, ffn,
                                          out + r * ffn, s);
            if (st) return st;
        }
        return MRI_OK;
    }
    const size_t n4 = rows * ffn / 4;
    hipLaunchKernelGGL(k_swiglu_rows4, dim3(grid_for(n4)), dim3(256), 0, s,
                       reinterpret_cast<const float4 *>(gu), (int)(ffn / 4), n4,
                       reinterpret_cast<float4 *>(out));
    MRI_LAUNCHED("k_swiglu_rows4");
    return MRI_OK;
}

mri_status launch_add(const float *a, const float *b, size_t n, float *out, hipStream_t s) {
    if (!n) return MRI_OK;
    if (n % 4 == 0 && al16(a) && al16(b) && al16(out))
        hipLaunchKernelGGL(k_add4, dim3(grid_for(n / 4)), dim3(256), 0, s,
                           reinterpret_cast<const float4 *>(a), reinterpret_cast<const float4 *>(b),
                           n / 4, reinterpret_cast<float4 *>(out));
    else
        hipLaunchKernelGGL(k_add, dim3(grid_for(n)), dim3(256), 0, s, a, b, n, out);
    MRI_LAUNCHED("k_add");
    return MRI_OK;
}

static mri_status launch_argmax_split(const float *v, size_t n, uint32_t *idx,
                                      const float *table, size_t d, float *x_out,
                                      hipStream_t s) {
    void *ws = nullptr;
    mri_status st = argmax_ws_get(s, &ws);
    if (st) return st;
    const unsigned blocks = (unsigned)std::min<size_t>(kArgSplit, std::max<size_t>(1, n / 512));
    hipLaunchKernelGGL(k_argmax_split, dim3(blocks), dim3(256), 0, s, v, (int)n, idx, table,
                       (int)d, x_out, static_cast<unsigned *>(ws));
    MRI_LAUNCHED("k_argmax_split");
    return MRI_OK;
}

mri_status launch_argmax_keys(const unsigned long long *keys, size_t n, uint32_t *idx,
                              const float *table, size_t d, float *x_out, hipStream_t s) {
    if (table && (d % 4 || !al16(table) || !al16(x_out)))
        return set_error(MRI_ERR_INVALID_ARGUMENT, "argmax: table rows must be float4-aligned");
    hipLaunchKernelGGL(k_argmax_keys, dim3(1), dim3(256), 0, s, keys, (int)n, idx, table, (int)d,
                       x_out);
    MRI_LAUNCHED("k_argmax_keys");
    return MRI_OK;
}

mri_status launch_argmax(const float *v, size_t rows, size_t n, uint32_t *idx, hipStream_t s) {
    if (!rows) return MRI_OK;
    if (rows == 1) return launch_argmax_split(v, n, idx, nullptr, 0, nullptr, s);
    hipLaunchKernelGGL(k_argmax, dim3((unsigned)rows), dim3(1024), 0, s, v, (int)n, idx);
    MRI_LAUNCHED("k_argmax");
    return MRI_OK;
}

mri_status launch_argmax_embed(const float *v, size_t n, uint32_t *idx, const float *table,
                               size_t d, float *x_out, hipStream_t s) {
    return launch_argmax_split(v, n, idx, table, d, x_out, s);
}

}  // namespace mri
