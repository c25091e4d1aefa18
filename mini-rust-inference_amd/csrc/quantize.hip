// quantize.hip — activation / weight quantizers on gfx950.
//
// All of them evaluate the reference's scalar formula exactly
// (quant/int8/symmetric.rs:42-57, per_channel.rs:98-128):
//   max_abs = fold(0, f32::max)(|v|)          (fmaxf ignores NaN as f32::max)
//   scale   = max_abs == 0 ? 1 : max_abs / 127 (correctly rounded divide)
//   inv     = 1 / scale                         (correctly rounded divide)
//   q       = clamp(round_half_away(v * inv), -127, 127) as i8, NaN -> 0
// The library is compiled with -ffp-contract=off and correctly rounded
// f32 division, so each operation rounds exactly once, as in Rust.
#include "common.hpp"

namespace mri {
namespace {

constexpr int kThreads = 256;
constexpr int kMaxPartials = 1024;

__device__ inline int8_t round_clamp_i8(float y) {
    float r = roundf(y);              // ties away from zero, like f32::round
    if (r != r) return 0;             // `NaN as i8` == 0
    r = fminf(fmaxf(r, -127.0f), 127.0f);
    return (int8_t)(int)r;
}

__device__ inline float scale_of(float max_abs) {
    return max_abs == 0.0f ? 1.0f : __fdiv_rn(max_abs, 127.0f);
}

// Block-wide max of non-negative floats (NaN-free inputs are not required:
// fmaxf drops NaN operands).
__device__ inline float block_max(float v, float *red) {
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o));
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    if (lane == 0) red[wave] = v;
    __syncthreads();
    float r = 0.0f;
    for (int w = 0; w < (int)(blockDim.x >> 6); ++w) r = fmaxf(r, red[w]);
    __syncthreads();
    return r;
}

__global__ __launch_bounds__(kThreads) void k_absmax_partial(
    const float *__restrict__ x, size_t n, float *__restrict__ partials) {
    __shared__ float red[kThreads / 64];
    float m = 0.0f;
    const size_t stride = (size_t)gridDim.x * blockDim.x;
    size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if ((reinterpret_cast<uintptr_t>(x) & 15) == 0) {
        const size_t n4 = n / 4;
        const float4 *x4 = reinterpret_cast<const float4 *>(x);
        for (size_t j = i; j < n4; j += stride) {
            float4 v = x4[j];
            m = fmaxf(m, fabsf(v.x));
            m = fmaxf(m, fabsf(v.y));
            m = fmaxf(m, fabsf(v.z));
            m = fmaxf(m, fabsf(v.w));
        }
        for (size_t j = n4 * 4 + i; j < n; j += stride) m = fmaxf(m, fabsf(x[j]));
    } else {
        for (size_t j = i; j < n; j += stride) m = fmaxf(m, fabsf(x[j]));
    }
    m = block_max(m, red);
    if (threadIdx.x == 0) partials[blockIdx.x] = m;
}

// Quantize [m,k] with the per-tensor scale reduced from `partials`.
// q_pad: [m][ld] (ld >= k, zero padded; chunk-permuted when perm) or null;
// q_plain: [m*k] row-major or null.
__global__ __launch_bounds__(kThreads) void k_quantize_tensor(
    const float *__restrict__ x, size_t m, size_t k, size_t ld, int perm,
    const float *__restrict__ partials, int n_partials,
    int8_t *__restrict__ q_pad, int8_t *__restrict__ q_plain,
    float *__restrict__ scale_out) {
    __shared__ float red[kThreads / 64];
    float mx = 0.0f;
    for (int i = threadIdx.x; i < n_partials; i += blockDim.x)
        mx = fmaxf(mx, partials[i]);
    mx = block_max(mx, red);
    const float scale = scale_of(mx);
    const float inv = __fdiv_rn(1.0f, scale);
    if (blockIdx.x == 0 && threadIdx.x == 0 && scale_out) *scale_out = scale;
    const size_t total = m * ld;
    const size_t stride = (size_t)gridDim.x * blockDim.x;
    for (size_t e = (size_t)blockIdx.x * blockDim.x + threadIdx.x; e < total;
         e += stride) {
        const size_t r = e / ld, kk = e - r * ld;
        int8_t q = 0;
        if (kk < k) {
            q = round_clamp_i8(x[r * k + kk] * inv);
            if (q_plain) q_plain[r * k + kk] = q;
        }
        if (q_pad) {
            size_t pos = kk;
            if (perm) pos = (kk & ~(size_t)63) + q8_perm((int)(kk & 63));
            q_pad[r * ld + pos] = q;
        }
    }
}

__device__ inline float absmax4(float m, const float4 &v) {
    return fmaxf(fmaxf(m, fmaxf(fabsf(v.x), fabsf(v.y))), fmaxf(fabsf(v.z), fabsf(v.w)));
}

// Offset of element kk (kk % 4 == 0 keeps 4 elements contiguous) in a
// padded output row, chunk-permuted when perm.
__device__ inline size_t row_pos(size_t kk, int perm) {
    return perm ? (kk & ~(size_t)63) + q8_perm((int)(kk & 63)) : kk;
}

// SwiGLU of one element, silu(g) * u (activation/swiglu.rs, silu.rs:23-26),
// in the expression of the prefill SwiGLU kernel (k_swiglu_rows4), so that
// the values are its own.
__device__ inline float swiglu_elem(float g, float u) { return g / (1.0f + expf(-g)) * u; }

// One block per row: quantize_symmetric of each row separately.  NV > 0:
// the row (16-byte aligned, k % 4 == 0, k <= NV * 4 * kThreads, 4-byte
// aligned outputs) is loaded once as float4 into registers, NV loads in
// flight per thread, and written four int8 at a time.  NV == 0: element-wise
// path for every other shape.  GLU: x holds rows of 2k, [gate | up], and
// the quantized row is their SwiGLU (what k_swiglu_rows4 writes, quantized
// as the separate pass would quantize it).
template <int NV, bool GLU = false, int TH = kThreads>
__global__ __launch_bounds__(TH) void k_quantize_rows(
    const float *__restrict__ x, size_t k, size_t ld, int perm,
    int8_t *__restrict__ q_pad, int8_t *__restrict__ q_plain,
    float *__restrict__ scales) {
    __shared__ float red[TH / 64];
    const size_t r = blockIdx.x;
    const float *row = x + r * (GLU ? 2 * k : k);
    const float *urow = row + k;  // GLU: the up half
    const size_t t = threadIdx.x;
    float mx = 0.0f;
    if constexpr (NV > 0) {
        const float4 *r4 = reinterpret_cast<const float4 *>(row);
        const size_t k4 = k / 4;
        float4 v[NV];
        if constexpr (GLU) {
            // unconditional loads at an in-row index (no branches, so all of
            // them are in flight at once); lanes past the row are zeroed
            const float4 *u4 = reinterpret_cast<const float4 *>(urow);
            float4 u[NV];
#pragma unroll
            for (int j = 0; j < NV; ++j) {
                const size_t i = min(t + (size_t)j * TH, k4 - 1);
                v[j] = r4[i];
                u[j] = u4[i];
            }
#pragma unroll
            for (int j = 0; j < NV; ++j) {
                const bool in = t + (size_t)j * TH < k4;
                v[j] = in ? float4{swiglu_elem(v[j].x, u[j].x), swiglu_elem(v[j].y, u[j].y),
                                   swiglu_elem(v[j].z, u[j].z), swiglu_elem(v[j].w, u[j].w)}
                          : float4{0.0f, 0.0f, 0.0f, 0.0f};
            }
        } else {
#pragma unroll
            for (int j = 0; j < NV; ++j) {
                const size_t i = t + (size_t)j * TH;
                v[j] = i < k4 ? r4[i] : float4{0.0f, 0.0f, 0.0f, 0.0f};
            }
        }
#pragma unroll
        for (int j = 0; j < NV; ++j) mx = absmax4(mx, v[j]);
        mx = block_max(mx, red);
        const float scale = scale_of(mx);
        const float inv = __fdiv_rn(1.0f, scale);
        if (t == 0 && scales) scales[r] = scale;
#pragma unroll
        for (int j = 0; j < NV; ++j) {
            const size_t kk = 4 * (t + (size_t)j * TH);
            if (kk < k) {
                const int packed = ((int)round_clamp_i8(v[j].x * inv) & 255) |
                                   (((int)round_clamp_i8(v[j].y * inv) & 255) << 8) |
                                   (((int)round_clamp_i8(v[j].z * inv) & 255) << 16) |
                                   ((int)round_clamp_i8(v[j].w * inv) << 24);
                if (q_plain) *reinterpret_cast<int *>(q_plain + r * k + kk) = packed;
                if (q_pad) *reinterpret_cast<int *>(q_pad + r * ld + row_pos(kk, perm)) = packed;
            }
        }
        // zero padding of the output row
        if (q_pad)
            for (size_t kk = k + 4 * t; kk < ld; kk += 4 * TH)
                *reinterpret_cast<int *>(q_pad + r * ld + row_pos(kk, perm)) = 0;
    } else {
        auto elem = [&](size_t i) { return GLU ? swiglu_elem(row[i], urow[i]) : row[i]; };
        for (size_t i = t; i < k; i += blockDim.x) mx = fmaxf(mx, fabsf(elem(i)));
        mx = block_max(mx, red);
        const float scale = scale_of(mx);
        const float inv = __fdiv_rn(1.0f, scale);
        if (t == 0 && scales) scales[r] = scale;
        for (size_t kk = t; kk < ld; kk += blockDim.x) {
            int8_t q = 0;
            if (kk < k) {
                q = round_clamp_i8(elem(kk) * inv);
                if (q_plain) q_plain[r * k + kk] = q;
            }
            if (q_pad) q_pad[r * ld + row_pos(kk, perm)] = q;
        }
    }
}

// float4s per thread of the register-resident row path for k with th
// threads per row (0: none).
inline int rows_nv(const float *x, size_t k, size_t ld, const int8_t *q_pad,
                   const int8_t *q_plain, size_t th = kThreads) {
    if ((k & 3) || (ld & 3) || (reinterpret_cast<uintptr_t>(x) & 15) ||
        (reinterpret_cast<uintptr_t>(q_pad) & 3) || (reinterpret_cast<uintptr_t>(q_plain) & 3))
        return 0;
    const size_t per = (k / 4 + th - 1) / th;
    return per <= 4 ? 4 : per <= 8 ? 8 : per <= 16 ? 16 : 0;
}

// GLU rows (two loads per element) run 1024 threads per row: with 256 the
// 512 rows of a prefill leave too few loads in flight (512 x 11008: 16.7 us
// at 256 threads, 13.0 us at 1024, against 11.7 + 13.0 us for the SwiGLU
// kernel followed by the separate pass).  So do up to 32 rows, where the
// launch is a handful of workgroups and its latency is the whole cost
// (matmul_q8_0_direct at 2-32 x 4096 -> 11008: 0.02-0.15 us less per call,
// the same bytes; from 128 rows up 1024 threads gave the same times).
template <bool GLU, int TH = GLU ? 1024 : kThreads>
void launch_rows(const float *x, size_t m, size_t k, size_t ld, int perm, int8_t *q_pad,
                 int8_t *q_plain, float *scales, hipStream_t s) {
    if constexpr (!GLU && TH == kThreads) {
        if (m <= 32) return launch_rows<false, 1024>(x, m, k, ld, perm, q_pad, q_plain, scales, s);
    }
    const dim3 grid((unsigned)m), block(TH);
    switch (rows_nv(x, k, ld, q_pad, q_plain, TH)) {
    case 4: hipLaunchKernelGGL((k_quantize_rows<4, GLU, TH>), grid, block, 0, s, x, k, ld, perm, q_pad, q_plain, scales); break;
    case 8: hipLaunchKernelGGL((k_quantize_rows<8, GLU, TH>), grid, block, 0, s, x, k, ld, perm, q_pad, q_plain, scales); break;
    case 16: hipLaunchKernelGGL((k_quantize_rows<16, GLU, TH>), grid, block, 0, s, x, k, ld, perm, q_pad, q_plain, scales); break;
    default: hipLaunchKernelGGL((k_quantize_rows<0, GLU, TH>), grid, block, 0, s, x, k, ld, perm, q_pad, q_plain, scales); break;
    }
}

__global__ __launch_bounds__(kThreads) void k_pad_rows(
    const int8_t *__restrict__ src, size_t m, size_t k, size_t kp,
    int8_t *__restrict__ dst) {
    const size_t total = m * kp;
    const size_t stride = (size_t)gridDim.x * blockDim.x;
    for (size_t e = (size_t)blockIdx.x * blockDim.x + threadIdx.x; e < total;
         e += stride) {
        const size_t r = e / kp, kk = e - r * kp;
        dst[e] = kk < k ? src[r * k + kk] : (int8_t)0;
    }
}

// Single-block int32 dot (wrapping arithmetic, as Rust release i32 adds).
__global__ __launch_bounds__(kThreads) void k_dot_i8(
    const int8_t *__restrict__ a, const int8_t *__restrict__ b, size_t n,
    int32_t *__restrict__ out) {
    __shared__ uint32_t red[kThreads / 64];
    uint32_t s = 0;
    for (size_t i = threadIdx.x; i < n; i += blockDim.x)
        s += (uint32_t)((int32_t)a[i] * (int32_t)b[i]);
    for (int o = 32; o > 0; o >>= 1) s += __shfl_xor(s, o);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = s;
    __syncthreads();
    if (threadIdx.x == 0) {
        uint32_t t = 0;
        for (int w = 0; w < kThreads / 64; ++w) t += red[w];
        *out = (int32_t)t;
    }
}

// Piece e (16 bytes) of the packed GEMM activation layout (common.hpp):
// returns its row and first k.
__device__ inline void pack_piece(size_t e, size_t mg, size_t *row, size_t *k0) {
    const size_t lane = e & 63, t = e >> 6;
    const size_t h = t & 1;
    const unsigned t2 = (unsigned)(t >> 1), mgu = (unsigned)mg;  // 32-bit: t2 < pieces / 128
    const size_t g = t2 % mgu, p = t2 / mgu;
    *row = 32 * g + (lane & 31);
    *k0 = 64 * p + 32 * h + 16 * (lane >> 5);
}

// quantize_symmetric with the per-tensor scale reduced from `partials`,
// written straight into the packed GEMM layout (zero padded to mg*32 rows
// and kp columns); q_plain (optional) receives the [m*k] row-major values.
__global__ __launch_bounds__(kThreads) void k_quantize_pack(
    const float *__restrict__ x, size_t m, size_t k, size_t mg, size_t kp,
    const float *__restrict__ partials, int n_partials, int8_t *__restrict__ packed,
    int8_t *__restrict__ q_plain, float *__restrict__ scale_out) {
    __shared__ float red[kThreads / 64];
    float mx = 0.0f;
    for (int i = threadIdx.x; i < n_partials; i += blockDim.x)
        mx = fmaxf(mx, partials[i]);
    mx = block_max(mx, red);
    const float scale = scale_of(mx);
    const float inv = __fdiv_rn(1.0f, scale);
    if (blockIdx.x == 0 && threadIdx.x == 0 && scale_out) *scale_out = scale;
    const size_t pieces = mg * 32 * kp / 16;
    const size_t stride = (size_t)gridDim.x * blockDim.x;
    // whole 16-element pieces of rows with k % 4 == 0 (16-byte aligned x):
    // four float4 loads; a plain int8 copy as one 16-byte store when its
    // rows are 16-byte aligned too
    const bool v4 = k % 4 == 0 && (reinterpret_cast<uintptr_t>(x) & 15) == 0;
    const bool p16 = k % 16 == 0 && (reinterpret_cast<uintptr_t>(q_plain) & 15) == 0;
    for (size_t e = (size_t)blockIdx.x * blockDim.x + threadIdx.x; e < pieces; e += stride) {
        size_t r, k0;
        pack_piece(e, mg, &r, &k0);
        int8_t q[16];
        if (v4 && r < m && k0 + 16 <= k) {
            const float4 *src = reinterpret_cast<const float4 *>(x + r * k + k0);
            float4 f[4];
#pragma unroll
            for (int u = 0; u < 4; ++u) f[u] = src[u];
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                q[4 * u + 0] = round_clamp_i8(f[u].x * inv);
                q[4 * u + 1] = round_clamp_i8(f[u].y * inv);
                q[4 * u + 2] = round_clamp_i8(f[u].z * inv);
                q[4 * u + 3] = round_clamp_i8(f[u].w * inv);
            }
            if (q_plain) {
                if (p16)
                    *reinterpret_cast<int4 *>(q_plain + r * k + k0) =
                        *reinterpret_cast<const int4 *>(q);
                else
                    for (int j = 0; j < 16; ++j) q_plain[r * k + k0 + j] = q[j];
            }
        } else {
#pragma unroll
            for (int j = 0; j < 16; ++j) {
                const size_t kk = k0 + j;
                q[j] = (r < m && kk < k) ? round_clamp_i8(x[r * k + kk] * inv) : (int8_t)0;
                if (q_plain && r < m && kk < k) q_plain[r * k + kk] = q[j];
            }
        }
        *reinterpret_cast<int4 *>(packed + e * 16) = *reinterpret_cast<const int4 *>(q);
    }
}

// Row-major int8 rows [m][ld] (k valid columns) into the packed GEMM layout.
__global__ __launch_bounds__(kThreads) void k_pack_gemm(
    const int8_t *__restrict__ src, size_t m, size_t k, size_t ld, size_t mg, size_t kp,
    int8_t *__restrict__ packed) {
    const size_t pieces = mg * 32 * kp / 16;
    const size_t stride = (size_t)gridDim.x * blockDim.x;
    // whole pieces of 16-byte aligned rows move as one 16-byte load
    const bool v16 = ld % 16 == 0 && (reinterpret_cast<uintptr_t>(src) & 15) == 0;
    for (size_t e = (size_t)blockIdx.x * blockDim.x + threadIdx.x; e < pieces; e += stride) {
        size_t r, k0;
        pack_piece(e, mg, &r, &k0);
        int4 v;
        if (v16 && r < m && k0 + 16 <= k) {
            v = *reinterpret_cast<const int4 *>(src + r * ld + k0);
        } else {
            int8_t q[16];
#pragma unroll
            for (int j = 0; j < 16; ++j) {
                const size_t kk = k0 + j;
                q[j] = (r < m && kk < k) ? src[r * ld + kk] : (int8_t)0;
            }
            v = *reinterpret_cast<const int4 *>(q);
        }
        *reinterpret_cast<int4 *>(packed + e * 16) = v;
    }
}

inline int grid_for(size_t n, int per_thread = 1) {
    size_t g = (n + (size_t)kThreads * per_thread - 1) / ((size_t)kThreads * per_thread);
    if (g < 1) g = 1;
    if (g > 4096) g = 4096;
    return (int)g;
}

}  // namespace

size_t quantize_partials_count(size_t n) {
    size_t g = (n + (size_t)kThreads * 16 - 1) / ((size_t)kThreads * 16);
    if (g < 1) g = 1;
    if (g > (size_t)kMaxPartials) g = kMaxPartials;
    return g;
}

mri_status launch_quantize_tensor(const float *x, size_t m, size_t k,
                                  size_t ld_out, bool q8_perm_layout,
                                  int8_t *q_pad, int8_t *q_plain,
                                  float *scale, float *partials,
                                  hipStream_t s) {
    const size_t n = m * k;
    const int g = (int)quantize_partials_count(n);
    hipLaunchKernelGGL(k_absmax_partial, dim3(g), dim3(kThreads), 0, s, x, n,
                       partials);
    MRI_LAUNCHED("k_absmax_partial");
    hipLaunchKernelGGL(k_quantize_tensor, dim3(grid_for(m * (q_pad ? ld_out : k), 4)),
                       dim3(kThreads), 0, s, x, m, k, q_pad ? ld_out : k,
                       q8_perm_layout ? 1 : 0, partials, g, q_pad, q_plain,
                       scale);
    MRI_LAUNCHED("k_quantize_tensor");
    return MRI_OK;
}

mri_status launch_quantize_pack(const float *x, size_t m, size_t k, size_t kp,
                                int8_t *packed, int8_t *q_plain, float *scale,
                                float *partials, hipStream_t s) {
    const size_t n = m * k;
    const int g = (int)quantize_partials_count(n);
    hipLaunchKernelGGL(k_absmax_partial, dim3(g), dim3(kThreads), 0, s, x, n, partials);
    MRI_LAUNCHED("k_absmax_partial");
    const size_t mg = gemm_row_groups(m);
    hipLaunchKernelGGL(k_quantize_pack, dim3(grid_for(mg * 32 * kp / 16)), dim3(kThreads), 0,
                       s, x, m, k, mg, kp, partials, g, packed, q_plain, scale);
    MRI_LAUNCHED("k_quantize_pack");
    return MRI_OK;
}

namespace {

// ---------------------------------------------------------------------------
// Quantization of RMS-normalized rows that are not in memory: row r is
// y = w * (x[r] * rms_inv[r]) (rmsnorm.rs:100-114, the operations of
// k_rmsnorm), with rms_inv[r] = stats[2r] and max |y| = stats[2r+1] from
// the statistics pass.  FORM 0: per-tensor scale (quantize_symmetric over
// all rows, as matmul_int8_from_f32 quantizes its input), GEMM-packed
// layout, grid over the rows padded to 32 (padding rows are zero); FORM 1:
// per-tensor, [rows][ld] plain; FORM 2: per-row scales (matmul_q8_0_direct),
// [rows][ld] chunk-permuted; FORM 3: the normalized f32 rows themselves.
// The quantized values equal those of quantizing the stored normalized
// rows: the same y, the same max, the same scale.
template <int NV, int FORM>
__global__ __launch_bounds__(kThreads) void k_norm_quant(
    const float *__restrict__ x, const float *__restrict__ w, const float *__restrict__ stats,
    int rows, int d, size_t ld, size_t mg, int8_t *__restrict__ q, float *__restrict__ scales,
    float *__restrict__ normed) {
    __shared__ float red[kThreads / 64];
    const int r = blockIdx.x;
    const int t = threadIdx.x;
    if (FORM == 0 && r >= rows) {  // padding rows of the packed layout
        for (size_t kk = 4 * (size_t)t; kk < ld; kk += 4 * kThreads)
            *reinterpret_cast<int *>(q + gemm_pack_offset(r, kk, mg)) = 0;
        return;
    }
    const float rms_inv = stats[2 * (size_t)r];
    const float4 *x4 = reinterpret_cast<const float4 *>(x + (size_t)r * d);
    const float4 *w4 = reinterpret_cast<const float4 *>(w);
    float4 y[NV];
#pragma unroll
    for (int c = 0; c < NV; ++c) {
        const int i = c * kThreads + t;
        if (4 * i < d) {
            const float4 xv = x4[i], wv = w4[i];
            y[c] = float4{wv.x * (xv.x * rms_inv), wv.y * (xv.y * rms_inv),
                          wv.z * (xv.z * rms_inv), wv.w * (xv.w * rms_inv)};
        } else {
            y[c] = float4{0.0f, 0.0f, 0.0f, 0.0f};
        }
    }
    if constexpr (FORM == 3) {
#pragma unroll
        for (int c = 0; c < NV; ++c) {
            const int i = c * kThreads + t;
            if (4 * i < d) reinterpret_cast<float4 *>(normed + (size_t)r * d)[i] = y[c];
        }
        return;
    }
    float mx;
    if constexpr (FORM == 2) {
        mx = stats[2 * (size_t)r + 1];
    } else {
        mx = 0.0f;
        for (int i = t; i < rows; i += kThreads) mx = fmaxf(mx, stats[2 * (size_t)i + 1]);
        mx = block_max(mx, red);
    }
    const float scale = scale_of(mx);
    const float inv = __fdiv_rn(1.0f, scale);
    if (t == 0 && (FORM == 2 || r == 0)) scales[FORM == 2 ? r : 0] = scale;
#pragma unroll
    for (int c = 0; c < NV; ++c) {
        const size_t kk = 4 * (size_t)(c * kThreads + t);
        if (kk < (size_t)d) {
            const int packed = ((int)round_clamp_i8(y[c].x * inv) & 255) |
                               (((int)round_clamp_i8(y[c].y * inv) & 255) << 8) |
                               (((int)round_clamp_i8(y[c].z * inv) & 255) << 16) |
                               ((int)round_clamp_i8(y[c].w * inv) << 24);
            const size_t pos = FORM == 0 ? gemm_pack_offset(r, kk, mg)
                                         : (size_t)r * ld + row_pos(kk, FORM == 2);
            *reinterpret_cast<int *>(q + pos) = packed;
        }
    }
    for (size_t kk = (size_t)d + 4 * t; kk < ld; kk += 4 * kThreads) {  // zero padding
        const size_t pos = FORM == 0 ? gemm_pack_offset(r, kk, mg)
                                     : (size_t)r * ld + row_pos(kk, FORM == 2);
        *reinterpret_cast<int *>(q + pos) = 0;
    }
}

}  // namespace

mri_status launch_norm_quant(int form, const float *x, const float *w, const float *stats,
                             size_t rows, size_t d, size_t ld, int8_t *q, float *scales,
                             float *normed, hipStream_t s) {
    if (!rows) return MRI_OK;
    if (d % 4 || d > 8192 || (form != 3 && (ld < d || ld % 4)))
        return set_error(MRI_ERR_INVALID_ARGUMENT, "norm quant: unsupported row shape");
    const size_t mg = gemm_row_groups(rows);
    const dim3 g((unsigned)(form == 0 ? mg * 32 : rows)), b(kThreads);
    auto go = [&](auto nv) {
        constexpr int NV = decltype(nv)::value;
        switch (form) {
        case 0: hipLaunchKernelGGL((k_norm_quant<NV, 0>), g, b, 0, s, x, w, stats, (int)rows, (int)d, ld, mg, q, scales, normed); break;
        case 1: hipLaunchKernelGGL((k_norm_quant<NV, 1>), g, b, 0, s, x, w, stats, (int)rows, (int)d, ld, mg, q, scales, normed); break;
        case 2: hipLaunchKernelGGL((k_norm_quant<NV, 2>), g, b, 0, s, x, w, stats, (int)rows, (int)d, ld, mg, q, scales, normed); break;
        default: hipLaunchKernelGGL((k_norm_quant<NV, 3>), g, b, 0, s, x, w, stats, (int)rows, (int)d, ld, mg, q, scales, normed); break;
        }
    };
    if (d <= 1024) go(std::integral_constant<int, 1>{});
    else if (d <= 2048) go(std::integral_constant<int, 2>{});
    else if (d <= 4096) go(std::integral_constant<int, 4>{});
    else go(std::integral_constant<int, 8>{});
    MRI_LAUNCHED("k_norm_quant");
    return MRI_OK;
}

mri_status launch_pack_gemm(const int8_t *src, size_t m, size_t k, size_t ld, size_t kp,
                            int8_t *packed, hipStream_t s) {
    const size_t mg = gemm_row_groups(m);
    hipLaunchKernelGGL(k_pack_gemm, dim3(grid_for(mg * 32 * kp / 16)), dim3(kThreads), 0, s,
                       src, m, k, ld, mg, kp, packed);
    MRI_LAUNCHED("k_pack_gemm");
    return MRI_OK;
}

mri_status launch_quantize_rows(const float *x, size_t m, size_t k,
                                size_t ld_out, bool q8_perm_layout,
                                int8_t *q_pad, int8_t *q_plain,
                                float *scales, hipStream_t s) {
    if (m == 0) return MRI_OK;
    launch_rows<false>(x, m, k, q_pad ? ld_out : k, q8_perm_layout ? 1 : 0, q_pad, q_plain,
                       scales, s);
    MRI_LAUNCHED("k_quantize_rows");
    return MRI_OK;
}

mri_status launch_swiglu_quantize_rows(const float *gu, size_t m, size_t k, size_t ld_out,
                                       bool q8_perm_layout, int8_t *q_pad, float *scales,
                                       hipStream_t s) {
    if (m == 0) return MRI_OK;
    launch_rows<true>(gu, m, k, ld_out, q8_perm_layout ? 1 : 0, q_pad, nullptr, scales, s);
    MRI_LAUNCHED("k_quantize_rows(swiglu)");
    return MRI_OK;
}

mri_status launch_quantize_per_channel(const float *w, size_t n, size_t k,
                                       int8_t *data, float *scales,
                                       hipStream_t s) {
    if (n == 0) return MRI_OK;
    launch_rows<false>(w, n, k, k, 0, data, nullptr, scales, s);
    MRI_LAUNCHED("k_quantize_rows(per_channel)");
    return MRI_OK;
}

mri_status launch_pad_rows(const int8_t *src, size_t m, size_t k, size_t kp,
                           int8_t *dst, hipStream_t s) {
    if (m * kp == 0) return MRI_OK;
    hipLaunchKernelGGL(k_pad_rows, dim3(grid_for(m * kp, 4)), dim3(kThreads), 0,
                       s, src, m, k, kp, dst);
    MRI_LAUNCHED("k_pad_rows");
    return MRI_OK;
}

mri_status launch_dot_i8(const int8_t *a, const int8_t *b, size_t n,
                         int32_t *out, hipStream_t s) {
    hipLaunchKernelGGL(k_dot_i8, dim3(1), dim3(kThreads), 0, s, a, b, n, out);
    MRI_LAUNCHED("k_dot_i8");
    return MRI_OK;
}

}  // namespace mri
