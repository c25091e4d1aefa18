// q4_0.hip — W4A32 Q4_0 GEMV/GEMM on raw GGUF Q4_0 bytes
// (matmul_q4_0_dequant, ops/matmul/q4_0.rs:94-181).
//
// The reference dequantizes each block (w = d * (nibble - 8), interleaved
// nibble order: element 2i = low nibble of byte i, 2i+1 = high nibble,
// q4_0.rs:59-68) and accumulates x*w in f32 over K.  Here the dequantization
// happens in registers and the sum is regrouped per block:
//   sum_b d_b * (sum_e x_e * nib_e - 8 * sum_e x_e)
// which differs from the sequential sum only by rounding (the documented
// 1e-5 * max(|ref|, sum|terms|) contract).
//
// Two forms.
//
// k_q4_0_lds (16-byte aligned weights, K % 256 == 0, so that every row
// starts on 16 bytes; M <= 4): a workgroup takes R consecutive weight rows,
// one contiguous byte range, and moves them to LDS with 16-byte loads (all
// in flight at once); the activations are read from L2.  Lane l of a step
// covers elements 8*(l%4) .. +8 of block l/4 (4 quant
// bytes: low nibble = even element): it reads its 8 activations once and
// applies them to each of the wave's R/4 rows as d * (sum x*nib - 8 * sum x)
// (the regrouping below; the activation sum is shared by the rows).  Lane
// partials are added by a wave reduction.
//
// k_q4_0_dequant (any 2-byte aligned layout): one wave per weight row, two
// lanes per block (16 elements each), with the sum regrouped per block as
// sum_b d_b * (sum_e x_e * nib_e - 8 * sum_e x_e).
//
// GG (an option without a reference counterpart): upstream GGML's nibble
// order, element i = low nibble of byte i and element i + 16 = its high
// nibble (llama.cpp Q4_0 files); the lanes then read the bytes of their
// elements and take one nibble of each.
#include <algorithm>

#include "common.hpp"

namespace mri {
namespace {

constexpr int kThreads = 256;
constexpr int kRowsPerWave = 4;


// 8 quant bytes (two u32 words) against 16 activations: returns
// sum_e x_e * nib_e for the interleaved order.
__device__ inline float nib_dot(unsigned w0, unsigned w1, const float *x) {
    float s = 0.0f;
    const unsigned lo0 = w0 & 0x0F0F0F0Fu, hi0 = (w0 >> 4) & 0x0F0F0F0Fu;
    const unsigned lo1 = w1 & 0x0F0F0F0Fu, hi1 = (w1 >> 4) & 0x0F0F0F0Fu;
    s = fmaf(x[0], (float)(lo0 & 0xFF), s);
    s = fmaf(x[1], (float)(hi0 & 0xFF), s);
    s = fmaf(x[2], (float)((lo0 >> 8) & 0xFF), s);
    s = fmaf(x[3], (float)((hi0 >> 8) & 0xFF), s);
    s = fmaf(x[4], (float)((lo0 >> 16) & 0xFF), s);
    s = fmaf(x[5], (float)((hi0 >> 16) & 0xFF), s);
    s = fmaf(x[6], (float)(lo0 >> 24), s);
    s = fmaf(x[7], (float)(hi0 >> 24), s);
    s = fmaf(x[8], (float)(lo1 & 0xFF), s);
    s = fmaf(x[9], (float)(hi1 & 0xFF), s);
    s = fmaf(x[10], (float)((lo1 >> 8) & 0xFF), s);
    s = fmaf(x[11], (float)((hi1 >> 8) & 0xFF), s);
    s = fmaf(x[12], (float)((lo1 >> 16) & 0xFF), s);
    s = fmaf(x[13], (float)((hi1 >> 16) & 0xFF), s);
    s = fmaf(x[14], (float)(lo1 >> 24), s);
    s = fmaf(x[15], (float)(hi1 >> 24), s);
    return s;
}

// 16 bytes (four u32 words) against 16 activations, GGML order: element e
// is nibble `shift` / 4 of byte e.
__device__ inline float nib_dot_ggml(const unsigned (&wd)[4], int shift, const float *x) {
    float s = 0.0f;
#pragma unroll
    for (int e = 0; e < 16; ++e)
        s = fmaf(x[e], (float)((wd[e >> 2] >> (8 * (e & 3) + shift)) & 0xFu), s);
    return s;
}

template <bool GG>
__global__ __launch_bounds__(kThreads) void k_q4_0_dequant(
    const float *__restrict__ x, int M, int K, const uint16_t *__restrict__ w,
    int N, float *__restrict__ out) {
    const int lane = threadIdx.x & 63;
    const int wave = (blockIdx.x * kThreads + threadIdx.x) >> 6;
    const int n_waves = (gridDim.x * kThreads) >> 6;
    const int nb = K / 32;
    const int half = lane & 1;
    const size_t row_u16 = (size_t)nb * (kQ4Bytes / 2);
    for (int n = wave; n < N; n += n_waves) {
        const uint16_t *row = w + (size_t)n * row_u16;
        for (int m = 0; m < M; ++m) {
            const float *xr = x + (size_t)m * K;
            float acc = 0.0f;
            for (int b = lane >> 1; b < nb; b += 32) {
                const uint16_t *blk = row + (size_t)b * (kQ4Bytes / 2);
                const float d = f16_bits_to_f32(blk[0]);
                const float4 *xv = reinterpret_cast<const float4 *>(xr + b * 32 + half * 16);
                float xe[16];
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const float4 v = xv[j];
                    xe[4 * j] = v.x;
                    xe[4 * j + 1] = v.y;
                    xe[4 * j + 2] = v.z;
                    xe[4 * j + 3] = v.w;
                }
                float xs = 0.0f;
#pragma unroll
                for (int j = 0; j < 16; ++j) xs += xe[j];
                float s;
                if constexpr (GG) {
                    // elements 16 half .. +15: nibble `half` of all 16 bytes
                    unsigned wd[4];
#pragma unroll
                    for (int i = 0; i < 4; ++i)
                        wd[i] = (unsigned)blk[1 + 2 * i] | ((unsigned)blk[2 + 2 * i] << 16);
                    s = nib_dot_ggml(wd, 4 * half, xe);
                } else {
                    const uint16_t *qs = blk + 1 + half * 4;
                    const unsigned w0 = (unsigned)qs[0] | ((unsigned)qs[1] << 16);
                    const unsigned w1 = (unsigned)qs[2] | ((unsigned)qs[3] << 16);
                    s = nib_dot(w0, w1, xe);
                }
                acc = fmaf(d, fmaf(-8.0f, xs, s), acc);
            }
            for (int o = 32; o > 0; o >>= 1) acc += __shfl_xor(acc, o);
            if (lane == 0) out[(size_t)m * N + n] = acc;
        }
    }
}

template <int R, bool GG>
__global__ __launch_bounds__(kThreads) void k_q4_0_lds(const float *__restrict__ x, int M, int K,
                                                       const uint8_t *__restrict__ w, int N,
                                                       float *__restrict__ out) {
    constexpr int RW = R / 4;  // rows per wave
    extern __shared__ int4 s_raw[];
    const int t = threadIdx.x, lane = t & 63, wv = t >> 6;
    const int nb = K / 32, row_bytes = nb * kQ4Bytes;
    const int n0 = blockIdx.x * R, rows = min(R, N - n0);
    const uint8_t *s_w = reinterpret_cast<const uint8_t *>(s_raw);
    {
        // every load in flight before the first store (at most 12 pieces a
        // thread: the launcher keeps R rows within 48 KiB; the pieces past
        // the rows re-read the last one, which measured faster than
        // skipping them under a branch: 11.8 against 21.3 us at N = 11008)
        const int4 *src = reinterpret_cast<const int4 *>(w + (size_t)n0 * row_bytes);
        const int n16 = rows * row_bytes / 16;
        int4 v[12];
#pragma unroll
        for (int u = 0; u < 12; ++u) v[u] = src[min(t + kThreads * u, n16 - 1)];  // n16 >= 1
#pragma unroll
        for (int u = 0; u < 12; ++u) {
            const int i = t + kThreads * u;
            if (i < n16) s_raw[i] = v[u];
        }
    }
    __syncthreads();
    const int steps = (nb * 4 + 63) / 64;
    // rows past `rows` read stale LDS and are never stored
    for (int m = 0; m < M; ++m) {
        const float *xm = x + (size_t)m * K;
        float acc[RW];
#pragma unroll
        for (int r = 0; r < RW; ++r) acc[r] = 0.0f;
        for (int st = 0; st < steps; ++st) {
            const int idx = st * 64 + lane, p = idx & 3;
            const bool ok = (idx >> 2) < nb;
            const int b = ok ? idx >> 2 : nb - 1;
            const float4 *xv = reinterpret_cast<const float4 *>(xm + 32 * b + 8 * p);
            float4 xa = xv[0], xb = xv[1];
            if (!ok) xa = xb = float4{0, 0, 0, 0};
            float dq[RW];
            unsigned lo[RW], hi[RW];
#pragma unroll
            for (int r = 0; r < RW; ++r) {
                const uint8_t *blk = s_w + (size_t)(wv * RW + r) * row_bytes + b * kQ4Bytes;
                dq[r] = f16_bits_to_f32(*reinterpret_cast<const uint16_t *>(blk));
                if constexpr (GG) {
                    // elements 8p .. 8p+7: nibble p / 2 of bytes 8 (p % 2) .. +7,
                    // regrouped into the (even, odd) element words below
                    const uint16_t *qs = reinterpret_cast<const uint16_t *>(blk + 2 + 8 * (p & 1));
                    const int sh = 4 * (p >> 1);
                    const unsigned a0 = ((unsigned)qs[0] | ((unsigned)qs[1] << 16)) >> sh;
                    const unsigned a1 = ((unsigned)qs[2] | ((unsigned)qs[3] << 16)) >> sh;
                    // a0 bytes = elements 0..3, a1 bytes = elements 4..7
                    const unsigned e0 = a0 & 0x0F0F0F0Fu, e1 = a1 & 0x0F0F0F0Fu;
                    lo[r] = (e0 & 0xFFu) | ((e0 >> 8) & 0xFF00u) | ((e1 << 16) & 0xFF0000u) |
                            ((e1 << 8) & 0xFF000000u);          // elements 0, 2, 4, 6
                    hi[r] = ((e0 >> 8) & 0xFFu) | ((e0 >> 16) & 0xFF00u) |
                            ((e1 << 8) & 0xFF0000u) | (e1 & 0xFF000000u);  // 1, 3, 5, 7
                } else {
                    const unsigned q =
                        (unsigned)*reinterpret_cast<const uint16_t *>(blk + 2 + 4 * p) |
                        ((unsigned)*reinterpret_cast<const uint16_t *>(blk + 4 + 4 * p) << 16);
                    lo[r] = q & 0x0F0F0F0Fu;          // elements 0, 2, 4, 6 (low nibbles)
                    hi[r] = (q >> 4) & 0x0F0F0F0Fu;   // elements 1, 3, 5, 7
                }
            }
            // d * sum_e x_e * (nib_e - 8) = d * (sum_e x_e * nib_e - 8 * sum_e x_e);
            // the activation sum is shared by the wave's rows, and the rows'
            // chains are interleaved
            const float xs = ((xa.x + xa.y) + (xa.z + xa.w)) + ((xb.x + xb.y) + (xb.z + xb.w));
            float sn[RW];
#pragma unroll
            for (int r = 0; r < RW; ++r) sn[r] = xa.x * (float)(lo[r] & 0xFF);
#pragma unroll
            for (int r = 0; r < RW; ++r) sn[r] = fmaf(xa.y, (float)(hi[r] & 0xFF), sn[r]);
#pragma unroll
            for (int r = 0; r < RW; ++r) sn[r] = fmaf(xa.z, (float)((lo[r] >> 8) & 0xFF), sn[r]);
#pragma unroll
            for (int r = 0; r < RW; ++r) sn[r] = fmaf(xa.w, (float)((hi[r] >> 8) & 0xFF), sn[r]);
#pragma unroll
            for (int r = 0; r < RW; ++r) sn[r] = fmaf(xb.x, (float)((lo[r] >> 16) & 0xFF), sn[r]);
#pragma unroll
            for (int r = 0; r < RW; ++r) sn[r] = fmaf(xb.y, (float)((hi[r] >> 16) & 0xFF), sn[r]);
#pragma unroll
            for (int r = 0; r < RW; ++r) sn[r] = fmaf(xb.z, (float)(lo[r] >> 24), sn[r]);
#pragma unroll
            for (int r = 0; r < RW; ++r) sn[r] = fmaf(xb.w, (float)(hi[r] >> 24), sn[r]);
#pragma unroll
            for (int r = 0; r < RW; ++r) acc[r] = fmaf(dq[r], fmaf(-8.0f, xs, sn[r]), acc[r]);
        }
#pragma unroll
        for (int r = 0; r < RW; ++r) {
            float v = acc[r];
            for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
            const int row = wv * RW + r;
            if (lane == 0 && row < rows) out[(size_t)m * N + n0 + row] = v;
        }
    }
}

size_t q4_lds_bytes(int r, size_t k) { return (size_t)r * (k / 32) * kQ4Bytes; }

template <int R, bool GG>
mri_status launch_lds(const float *x, size_t m, size_t k, const uint8_t *w, size_t n_out,
                      float *out, hipStream_t s) {
    static DeviceOnce attr;
    MRI_HIP(attr.run([](int) {
        return hipFuncSetAttribute(reinterpret_cast<const void *>(&k_q4_0_lds<R, GG>),
                                   hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);
    }));
    hipLaunchKernelGGL((k_q4_0_lds<R, GG>), dim3((unsigned)((n_out + R - 1) / R)),
                       dim3(kThreads), q4_lds_bytes(R, k), s, x, (int)m, (int)k, w, (int)n_out,
                       out);
    MRI_LAUNCHED("k_q4_0_lds");
    return MRI_OK;
}

template <bool GG>
mri_status launch_q4(const float *x, size_t m, size_t k, const uint8_t *w, size_t n_out,
                     float *out, hipStream_t s) {
    // the staged form: 16-byte aligned rows (K % 256 == 0) and operands, and
    // at most 64 KiB of LDS per workgroup (several workgroups per CU)
    const bool al = ((uintptr_t)w & 15) == 0 && ((uintptr_t)x & 15) == 0 && k % 256 == 0;
    if (al && m <= 4 && k <= (1u << 16) && n_out <= (1u << 30)) {
        // rows per workgroup: 8, or 4 where 8 rows exceed ~40 KiB of LDS.
        // Measured at K = 4096 (us per call): 8 rows 11.8 (N = 11008) and
        // 6.4 (N = 4096), against 13.1 and 8.4 for 16 rows and 12.7 and 6.4
        // for 4 (more workgroups per CU overlap one's loads with another's
        // arithmetic)
        if (q4_lds_bytes(8, k) <= 40 * 1024) return launch_lds<8, GG>(x, m, k, w, n_out, out, s);
        if (q4_lds_bytes(4, k) <= 48 * 1024) return launch_lds<4, GG>(x, m, k, w, n_out, out, s);
    }
    const size_t waves = (n_out + kRowsPerWave - 1) / kRowsPerWave;
    size_t grid = (waves + (kThreads / 64) - 1) / (kThreads / 64);
    if (grid < 1) grid = 1;
    if (grid > 65535) grid = 65535;
    hipLaunchKernelGGL((k_q4_0_dequant<GG>), dim3((unsigned)grid), dim3(kThreads), 0, s,
                       x, (int)m, (int)k, reinterpret_cast<const uint16_t *>(w),
                       (int)n_out, out);
    MRI_LAUNCHED("k_q4_0_dequant");
    return MRI_OK;
}

}  // namespace

mri_status launch_q4_0_dequant(const float *x, size_t m, size_t k, const uint8_t *w,
                               size_t n_out, bool ggml_order, float *out, hipStream_t s) {
    if (m == 0 || n_out == 0) return MRI_OK;
    return ggml_order ? launch_q4<true>(x, m, k, w, n_out, out, s)
                      : launch_q4<false>(x, m, k, w, n_out, out, s);
}

}  // namespace mri
