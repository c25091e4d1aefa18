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
// Mapping: one wave per weight row, two lanes per block (8 quant bytes =
// 16 elements each); a step covers 32 blocks, so K = 4096 takes 4 steps.
// Raw blocks are 18 bytes (2-byte aligned), so the row is read with 16-bit
// loads; the loads of consecutive lanes are contiguous.
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
                const uint16_t *qs = blk + 1 + half * 4;
                const unsigned w0 = (unsigned)qs[0] | ((unsigned)qs[1] << 16);
                const unsigned w1 = (unsigned)qs[2] | ((unsigned)qs[3] << 16);
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
                const float s = nib_dot(w0, w1, xe);
                acc = fmaf(d, fmaf(-8.0f, xs, s), acc);
            }
            for (int o = 32; o > 0; o >>= 1) acc += __shfl_xor(acc, o);
            if (lane == 0) out[(size_t)m * N + n] = acc;
        }
    }
}

}  // namespace

mri_status launch_q4_0_dequant(const float *x, size_t m, size_t k,
                               const uint8_t *w, size_t n_out, float *out,
                               hipStream_t s) {
    if (m == 0 || n_out == 0) return MRI_OK;
    const size_t waves = (n_out + kRowsPerWave - 1) / kRowsPerWave;
    size_t grid = (waves + (kThreads / 64) - 1) / (kThreads / 64);
    if (grid < 1) grid = 1;
    if (grid > 65535) grid = 65535;
    hipLaunchKernelGGL(k_q4_0_dequant, dim3((unsigned)grid), dim3(kThreads), 0, s,
                       x, (int)m, (int)k, reinterpret_cast<const uint16_t *>(w),
                       (int)n_out, out);
    MRI_LAUNCHED("k_q4_0_dequant");
    return MRI_OK;
}

}  // namespace mri
