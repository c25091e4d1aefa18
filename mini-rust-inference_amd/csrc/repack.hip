// repack.hip — one-time weight upload transforms into the slab-major MFMA
// chunk layouts described in common.hpp.  Run once per weight handle, off the hot path.
#include "common.hpp"

namespace mri {
namespace {

constexpr int kThreads = 256;

// One thread per 16-byte lane piece of the per-channel INT8 tiles.
__global__ __launch_bounds__(kThreads) void k_repack_int8(
    const int8_t *__restrict__ data, size_t n, size_t k, size_t n_tiles,
    size_t P, int8_t *__restrict__ tiles) {
    const size_t total = n_tiles * P * 64;
    const size_t stride = (size_t)gridDim.x * blockDim.x;
    for (size_t e = (size_t)blockIdx.x * blockDim.x + threadIdx.x; e < total;
         e += stride) {
        const size_t lane = e & 63, pt = e >> 6;
        const size_t p = pt / n_tiles, T = pt - p * n_tiles;
        const size_t row = T * kTileN + (lane & 15);
        const size_t k0 = p * kChunkK + (lane >> 4) * 16;
        int8_t v[16];
#pragma unroll
        for (int j = 0; j < 16; ++j)
            v[j] = (row < n && k0 + j < k) ? data[row * k + k0 + j] : (int8_t)0;
        int8_t *dst = tiles + e * 16;
#pragma unroll
        for (int j = 0; j < 16; ++j) dst[j] = v[j];
    }
}

__global__ __launch_bounds__(kThreads) void k_pad_scales(
    const float *__restrict__ scales, size_t n, size_t np,
    float *__restrict__ out) {
    size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < np) out[i] = i < n ? scales[i] : 0.0f;
}

// One thread per 16-byte lane piece of the Q8_0 quants, enumerated in the
// order of the lap blocks: piece e = (lap block, chunk c, lane).
__global__ __launch_bounds__(kThreads) void k_repack_q8_quants(
    const uint8_t *__restrict__ raw, size_t n, size_t nb, size_t G, size_t total,
    int8_t *__restrict__ laps) {
    const size_t stride = (size_t)gridDim.x * blockDim.x;
    for (size_t e = (size_t)blockIdx.x * blockDim.x + threadIdx.x; e < total;
         e += stride) {
        const size_t lane = e & 63, c = (e >> 6) & 3, lb = e >> 8;
        const size_t T = lb / G, q = lb - T * G;
        const size_t p = 4 * q + c;
        const size_t row = T * kTileN + (lane & 15);
        const size_t g = lane >> 4;
        int8_t *dst = laps + lb * kQ8LapBytes + (c * 64 + lane) * 16;
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const size_t b = 2 * p + h;
            const bool ok = row < n && b < nb;
            const uint8_t *src = raw + (row * nb + b) * kQ8Bytes + 2 + g * 8;
#pragma unroll
            for (int j = 0; j < 8; ++j)
                dst[h * 8 + j] = ok ? (int8_t)src[j] : (int8_t)0;
        }
    }
}

// One thread per (lap block, row): the row's 8 f16 scales of the lap
// (raw blocks of block_bytes, lap blocks of lap_bytes, scales at scale_off).
__global__ __launch_bounds__(kThreads) void k_repack_scales(
    const uint8_t *__restrict__ raw, size_t n, size_t nb, size_t G, size_t total,
    int block_bytes, int lap_bytes, int scale_off, int8_t *__restrict__ laps) {
    const size_t stride = (size_t)gridDim.x * blockDim.x;
    for (size_t e = (size_t)blockIdx.x * blockDim.x + threadIdx.x; e < total;
         e += stride) {
        const size_t r = e & 15, lb = e >> 4;
        const size_t T = lb / G, q = lb - T * G;
        const size_t row = T * kTileN + r;
        uint16_t *dst =
            reinterpret_cast<uint16_t *>(laps + lb * lap_bytes + scale_off + r * 16);
#pragma unroll
        for (int j = 0; j < kQ8ScaleGroup; ++j) {
            const size_t b = q * kQ8ScaleGroup + j;
            uint16_t d = 0;
            if (row < n && b < nb) {
                const uint8_t *src = raw + (row * nb + b) * block_bytes;
                d = (uint16_t)(src[0] | (src[1] << 8));
            }
            dst[j] = d;
        }
    }
}

// One thread per 16-byte quant piece of the W4A8 lap blocks: piece
// e = (lap block, u, lane).  Word 2c' + h of the piece holds block
// b = 2p + h, p = 4q + 2u + c': byte i = element 8g + i (low nibble) and
// element 8g + 4 + i (high nibble), each as raw nibble ^ 8.  Missing rows
// and blocks past nb are quant 0 (stored 0).
__global__ __launch_bounds__(kThreads) void k_repack_q4_quants(
    const uint8_t *__restrict__ raw, size_t n, size_t nb, size_t G, size_t total,
    int ggml, int8_t *__restrict__ laps) {
    const size_t stride = (size_t)gridDim.x * blockDim.x;
    for (size_t e = (size_t)blockIdx.x * blockDim.x + threadIdx.x; e < total;
         e += stride) {
        const size_t lane = e & 63, u = (e >> 6) & 1, lb = e >> 7;
        const size_t T = lb / G, q = lb - T * G;
        const size_t row = T * kTileN + (lane & 15);
        const int g = (int)(lane >> 4);
        uint32_t words[4];
#pragma unroll
        for (int wd = 0; wd < 4; ++wd) {
            const size_t p = 4 * q + 2 * u + (wd >> 1);
            const size_t b = 2 * p + (wd & 1);
            uint32_t v = 0;
            if (row < n && b < nb) {
                const uint8_t *qs = raw + (row * nb + b) * kQ4Bytes + 2;
                auto nib = [&](int el) -> uint32_t {  // raw nibble of element el
                    const int byte = ggml ? (el & 15) : (el >> 1);
                    const int hi = ggml ? (el >> 4) : (el & 1);
                    return (uint32_t)((qs[byte] >> (4 * hi)) & 0x0F);
                };
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const uint32_t lo = nib(8 * g + i) ^ 8u, hi = nib(8 * g + 4 + i) ^ 8u;
                    v |= (lo | (hi << 4)) << (8 * i);
                }
            }
            words[wd] = v;
        }
        uint32_t *dst = reinterpret_cast<uint32_t *>(laps + lb * kQ4LapBytes + (u * 64 + lane) * 16);
#pragma unroll
        for (int wd = 0; wd < 4; ++wd) dst[wd] = words[wd];
    }
}

inline int grid_for(size_t n) {
    size_t g = (n + kThreads - 1) / kThreads;
    if (g < 1) g = 1;
    if (g > 8192) g = 8192;
    return (int)g;
}

}  // namespace

mri_status launch_repack_int8(const int8_t *data, const float *scales,
                              QMatrixDev &w, hipStream_t s) {
    const size_t P = w.kp / kChunkK;
    const size_t pieces = w.n_tiles * P * 64;
    if (pieces) {
        hipLaunchKernelGGL(k_repack_int8, dim3(grid_for(pieces)), dim3(kThreads),
                           0, s, data, w.n_out, w.k_in, w.n_tiles, P, w.tiles);
        MRI_LAUNCHED("k_repack_int8");
    }
    const size_t np = w.n_tiles * kTileN;
    if (np) {
        hipLaunchKernelGGL(k_pad_scales, dim3(grid_for(np)), dim3(kThreads), 0, s,
                           scales, w.n_out, np, w.scales);
        MRI_LAUNCHED("k_pad_scales");
    }
    return MRI_OK;
}

mri_status launch_repack_q8_0(const uint8_t *raw, Q8MatrixDev &w,
                              hipStream_t s) {
    const size_t G = w.laps_per_tile();
    const size_t pieces = w.n_tiles * G * 256;
    if (pieces) {
        hipLaunchKernelGGL(k_repack_q8_quants, dim3(grid_for(pieces)),
                           dim3(kThreads), 0, s, raw, w.n_out, w.n_blocks, G, pieces,
                           w.laps);
        MRI_LAUNCHED("k_repack_q8_quants");
        const size_t rows = w.n_tiles * G * kTileN;
        hipLaunchKernelGGL(k_repack_scales, dim3(grid_for(rows)), dim3(kThreads), 0, s,
                           raw, w.n_out, w.n_blocks, G, rows, kQ8Bytes, kQ8LapBytes, 4096,
                           w.laps);
        MRI_LAUNCHED("k_repack_scales");
    }
    return MRI_OK;
}

mri_status launch_repack_q4_0(const uint8_t *raw, bool ggml_order, Q8MatrixDev &w,
                              hipStream_t s) {
    const size_t G = w.laps_per_tile();
    const size_t pieces = w.n_tiles * G * 128;
    if (pieces) {
        hipLaunchKernelGGL(k_repack_q4_quants, dim3(grid_for(pieces)), dim3(kThreads), 0, s,
                           raw, w.n_out, w.n_blocks, G, pieces, ggml_order ? 1 : 0, w.laps);
        MRI_LAUNCHED("k_repack_q4_quants");
        const size_t rows = w.n_tiles * G * kTileN;
        hipLaunchKernelGGL(k_repack_scales, dim3(grid_for(rows)), dim3(kThreads), 0, s,
                           raw, w.n_out, w.n_blocks, G, rows, kQ4Bytes, kQ4LapBytes, 2048,
                           w.laps);
        MRI_LAUNCHED("k_repack_scales");
    }
    return MRI_OK;
}

}  // namespace mri
