// hbm_read.hip — a plain streaming read of device memory, the measured
// ceiling of a one-kernel HBM read at a given size (a diagnostic for the
// benchmark: the decode GEMVs are bounded by it, not by the datasheet peak).
#include <algorithm>

#include "common.hpp"

namespace mri {
namespace {

typedef int v4i __attribute__((ext_vector_type(4)));

// Each wave reads one contiguous 4 KiB chunk (four 16-byte non-temporal
// loads per lane, all issued before any use); the values are folded into
// one word that is stored only if it equals a value the data never produce
// in practice, so the loads cannot be dropped.  Measured on MI355X over 48 MB
// (9 rotated copies): 8.16 us, against 8.2-8.7 us for 8-16 KiB per wave,
// 10.1 us for 32 KiB, 8.2-8.9 us for persistent waves looping over 4 KiB
// chunks, and 8.8 us for a grid-stride loop of single loads.
__global__ __launch_bounds__(256) void k_hbm_read(const v4i *__restrict__ p, size_t n16,
                                                  int *__restrict__ sink) {
    const int l = threadIdx.x & 63;
    const size_t base = ((size_t)blockIdx.x * 4 + (threadIdx.x >> 6)) * 256;
    int acc = 0;
    if (base + 256 <= n16) {
        v4i r[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) r[u] = __builtin_nontemporal_load(p + base + u * 64 + l);
#pragma unroll
        for (int u = 0; u < 4; ++u) acc ^= r[u].x ^ r[u].w;
    } else {
        for (size_t i = base + l; i < n16; i += 64) acc ^= p[i].x;
    }
    if (acc == 0x5a5a5a5a && sink) *sink = acc;
}

}  // namespace

mri_status launch_hbm_read(const void *p, size_t bytes, int32_t *sink, hipStream_t s) {
    const size_t n16 = bytes / 16;
    if (n16 == 0) return MRI_OK;
    const size_t waves = (n16 + 255) / 256;  // one 4 KiB chunk per wave
    if ((waves + 3) / 4 > 0x7fffffff) return set_error(MRI_ERR_UNSUPPORTED, "hbm_read: too large");
    const unsigned grid = (unsigned)((waves + 3) / 4);
    hipLaunchKernelGGL(k_hbm_read, dim3(grid), dim3(256), 0, s, static_cast<const v4i *>(p), n16,
                       reinterpret_cast<int *>(sink));
    MRI_LAUNCHED("k_hbm_read");
    return MRI_OK;
}

}  // namespace mri

namespace mri {
namespace {

typedef int v16i __attribute__((ext_vector_type(16)));

// The int8 MFMA ceiling with operands of real data: every wave loads its
// operands once from `src` (random int8 from the caller), then runs `iters`
// rounds of 8 v_mfma_i32_32x32x32_i8 on 4 independent accumulators (two
// waves per SIMD, the configuration that keeps the pipe fullest) with no
// memory traffic, and folds the accumulators into one word that is stored
// only in a case that does not occur.
__global__ __launch_bounds__(512) void k_mfma_peak(const v4i *__restrict__ src, int iters,
                                                   int *__restrict__ sink) {
    const int l = threadIdx.x & 63, wv = threadIdx.x >> 6;
    v4i a[2], b[2];
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        a[i] = src[(wv * 4 + i) * 64 + l];
        b[i] = src[(wv * 4 + 2 + i) * 64 + l];
    }
    v16i acc[4] = {};
    for (int it = 0; it < iters; ++it) {
#pragma unroll
        for (int h = 0; h < 2; ++h)
#pragma unroll
            for (int q = 0; q < 4; ++q)
                acc[q] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a[(q >> 1) ^ h], b[(q & 1) ^ h],
                                                               acc[q], 0, 0, 0);
    }
    int s = 0;
#pragma unroll
    for (int q = 0; q < 4; ++q)
#pragma unroll
        for (int r = 0; r < 16; ++r) s ^= acc[q][r];
    if (s == 0x5a5a5a5a && sink) *sink = s;
}

}  // namespace

mri_status launch_mfma_peak(const int8_t *src, int iters, int32_t *sink, hipStream_t s) {
    const int cus = device_cus();
    hipLaunchKernelGGL(k_mfma_peak, dim3((unsigned)(cus > 0 ? cus : 256)), dim3(512), 0, s,
                       reinterpret_cast<const v4i *>(src), iters, reinterpret_cast<int *>(sink));
    MRI_LAUNCHED("k_mfma_peak");
    return MRI_OK;
}

}  // namespace mri
