// skinny.hip — decode-shaped (M <= 32) quantized matmul on CDNA4 MFMA.
//
// The weight stream dominates (M*K activation bytes vs N*K weight bytes), so
// the kernel is built around streaming the 1 KiB weight chunks of one
// 16-row tile per wave with deep software prefetch:
//   * one wave (= one workgroup) per tile of 16 output channels, all of K;
//   * per chunk (64 k): one 16-byte global load per lane for the weights and
//     one 16-byte read per 16-row activation tile;
//   * per-channel INT8: v_mfma_i32_16x16x64_i8 accumulates exact int32 dot
//     products for 16 (m) x 16 (n) outputs; the f32 epilogue
//     ((f32)acc * s_a) * s_w runs once at the end (int8.rs:93);
//   * Q8_0: one v_mfma_i32_16x16x32_i8 per 32-element block gives the exact
//     per-block int32 dot; each lane then applies ((f32)dot * s_a[m]) * d[n,b]
//     and adds it to its running f32 sum in block order — the order of
//     q8_direct.rs:269-282, so the f32 result is bit-identical.
// MFMA output mapping (16x16 family): lane l, register i holds row
// (activation) m = 4*(l/16) + i and column (weight row) n = l % 16.
//
// This is the general M <= 32 path (one wave per tile, activations read from
// a quantized [M][kp] buffer).  The M <= 4 decode case uses the K-split
// kernels of gemv.hip instead.
#include <type_traits>

#include "common.hpp"

namespace mri {
namespace {

typedef int v4i __attribute__((ext_vector_type(4)));

constexpr int kWave = 64;

__device__ inline long lo8(const v4i &v) {
    return (long)(((unsigned long)(unsigned)v.y << 32) | (unsigned)v.x);
}
__device__ inline long hi8(const v4i &v) {
    return (long)(((unsigned long)(unsigned)v.w << 32) | (unsigned)v.z);
}

// ---------------------------------------------------------------------------
// Per-channel INT8.  MT activation tiles of 16 rows; NI = output registers
// per lane that can hold a valid row (M <= 4 uses only lane group 0).
// ---------------------------------------------------------------------------
template <int MT, int NI, int U>
__global__ __launch_bounds__(kWave) void k_skinny_int8(
    const int8_t *__restrict__ act, int M, size_t kp,
    const float *__restrict__ sa_ptr, int sa_stride, float sa_value,
    const v4i *__restrict__ tiles, const float *__restrict__ wscales, int N,
    int P, float *__restrict__ out, int32_t *__restrict__ acc_out) {
    const int T = blockIdx.x;
    const int l = threadIdx.x;
    const int r = l & 15, g = l >> 4;
    const size_t pitch = (size_t)gridDim.x * kWave;  // slab-major chunks
    const v4i *wp = tiles + (size_t)T * kWave + l;
    const v4i *ap[MT];
    bool aval[MT];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
        const int m = mt * 16 + r;
        aval[mt] = m < M;
        ap[mt] = reinterpret_cast<const v4i *>(act + (size_t)(aval[mt] ? m : 0) * kp) + g;
    }
    const v4i zero = {0, 0, 0, 0};
    v4i acc[MT];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) acc[mt] = zero;

    v4i wb[2][U];
    v4i ab[2][MT][U];

    // Weight loads are unconditional (the chunk index is clamped to the last
    // one) and rows m >= M are zeroed at use, so the compiler never has to
    // wait for an older load before a conditional write to the same registers.
    auto load_w = [&](int buf, int p0) __attribute__((always_inline)) {
#pragma unroll
        for (int u = 0; u < U; ++u)
            wb[buf][u] = __builtin_nontemporal_load(wp + (size_t)min(p0 + u, P - 1) * pitch);
    };
    auto load_a = [&](int buf, int p0) __attribute__((always_inline)) {
#pragma unroll
        for (int u = 0; u < U; ++u)
#pragma unroll
            for (int mt = 0; mt < MT; ++mt)
                ab[buf][mt][u] = ap[mt][(size_t)min(p0 + u, P - 1) * 4];
    };
    // GUARD: only the last groups can run past P.
    auto compute = [&](int buf, int p0, auto guard) __attribute__((always_inline)) {
#pragma unroll
        for (int u = 0; u < U; ++u) {
            if (!decltype(guard)::value || p0 + u < P) {
#pragma unroll
                for (int mt = 0; mt < MT; ++mt) {
                    const v4i a = aval[mt] ? ab[buf][mt][u] : zero;
                    acc[mt] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a, wb[buf][u], acc[mt],
                                                                    0, 0, 0);
                }
            }
        }
    };

    load_w(0, 0);
    load_a(0, 0);

    // Two register buffers: while one group of U chunks is consumed the next
    // group's loads are in flight.  sched_barrier keeps the phases in this
    // order so the waits before each compute phase stay partial.
    const int p_full = P - P % (2 * U);
    int p0 = 0;
    for (; p0 < p_full; p0 += 2 * U) {
        load_w(1, p0 + U);
        load_a(1, p0 + U);
        __builtin_amdgcn_sched_barrier(0);
        compute(0, p0, std::false_type{});
        __builtin_amdgcn_sched_barrier(0);
        load_w(0, p0 + 2 * U);
        load_a(0, p0 + 2 * U);
        __builtin_amdgcn_sched_barrier(0);
        compute(1, p0 + U, std::false_type{});
        __builtin_amdgcn_sched_barrier(0);
    }
    if (p0 < P) {
        load_w(1, p0 + U);
        load_a(1, p0 + U);
        __builtin_amdgcn_sched_barrier(0);
        compute(0, p0, std::true_type{});
        compute(1, p0 + U, std::true_type{});
    }

    const int n = T * 16 + r;
    if (n >= N) return;
    const float sw = wscales[n];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
#pragma unroll
        for (int i = 0; i < NI; ++i) {
            const int m = mt * 16 + 4 * g + i;
            if (m < M) {
                const float sa = sa_ptr ? sa_ptr[(size_t)m * sa_stride] : sa_value;
                float v = (float)acc[mt][i] * sa;
                v = v * sw;
                out[(size_t)m * N + n] = v;
                if (acc_out) acc_out[(size_t)m * N + n] = acc[mt][i];
            }
        }
    }
}

// ---------------------------------------------------------------------------
// Q8_0.  U must be a multiple of 4: one 16-byte scale load covers 8 blocks
// = 4 chunks of the lane's weight row.
// ---------------------------------------------------------------------------
template <int MT, int NI, int U>
__global__ __launch_bounds__(kWave) void k_skinny_q8_0(
    const int8_t *__restrict__ act, int M, size_t kp,
    const float *__restrict__ sa_rows, const v4i *__restrict__ tiles,
    const v4i *__restrict__ qscales, int N, int P, int Q, int nb,
    float *__restrict__ out, int32_t *__restrict__ block_dots) {
    static_assert(U % 4 == 0, "U must cover whole scale groups");
    const int T = blockIdx.x;
    const int l = threadIdx.x;
    const int r = l & 15, g = l >> 4;
    const int Pe = (nb + 1) / 2;  // chunks holding real blocks
    const size_t pitch = (size_t)gridDim.x * kWave;   // slab-major chunks
    const size_t spitch = (size_t)gridDim.x * 16;     // slab-major scale groups
    const v4i *wp = tiles + (size_t)T * kWave + l;
    const v4i *sp = qscales + (size_t)T * 16 + r;
    const v4i *ap[MT];
    bool aval[MT];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
        const int m = mt * 16 + r;
        aval[mt] = m < M;
        ap[mt] = reinterpret_cast<const v4i *>(act + (size_t)(aval[mt] ? m : 0) * kp) + g;
    }
    const v4i zero = {0, 0, 0, 0};
    float fs[MT][NI];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int i = 0; i < NI; ++i) fs[mt][i] = 0.0f;

    v4i wb[2][U];
    v4i ab[2][MT][U];
    v4i sb[2][U / 4];
    const int n = T * 16 + r;
    const bool n_ok = n < N;

    auto load_w = [&](int buf, int p0) __attribute__((always_inline)) {
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int p = min(p0 + u, Pe - 1);
            wb[buf][u] = __builtin_nontemporal_load(wp + (size_t)p * pitch);
            if ((u & 3) == 0) sb[buf][u / 4] = sp[(size_t)(p / 4) * spitch];
        }
    };
    auto load_a = [&](int buf, int p0) __attribute__((always_inline)) {
#pragma unroll
        for (int u = 0; u < U; ++u)
#pragma unroll
            for (int mt = 0; mt < MT; ++mt)
                ab[buf][mt][u] = ap[mt][(size_t)min(p0 + u, Pe - 1) * 4];
    };

    float sa[MT][NI];
    // Phase 1 issues the 2U independent block MFMAs of a group; phase 2
    // applies the f32 epilogue and adds the terms in block order.
    auto compute = [&](int buf, int p0, auto guard) __attribute__((always_inline)) {
        constexpr bool G = decltype(guard)::value;
        v4i dots[U][2][MT];
#pragma unroll
        for (int u = 0; u < U; ++u)
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                const long wv = h ? hi8(wb[buf][u]) : lo8(wb[buf][u]);
#pragma unroll
                for (int mt = 0; mt < MT; ++mt) {
                    const v4i a = aval[mt] ? ab[buf][mt][u] : zero;
                    dots[u][h][mt] = __builtin_amdgcn_mfma_i32_16x16x32_i8(
                        h ? hi8(a) : lo8(a), wv, zero, 0, 0, 0);
                }
            }
#pragma unroll
        for (int u = 0; u < U; ++u) {
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                const int b = 2 * (p0 + u) + h;
                if (!G || b < nb) {
                    const int j = (2 * u + h) & 7;  // block within scale group
                    const unsigned word = (unsigned)sb[buf][u / 4][j >> 1];
                    const float d =
                        f16_bits_to_f32((j & 1) ? (word >> 16) : (word & 0xFFFFu));
#pragma unroll
                    for (int mt = 0; mt < MT; ++mt) {
#pragma unroll
                        for (int i = 0; i < NI; ++i) {
                            float t = (float)dots[u][h][mt][i] * sa[mt][i];
                            t = t * d;
                            fs[mt][i] = fs[mt][i] + t;
                        }
                        if (block_dots && n_ok) {
#pragma unroll
                            for (int i = 0; i < NI; ++i) {
                                const int m = mt * 16 + 4 * g + i;
                                if (m < M)
                                    block_dots[((size_t)m * N + n) * nb + b] =
                                        dots[u][h][mt][i];
                            }
                        }
                    }
                }
            }
        }
    };

#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int i = 0; i < NI; ++i) {
            const int m = mt * 16 + 4 * g + i;
            sa[mt][i] = m < M ? sa_rows[m] : 0.0f;
        }
    load_w(0, 0);
    load_a(0, 0);

    // Full groups (all 2U blocks real) run unguarded; the tail is guarded.
    const int p_full =
        (nb % 2 == 0) ? Pe - Pe % (2 * U) : (Pe - 1) - (Pe - 1) % (2 * U);
    int p0 = 0;
    for (; p0 < p_full; p0 += 2 * U) {
        load_w(1, p0 + U);
        load_a(1, p0 + U);
        __builtin_amdgcn_sched_barrier(0);
        compute(0, p0, std::false_type{});
        __builtin_amdgcn_sched_barrier(0);
        load_w(0, p0 + 2 * U);
        load_a(0, p0 + 2 * U);
        __builtin_amdgcn_sched_barrier(0);
        compute(1, p0 + U, std::false_type{});
        __builtin_amdgcn_sched_barrier(0);
    }
    for (; p0 < Pe; p0 += U) {
        // tail: one group at a time from buffer 0
        __builtin_amdgcn_sched_barrier(0);
        compute(0, p0, std::true_type{});
        __builtin_amdgcn_sched_barrier(0);
        load_w(0, p0 + U);
        load_a(0, p0 + U);
    }

    if (!n_ok) return;
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int i = 0; i < NI; ++i) {
            const int m = mt * 16 + 4 * g + i;
            if (m < M) out[(size_t)m * N + n] = fs[mt][i];
        }
}

constexpr int kU = 8;

template <int MT, int NI, int U>
void launch_i8(const int8_t *act, size_t m, size_t kp, const float *sa_ptr,
               int sa_stride, float sa_value, const QMatrixDev &w, float *out,
               int32_t *acc_out, hipStream_t s) {
    hipLaunchKernelGGL((k_skinny_int8<MT, NI, U>), dim3((unsigned)w.n_tiles),
                       dim3(kWave), 0, s, act, (int)m, kp, sa_ptr, sa_stride,
                       sa_value, reinterpret_cast<const v4i *>(w.tiles), w.scales,
                       (int)w.n_out, (int)(w.kp / kChunkK), out, acc_out);
}

template <int MT, int NI, int U>
void launch_q8(const int8_t *act, size_t m, size_t kp, const float *sa_rows,
               const Q8MatrixDev &w, float *out, int32_t *block_dots, hipStream_t s) {
    hipLaunchKernelGGL((k_skinny_q8_0<MT, NI, U>), dim3((unsigned)w.n_tiles),
                       dim3(kWave), 0, s, act, (int)m, kp, sa_rows,
                       reinterpret_cast<const v4i *>(w.tiles),
                       reinterpret_cast<const v4i *>(w.scales), (int)w.n_out,
                       (int)(w.kp / kChunkK), (int)(w.kp / (kQK * kQ8ScaleGroup)),
                       (int)w.n_blocks, out, block_dots);
}

}  // namespace

mri_status launch_skinny_int8(const int8_t *act, size_t m, const float *sa_ptr,
                              int sa_stride, float sa_value,
                              const QMatrixDev &w, float *out,
                              int32_t *acc_out, hipStream_t s) {
    if (w.n_tiles == 0 || m == 0) return MRI_OK;
    const size_t kp = w.kp;
    for (size_t m0 = 0; m0 < m; m0 += 32) {
        const size_t mc = m - m0 < 32 ? m - m0 : 32;
        const int8_t *a = act + m0 * kp;
        const float *sp = sa_ptr ? sa_ptr + m0 * (size_t)sa_stride : nullptr;
        float *o = out + m0 * w.n_out;
        int32_t *ao = acc_out ? acc_out + m0 * w.n_out : nullptr;
        if (mc <= 16) launch_i8<1, 4, kU>(a, mc, kp, sp, sa_stride, sa_value, w, o, ao, s);
        else launch_i8<2, 4, kU>(a, mc, kp, sp, sa_stride, sa_value, w, o, ao, s);
        MRI_LAUNCHED("k_skinny_int8");
    }
    return MRI_OK;
}

mri_status launch_skinny_q8_0(const int8_t *act, size_t m,
                              const float *sa_rows, const Q8MatrixDev &w,
                              float *out, int32_t *block_dots,
                              hipStream_t s) {
    if (w.n_tiles == 0 || m == 0) return MRI_OK;
    const size_t kp = w.kp;
    for (size_t m0 = 0; m0 < m; m0 += 32) {
        const size_t mc = m - m0 < 32 ? m - m0 : 32;
        const int8_t *a = act + m0 * kp;
        const float *sp = sa_rows + m0;
        float *o = out + m0 * w.n_out;
        int32_t *bd = block_dots ? block_dots + m0 * w.n_out * w.n_blocks : nullptr;
        if (mc <= 16) launch_q8<1, 4, kU>(a, mc, kp, sp, w, o, bd, s);
        else launch_q8<2, 4, 4>(a, mc, kp, sp, w, o, bd, s);
        MRI_LAUNCHED("k_skinny_q8_0");
    }
    return MRI_OK;
}

}  // namespace mri
