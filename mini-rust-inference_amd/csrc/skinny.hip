// skinny.hip — decode-shaped (5..32 rows per launch; larger M loops over
// 32-row slices) quantized matmul on CDNA4 MFMA.
//
// The weight stream dominates (M*K activation bytes vs N*K weight bytes), so
// both kernels stream the 1 KiB weight chunks of one 16-row tile per wave
// (INT8: slab-major chunks; Q8_0: the tile's lap blocks, quants and scales
// together), with the activation rows read from a quantized [M][kp] buffer:
//   * per-channel INT8: v_mfma_i32_16x16x64_i8 accumulates exact int32 dot
//     products for 16 (m) x 16 (n) outputs; the f32 epilogue
//     ((f32)acc * s_a) * s_w runs once at the end (int8.rs:93);
//   * Q8_0: one v_mfma_i32_16x16x32_i8 per 32-element block gives the exact
//     per-block int32 dot; each lane then applies ((f32)dot * s_a[m]) * d[n,b]
//     and adds it to its running f32 sum in block order — the order of
//     q8_direct.rs:269-282, so the f32 result is bit-identical.
// MFMA output mapping (16x16 family): lane l, register i holds row
// (activation) m = 4*(l/16) + i and column (weight row) n = l % 16.
// The M <= 4 decode case uses the K-split kernels of gemv_int8.hip and
// gemv_q8.hip instead.
#include <type_traits>

#include "gemv_common.hpp"

namespace mri {
using namespace gemv;
namespace {

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
// Q8_0, up to 32 rows: AG groups of 16 activation rows.  One wave per tile
// of 16 output channels sweeps all of K in laps of one scale group (4
// chunks = 8 blocks) and keeps RL laps of loads in flight: per chunk one
// 16-byte load of the weight chunk and, per activation group, one 16-byte
// load of the rows' matching activation bytes (chunk-permuted, so its two
// halves are the A operands of the chunk's two blocks).  Per block and
// group one v_mfma_i32_16x16x32_i8 gives the exact int32 dots of 16 rows x
// 16 channels; each lane then adds ((f32)dot * s_a[m]) * d[n,b] to its
// running sums in block order (q8_direct.rs:269-282), so the f32 result is
// bit-identical.  The sweep has no global memory instruction other than the
// ring's loads and no data-dependent branch, so every wait leaves the
// younger loads in flight.  Rows m >= M read row 0's activations; their
// results are never stored.
//
// W4 (Q4_0 weights of the W4A8 path): a lap's quants are two 16-byte pieces
// per lane; the 8-byte B operand of block h of chunk c is the u32 word
// 2(c % 2) + h of piece c / 2 with each nibble moved to the high half of its
// byte (16 * quant as int8), and the MFMA result is divided by 16 exactly.
// ---------------------------------------------------------------------------
template <int AG, int NT, int TPW, int RL, bool DEBUG, bool W4>
__global__ __launch_bounds__(TPW * kWave) void k_skinny_q8_0(
    const int8_t *__restrict__ act, int M, int kp, const float *__restrict__ sa_rows,
    const v4i *__restrict__ laps, int N, int n_tiles, int G, int nb, float *__restrict__ out,
    int32_t *__restrict__ block_dots, int ns) {
    // wave -> (group of NT adjacent tiles, set of AG activation groups); the
    // ns waves of a tile group are adjacent, so they share a workgroup (or
    // neighbouring ones) and the weight chunks they all stream are fetched
    // from HBM once.  NT > 1 spreads each activation load over NT tiles.
    // With several workgroups per tile group the grid (a multiple of 8) is
    // taken XCD-major: workgroups are dispatched to the 8 XCDs round-robin,
    // and consecutive indices of one XCD share its L2.
    int blk = blockIdx.x;
    if (ns > TPW) blk = (int)(blockIdx.x % 8) * (int)(gridDim.x / 8) + (int)(blockIdx.x / 8);
    const int wv = blk * TPW + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int TG = wv / ns;
    const int a0 = (wv - TG * ns) * AG;  // first activation group of the wave
    if (TG * NT >= n_tiles) return;  // whole waves only; the kernel has no barrier
    const int l = threadIdx.x & 63;
    const int r = l & 15, g = l >> 4;
    // the tiles' lap blocks: quant piece c of lap q at v4i offset
    // q * LB + c * 64 (+ lane), the lap's scales at q * LB + SO (+ row);
    // tiles past the end read the last tile and store nothing
    constexpr size_t LB = (W4 ? kQ4LapBytes : kQ8LapBytes) / 16;
    constexpr int SO = W4 ? 128 : 256;
    constexpr int NP = W4 ? 2 : 4;  // quant pieces per lap and lane
    const v4i *wp[NT];
    const v4i *sp[NT];
    int n[NT];
#pragma unroll
    for (int t = 0; t < NT; ++t) {
        const int T = min(TG * NT + t, n_tiles - 1);
        wp[t] = laps + (size_t)T * G * LB + l;
        sp[t] = laps + (size_t)T * G * LB + SO + r;
        n[t] = TG * NT + t < n_tiles ? (TG * NT + t) * 16 + r : N;
    }
    const v4i *ap[AG];
    float sa[AG][4], fs[AG][NT][4];
#pragma unroll
    for (int a = 0; a < AG; ++a) {
        const int m = 16 * (a0 + a) + r;
        ap[a] = reinterpret_cast<const v4i *>(act + (size_t)(m < M ? m : 0) * kp) + g;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            sa[a][i] = sa_rows[min(16 * (a0 + a) + 4 * g + i, M - 1)];
#pragma unroll
            for (int t = 0; t < NT; ++t) fs[a][t][i] = 0.0f;
        }
    }
    v4i wr[RL][NT][4];
    v4i xr[RL][4][AG];
    v4i sr[RL][NT];
#pragma unroll
    for (int u = 0; u < RL; ++u) {
        const int q = min(u, G - 1);
#pragma unroll
        for (int c = 0; c < 4; ++c) {
#pragma unroll
            for (int t = 0; t < NT; ++t)
                if (c < NP) wr[u][t][c] = __builtin_nontemporal_load(wp[t] + (size_t)q * LB + c * 64);
#pragma unroll
            for (int a = 0; a < AG; ++a) xr[u][c][a] = ap[a][(size_t)(4 * q + c) * 4];
        }
#pragma unroll
        for (int t = 0; t < NT; ++t) sr[u][t] = sp[t][(size_t)q * LB];
    }
    const v4i zero = {0, 0, 0, 0};
    // Without W4 each block's MFMA starts from the bits of 1.5 * 2^23, so an
    // output register read as f32 is 12582912 + dot exactly (|dot| < 2^22);
    // one full-rate subtract gives (f32)dot, bit for bit what the half-rate
    // v_cvt_f32_i32 gives.
    const v4i cinit = W4 ? zero : v4i{kDotBias, kDotBias, kDotBias, kDotBias};

    // Lap L in ring slot U.  REFILL: lap L + RL exists and is loaded into
    // the slot; CHECK: skip padding blocks past nb (last laps only).
    auto lap = [&](int L, auto slot, bool refill, auto check) __attribute__((always_inline)) {
        constexpr int U = decltype(slot)::value;
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            v4i d[2][AG][NT];
#pragma unroll
            for (int h = 0; h < 2; ++h) {
#pragma unroll
                for (int t = 0; t < NT; ++t) {
                    long bv;
                    if constexpr (W4) {
                        const v4i pc = wr[U][t][c >> 1];
                        const int wd = (c & 1) ? (h ? pc.w : pc.z) : (h ? pc.y : pc.x);
                        constexpr int kHi = (int)0xF0F0F0F0u;
                        bv = (long)(((unsigned long)(unsigned)(wd & kHi) << 32) |
                                    (unsigned)((wd << 4) & kHi));
                    } else {
                        bv = h ? hi8(wr[U][t][c]) : lo8(wr[U][t][c]);
                    }
#pragma unroll
                    for (int a = 0; a < AG; ++a) {
                        d[h][a][t] = __builtin_amdgcn_mfma_i32_16x16x32_i8(
                            h ? hi8(xr[U][c][a]) : lo8(xr[U][c][a]), bv, cinit, 0, 0, 0);
                        if constexpr (W4) {
#pragma unroll
                            for (int i = 0; i < 4; ++i) d[h][a][t][i] >>= 4;
                        }
                    }
                }
            }
            if (refill) {
                const size_t p = (size_t)(4 * (L + RL) + c);
                if (!W4 || (c & 1)) {
                    const int pi = W4 ? c >> 1 : c;
#pragma unroll
                    for (int t = 0; t < NT; ++t)
                        wr[U][t][pi] =
                            __builtin_nontemporal_load(wp[t] + (size_t)(L + RL) * LB + pi * 64);
                }
#pragma unroll
                for (int a = 0; a < AG; ++a) xr[U][c][a] = ap[a][p * 4];
            }
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                const int b = 8 * L + 2 * c + h;
                if (!decltype(check)::value || b < nb) {
#pragma unroll
                    for (int t = 0; t < NT; ++t) {
                        const unsigned word = (unsigned)sr[U][t][c];
                        const float ds = f16_bits_to_f32(h ? (word >> 16) : (word & 0xFFFFu));
#pragma unroll
                        for (int a = 0; a < AG; ++a) {
#pragma unroll
                            for (int i = 0; i < 4; ++i) {
                                const int dv = d[h][a][t][i];
                                float tm = (W4 ? (float)dv : __int_as_float(dv) - kDotBiasF) *
                                           sa[a][i];
                                tm = tm * ds;
                                fs[a][t][i] = fs[a][t][i] + tm;
                            }
                            if constexpr (DEBUG) {
#pragma unroll
                                for (int i = 0; i < 4; ++i) {
                                    const int m = 16 * (a0 + a) + 4 * g + i;
                                    if (m < M && n[t] < N)
                                        block_dots[((size_t)m * N + n[t]) * nb + b] =
                                            W4 ? d[h][a][t][i] : d[h][a][t][i] - kDotBias;
                                }
                            }
                        }
                    }
                }
            }
        }
        if (refill) {
#pragma unroll
            for (int t = 0; t < NT; ++t) sr[U][t] = sp[t][(size_t)(L + RL) * LB];
        }
        // keep the next lap's uses of its (younger) loads below this point
        __builtin_amdgcn_sched_barrier(0);
    };

    using T1 = std::true_type;
    using F0 = std::false_type;
    {
        const int k = G / RL, rem = G - k * RL;
        for (int it = 0; it + 1 < k; ++it)
            static_for<RL>([&](auto u) { lap(it * RL + u, u, true, F0{}); });
        if (k > 0)
            static_for<RL>([&](auto u) { lap((k - 1) * RL + u, u, u < rem, T1{}); });
        static_for<RL>([&](auto u) {
            if (u < rem) lap(k * RL + u, u, false, T1{});
        });
    }
#pragma unroll
    for (int t = 0; t < NT; ++t) {
        if (n[t] >= N) continue;
#pragma unroll
        for (int a = 0; a < AG; ++a)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int m = 16 * (a0 + a) + 4 * g + i;
                if (m < M) out[(size_t)m * N + n[t]] = fs[a][t][i];
            }
    }
}

constexpr int kU = 8;

// Prefill-sized M (one launch, ceil(M/32) waves per tile group): tiles per
// wave and laps in flight (measured on MI355X at M = 64 .. 2048: two tiles
// per wave run 1.4-1.5x faster than one; four are slower than two).
constexpr int kPrefillNT = 2;
constexpr int kPrefillRL = 2;

template <int MT, int NI, int U>
void launch_i8(const int8_t *act, size_t m, size_t kp, const float *sa_ptr,
               int sa_stride, float sa_value, const QMatrixDev &w, float *out,
               int32_t *acc_out, hipStream_t s) {
    hipLaunchKernelGGL((k_skinny_int8<MT, NI, U>), dim3((unsigned)w.n_tiles),
                       dim3(kWave), 0, s, act, (int)m, kp, sa_ptr, sa_stride,
                       sa_value, reinterpret_cast<const v4i *>(w.tiles), w.scales,
                       (int)w.n_out, (int)(w.kp / kChunkK), out, acc_out);
}

// AG activation groups per wave, ns waves per tile (AG * ns groups of 16 rows).
template <int AG, int NT, int TPW, int RL, bool DEBUG, bool W4>
void launch_q8_w(const int8_t *act, size_t m, size_t kp, const float *sa_rows,
                 const Q8MatrixDev &w, float *out, int32_t *block_dots, int ns, hipStream_t s) {
    const int G = (int)w.laps_per_tile();
    const size_t waves = (w.n_tiles + NT - 1) / NT * (size_t)ns;
    size_t grid = (waves + TPW - 1) / TPW;
    if (ns > TPW) grid = (grid + 7) / 8 * 8;  // XCD-major mapping (whole waves past the end exit)
    hipLaunchKernelGGL((k_skinny_q8_0<AG, NT, TPW, RL, DEBUG, W4>),
                       dim3((unsigned)grid), dim3(TPW * kWave), 0, s,
                       act, (int)m, (int)kp, sa_rows, reinterpret_cast<const v4i *>(w.laps),
                       (int)w.n_out, (int)w.n_tiles, G,
                       (int)w.n_blocks, out, block_dots, ns);
}

template <int AG, int NT, int TPW, int RL, bool DEBUG>
void launch_q8(const int8_t *act, size_t m, size_t kp, const float *sa_rows,
               const Q8MatrixDev &w, float *out, int32_t *block_dots, int ns, hipStream_t s) {
    if (w.w4)
        launch_q8_w<AG, NT, TPW, RL, DEBUG, true>(act, m, kp, sa_rows, w, out, block_dots, ns, s);
    else
        launch_q8_w<AG, NT, TPW, RL, DEBUG, false>(act, m, kp, sa_rows, w, out, block_dots, ns, s);
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
    if (m > 32) {
        // one launch for all rows: ceil(m/32) waves of 32 rows per weight
        // tile, four to a workgroup; the weights stream from HBM about once
        // instead of once per 32-row slice
        const int ns = (int)((m + 31) / 32);
        if (block_dots)
            launch_q8<2, kPrefillNT, 4, kPrefillRL, true>(act, m, kp, sa_rows, w, out, block_dots, ns, s);
        else
            launch_q8<2, kPrefillNT, 4, kPrefillRL, false>(act, m, kp, sa_rows, w, out, block_dots, ns, s);
        MRI_LAUNCHED("k_skinny_q8_0");
        return MRI_OK;
    }
    for (size_t m0 = 0; m0 < m; m0 += 32) {
        const size_t mc = m - m0 < 32 ? m - m0 : 32;
        const int8_t *a = act + m0 * kp;
        const float *sp = sa_rows + m0;
        float *o = out + m0 * w.n_out;
        int32_t *bd = block_dots ? block_dots + m0 * w.n_out * w.n_blocks : nullptr;
        // one wave per tile and workgroup (measured on MI355X: splitting a
        // tile's row groups over waves, or grouping tiles, is slower)
        if (bd) {
            if (mc <= 16) launch_q8<1, 1, 1, 2, true>(a, mc, kp, sp, w, o, bd, 1, s);
            else launch_q8<2, 1, 1, 2, true>(a, mc, kp, sp, w, o, bd, 1, s);
        } else {
            if (mc <= 16) launch_q8<1, 1, 1, 3, false>(a, mc, kp, sp, w, o, bd, 1, s);
            else launch_q8<2, 1, 1, 2, false>(a, mc, kp, sp, w, o, bd, 1, s);
        }
        MRI_LAUNCHED("k_skinny_q8_0");
    }
    return MRI_OK;
}

}  // namespace mri
