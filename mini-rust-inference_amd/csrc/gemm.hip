// gemm.hip — prefill-sized per-channel INT8 matmul (matmul_int8,
// int8.rs:61-98, and its parallel form parallel.rs:308-346) as a dense
// contraction on CDNA4 int8 MFMA.
//
//   acc[m, n] = sum_k act_q[m, k] * w[n, k]            (exact int32)
//   out[m, n] = ((f32)acc[m, n] * s_a[m]) * s_w[n]      (int8.rs:93)
//
// Tiling: a workgroup of WM x WN waves computes a BM x BN output tile; wave
// (wm, wn) owns a (BM/WM) x (BN/WN) block of 16 x 16 MFMA tiles and runs
// one v_mfma_i32_16x16x64_i8 per tile per K step of 64.  Both operands are
// staged through LDS in the MFMA fragment layout: a 16-row x 64-k fragment
// is 1 KiB with lane l's 16 bytes at l * 16 (row l % 16, k 16*(l/16)..+16),
// so every LDS read is one contiguous, conflict-free ds_read_b128 per wave.
// The weight chunks are stored in exactly this layout (slab-major), so a
// workgroup's BN/16 chunks of one K slab are one contiguous block of
// global memory; the activation rows are permuted into fragments by the
// copy.
//
// Pipeline: the global loads of K step s + PF are issued at step s into
// one of PF register sets; the set of step s + 1 is written to the other
// LDS buffer after step s's MFMAs, then one barrier.  The activations are
// L2-resident (M x K bytes); the weights stream from HBM once per M tile.
#include <utility>

#include "common.hpp"

namespace mri {
namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
constexpr int kWave = 64;

template <typename F, int... I>
__device__ inline void static_for_impl(F &&f, std::integer_sequence<int, I...>) {
    (f(std::integral_constant<int, I>{}), ...);
}
template <int N, typename F>
__device__ inline void static_for(F &&f) {
    static_for_impl(f, std::make_integer_sequence<int, N>{});
}

template <int BM, int BN, int WM, int WN, int PF>
__global__ __launch_bounds__(WM * WN * kWave) void k_gemm_int8(
    const int8_t *__restrict__ act, int M, int lda, const float *__restrict__ sa_ptr,
    int sa_stride, float sa_value, const v4i *__restrict__ tiles,
    const float *__restrict__ wscales, int N, int n_tiles, int P, float *__restrict__ out,
    int32_t *__restrict__ acc_out) {
    constexpr int NT = WM * WN * kWave;        // threads
    constexpr int FA = BM / 16, FB = BN / 16;  // fragments per K step
    constexpr int TM = BM / WM / 16, TN = BN / WN / 16;  // MFMA tiles per wave
    constexpr int LA = FA * kWave / NT;        // 16-byte A pieces per thread per step
    constexpr int LB = FB * kWave / NT;        // 16-byte B pieces per thread per step
    static_assert(FA * kWave % NT == 0 && FB * kWave % NT == 0, "copy split");
    constexpr int STAGE = (FA + FB) * 1024;    // bytes of one LDS buffer
    __shared__ v4i s_buf[2 * STAGE / 16];

    // Workgroup -> tile.  Consecutive workgroups walk M first so that the
    // M tiles sharing a weight column block run close together in time.
    const int n_mt = (M + BM - 1) / BM;
    const int mt = blockIdx.x % n_mt, nt = blockIdx.x / n_mt;
    const int m0 = mt * BM, T0 = nt * FB;      // first row, first weight tile

    const int t = threadIdx.x;
    const int wv = t >> 6, l = t & 63;
    const int wm = wv / WN, wn = wv % WN;

    // Copy assignment: piece q = t + NT * j of the step; A piece q is lane
    // q % 64 of fragment q / 64: row m0 + 16*(q/64) + q%16, k + 16*((q%64)/16).
    const int8_t *a_src[LA];
    bool a_ok[LA];
#pragma unroll
    for (int j = 0; j < LA; ++j) {
        const int q = t + NT * j, f = q >> 6, ql = q & 63;
        const int m = m0 + 16 * f + (ql & 15);
        a_ok[j] = m < M;
        a_src[j] = act + (size_t)(a_ok[j] ? m : 0) * lda + 16 * (ql >> 4);
    }
    const v4i *b_src[LB];
#pragma unroll
    for (int j = 0; j < LB; ++j) {
        const int q = t + NT * j, f = q >> 6, ql = q & 63;
        const int T = min(T0 + f, n_tiles - 1);
        b_src[j] = tiles + (size_t)T * kWave + ql;
    }
    const size_t b_pitch = (size_t)n_tiles * kWave;  // v4i per K slab

    v4i ra[PF][LA], rb[PF][LB];
    auto gload = [&](auto set, int p) __attribute__((always_inline)) {
        constexpr int SET = decltype(set)::value;
        const int pc = min(p, P - 1);              // clamped: loads past P are unused
#pragma unroll
        for (int j = 0; j < LA; ++j)
            ra[SET][j] = *reinterpret_cast<const v4i *>(a_src[j] + (size_t)pc * 64);
#pragma unroll
        for (int j = 0; j < LB; ++j)
            rb[SET][j] = __builtin_nontemporal_load(b_src[j] + (size_t)pc * b_pitch);
    };
    auto lstore = [&](auto set, int buf) __attribute__((always_inline)) {
        constexpr int SET = decltype(set)::value;
        v4i *dst = s_buf + (size_t)buf * (STAGE / 16);
        const v4i zero = {0, 0, 0, 0};
#pragma unroll
        for (int j = 0; j < LA; ++j) dst[t + NT * j] = a_ok[j] ? ra[SET][j] : zero;
#pragma unroll
        for (int j = 0; j < LB; ++j) dst[FA * kWave + t + NT * j] = rb[SET][j];
    };

    v4i acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) acc[i][j] = v4i{0, 0, 0, 0};

    auto compute = [&](int buf) __attribute__((always_inline)) {
        const v4i *sa_ = s_buf + (size_t)buf * (STAGE / 16) + (wm * TM) * kWave + l;
        const v4i *sb_ = s_buf + (size_t)buf * (STAGE / 16) + (FA + wn * TN) * kWave + l;
        v4i fa[TM], fb[TN];
#pragma unroll
        for (int i = 0; i < TM; ++i) fa[i] = sa_[i * kWave];
#pragma unroll
        for (int j = 0; j < TN; ++j) fb[j] = sb_[j * kWave];
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
            for (int j = 0; j < TN; ++j)
                acc[i][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(fa[i], fb[j], acc[i][j], 0, 0, 0);
    };

    // Invariant at the start of step p: LDS buffer p % 2 holds step p, the
    // register sets hold steps p+1 .. p+PF-1 (in flight) and set p % PF is
    // free.  Step p: refill set p % PF with step p + PF, MFMAs on buffer
    // p % 2, store set (p+1) % PF (step p + 1) to the other buffer, barrier.
    static_for<PF>([&](auto s) { gload(s, s); });
    lstore(std::integral_constant<int, 0>{}, 0);
    __syncthreads();
    auto step = [&](int p, auto s, bool refill, bool store) __attribute__((always_inline)) {
        constexpr int SET = decltype(s)::value % PF;
        constexpr int NXT = (decltype(s)::value + 1) % PF;
        if (refill) gload(std::integral_constant<int, SET>{}, p + PF);
        compute(p & 1);
        if (store) lstore(std::integral_constant<int, NXT>{}, (p + 1) & 1);
        __syncthreads();
    };
    // blocks of PF steps whose refills all exist: branch-free, so the waits
    // before each LDS store stay exact
    int base = 0;
    for (; base + 2 * PF <= P; base += PF)
        static_for<PF>([&](auto s) { step(base + s, s, true, true); });
    // the last 1 .. 2*PF - 1 steps
    static_for<2 * PF>([&](auto s) {
        const int p = base + s;
        if (p < P) step(p, s, p + PF < P, p + 1 < P);
    });

    // epilogue: lane l, register r of tile (i, j) holds row
    // m0 + wm*TM*16 + 16i + 4*(l/16) + r, column n = 16*(T0 + wn*TN + j) + l%16
#pragma unroll
    for (int j = 0; j < TN; ++j) {
        const int n = 16 * (T0 + wn * TN + j) + (l & 15);
        if (n >= N) continue;
        const float sw = wscales[n];
#pragma unroll
        for (int i = 0; i < TM; ++i) {
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int m = m0 + 16 * (wm * TM + i) + 4 * (l >> 4) + r;
                if (m < M) {
                    const float sa = sa_ptr ? sa_ptr[(size_t)m * sa_stride] : sa_value;
                    float v = (float)acc[i][j][r] * sa;
                    v = v * sw;
                    out[(size_t)m * N + n] = v;
                    if (acc_out) acc_out[(size_t)m * N + n] = acc[i][j][r];
                }
            }
        }
    }
}

template <int BM, int BN, int WM, int WN, int PF>
void launch(const int8_t *act, size_t m, size_t lda, const float *sa_ptr, int sa_stride,
            float sa_value, const QMatrixDev &w, float *out, int32_t *acc_out,
            hipStream_t s) {
    const size_t n_mt = (m + BM - 1) / BM;
    const size_t n_nt = (w.n_tiles + BN / 16 - 1) / (BN / 16);
    hipLaunchKernelGGL((k_gemm_int8<BM, BN, WM, WN, PF>), dim3((unsigned)(n_mt * n_nt)),
                       dim3(WM * WN * kWave), 0, s, act, (int)m, (int)lda, sa_ptr,
                       sa_stride, sa_value, reinterpret_cast<const v4i *>(w.tiles),
                       w.scales, (int)w.n_out, (int)w.n_tiles, (int)(w.kp / kChunkK), out,
                       acc_out);
}

}  // namespace

// act: [m][lda] int8 rows (lda >= kp, a multiple of 16, zero padded to kp).
mri_status launch_gemm_int8(const int8_t *act, size_t m, const float *sa_ptr,
                            int sa_stride, float sa_value, const QMatrixDev &w,
                            float *out, int32_t *acc_out, hipStream_t s) {
    if (w.n_tiles == 0 || m == 0) return MRI_OK;
    launch<256, 128, 2, 2, 3>(act, m, w.kp, sa_ptr, sa_stride, sa_value, w, out, acc_out, s);
    MRI_LAUNCHED("k_gemm_int8");
    return MRI_OK;
}

}  // namespace mri
