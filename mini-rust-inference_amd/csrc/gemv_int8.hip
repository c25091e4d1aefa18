// gemv_int8.hip — per-channel INT8 decode GEMV (M <= 4): matmul_int8 /
// matmul_int8_from_f32 (int8.rs:61-143) on the slab-major MFMA chunks.
//
// v_mfma_i32_16x16x64_i8 accumulates exact int32 sums over the wave's K
// segment; with S > 1 the S partial accumulators are added through LDS and
// wave 0 of the tile applies ((f32)acc * s_a) * s_w (int8.rs:93).  Each wave
// keeps D chunk loads in flight in a ring of registers.
//
// LAZY (the fused row without a quantized-row output, below 1024 tiles): the
// prologue stages the f32 row in LDS and reduces max|x| without quantizing
// it; each wave then quantizes one lap (its next D chunks, 64 D values, D/4
// float4 a lane) into an LDS area of its own after the previous lap's MFMAs,
// while the lap's loads are in flight.  Same scale, same rounding: the int8
// values, int32 sums and outputs are those of the up-front quantization.
#include "gemv_common.hpp"

namespace mri {
using namespace gemv;
namespace {

// ---------------------------------------------------------------------------
// Per-channel INT8.
// ---------------------------------------------------------------------------
template <int NI, int S, int TPW, int D, int XR, bool FUSED, bool OPS, bool LAZY = false>
__global__ __launch_bounds__(S * TPW * kWave) void k_gemv_int8(
    ActIn in, int M, int kp, const float *__restrict__ sa_ptr, int sa_stride,
    float sa_value, const v4i *__restrict__ tiles, const float *__restrict__ wscales,
    int N, int n_tiles, int P, float *__restrict__ out, int32_t *__restrict__ acc_out) {
    constexpr int NW = S * TPW;
    static_assert(!LAZY || (FUSED && NI == 1 && D % 4 == 0), "lap-wise: the fused row");
    extern __shared__ v4i s_lds[];
    // wave index as a scalar: segment bounds and loop guards stay uniform, so
    // no MFMA ever sits under a partial EXEC mask.
    const int wl = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int tw_ = wl / S;                   // tile of the wave within the WG
    const int w = wl - tw_ * S;               // segment of the wave
    const int T = blockIdx.x * TPW + tw_;
    const bool tile_ok = T < n_tiles;
    const int Tc = tile_ok ? T : n_tiles - 1;
    const int l = threadIdx.x & 63;
    const int r = l & 15, g = l >> 4;
    const int c0 = split_lo(P, S, w), c1 = tile_ok ? split_lo(P, S, w + 1) : c0;
    const int nc = c1 - c0;
    const int last = max(c1 - 1, 0);
    const size_t pitch = (size_t)n_tiles * kWave;  // v4i per slab of chunks
    const v4i *wp = tiles + (size_t)Tc * kWave + l;

    // LDS: [act M*kp, or with LAZY the f32 row (kp floats)][red NW floats]
    // [partials TPW x (S-1) x 64 v4i][LAZY: one quantized lap (64 D bytes) per
    // wave, then 64 D bytes of zeros that the lanes of rows >= M read]
    int8_t *s_act = reinterpret_cast<int8_t *>(s_lds);
    float *red = reinterpret_cast<float *>(s_act + (size_t)(LAZY ? 4 : M) * kp);
    v4i *part = reinterpret_cast<v4i *>(red + 4 * NW) + (size_t)tw_ * (S - 1) * kWave;
    int8_t *s_lap = reinterpret_cast<int8_t *>(reinterpret_cast<v4i *>(red + 4 * NW) +
                                               (size_t)TPW * (S - 1) * kWave) +
                    (size_t)wl * 64 * D;

    const bool aval = r < M;
    int8_t *s_zero = s_lap + (size_t)(NW - wl) * 64 * D;  // LAZY
    const v4i *ap = LAZY ? reinterpret_cast<const v4i *>(aval ? s_lap : s_zero) + g
                         : reinterpret_cast<const v4i *>(s_act + (size_t)(aval ? r : 0) * kp) + g;
    const v4i zero = {0, 0, 0, 0};
    v4i acc = zero;
    v4i wr[D];

    v4i xr[XR];
    const int n16 = FUSED ? in.K / 4 : M * kp / 16;
    const float *xrow = in.x;
    if constexpr (FUSED && OPS) xrow = row_of_keys<NW>(in);  // the step's token row
    stage_load<NW, XR>(FUSED ? reinterpret_cast<const v4i *>(xrow)
                             : reinterpret_cast<const v4i *>(in.act),
                       n16, xr);
    v4i wn[XR];  // RMS norm weights (row operations)
    if constexpr (FUSED && OPS) {
        if (in.norm_w) stage_load<NW, XR>(reinterpret_cast<const v4i *>(in.norm_w), n16, wn);
        else if (in.up) stage_load<NW, XR>(reinterpret_cast<const v4i *>(in.up), n16, wn);
    }
    // activation loads before the ring's (they return first; see gemv_q8.hip)
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int s = 0; s < D; ++s)
        wr[s] = __builtin_nontemporal_load(wp + (size_t)min(c0 + s, last) * pitch);
    // the epilogue's weight scale and row-operation destination, loaded now
    // (issued after the ring's loads, so the prologue does not wait for
    // them), so that the epilogue waits for no load of its own
    const int n = T * 16 + r;
    const float sw = wscales[min(n, N - 1)];
    RowDst dst{};
    if constexpr (OPS) {
        if (w == 0) dst = row_dst(in, out, n, N);
    }
    if constexpr (FUSED && OPS) {
        if (in.up) act_swiglu<NW, XR>(in, xr, wn);
    }
    if constexpr (LAZY) {  // the zero area (the prologue's barrier orders it)
        if ((int)threadIdx.x < 4 * D) reinterpret_cast<v4i *>(s_zero)[threadIdx.x] = zero;
    }
    act_begin<NW, XR, FUSED, OPS>(in, n16, xr, s_act, red);
    float inv = 0.0f;  // LAZY: 1 / scale of the row
    if constexpr (LAZY)
        inv = act_end_lazy<NW, XR, OPS>(in, xr, wn, reinterpret_cast<float *>(s_act), red,
                                        sa_value, blockIdx.x == 0);
    else
        act_end<NW, XR, FUSED, OPS>(in, kLayPlain, xr, wn, s_act, red, sa_value, blockIdx.x == 0);
    if constexpr (FUSED) sa_ptr = nullptr;

    // LAZY: quantize lap L (chunks c0 + L*D ..; lane l: values 256 e + 4 l of
    // the lap, zero past K) into this wave's area, in plain order
    auto quant_lap = [&](int L) __attribute__((always_inline)) {
        const float4 *xf = reinterpret_cast<const float4 *>(s_act);
        const int base = 64 * (c0 + L * D);
#pragma unroll
        for (int e = 0; e < D / 4; ++e) {
            const int kk = base + 256 * e + 4 * l;
            float4 v = float4{0.0f, 0.0f, 0.0f, 0.0f};
            if (kk < in.K) v = xf[kk >> 2];
            *reinterpret_cast<int *>(s_lap + 256 * e + 4 * l) = quant4_packed(v, inv);
        }
    };
    if constexpr (LAZY) {
        if (nc > 0) quant_lap(0);
    }
    auto mfma = [&](int s, int i) __attribute__((always_inline)) {
        const v4i a = LAZY ? ap[s * 4] : aval ? ap[(size_t)(c0 + i) * 4] : zero;
        acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(a, wr[s], acc, 0, 0, 0);
    };
    // full laps with refills: chunk i is consumed from slot i % D, then the
    // slot is reloaded with chunk i + D, which exists (i + D < laps * D <= nc)
    const int laps = nc / D;
    for (int lap = 0; lap + 1 < laps; ++lap) {
#pragma unroll
        for (int s = 0; s < D; ++s) {
            const int i = lap * D + s;
            mfma(s, i);
            wr[s] = __builtin_nontemporal_load(wp + (size_t)(c0 + i + D) * pitch);
        }
        if constexpr (LAZY) quant_lap(lap + 1);  // after this lap's reads of the area
    }
    // last full lap: refill only the slots of the remaining nc % D chunks
    const int rem = nc - laps * D;
    if (laps > 0) {
#pragma unroll
        for (int s = 0; s < D; ++s) {
            const int i = (laps - 1) * D + s;
            mfma(s, i);
            if (s < rem)
                wr[s] = __builtin_nontemporal_load(wp + (size_t)(c0 + i + D) * pitch);
        }
        if constexpr (LAZY) {
            if (rem > 0) quant_lap(laps);
        }
    }
#pragma unroll
    for (int s = 0; s < D; ++s)
        if (s < rem) mfma(s, laps * D + s);

    // exact int32 reduction over the S segments
    if constexpr (S > 1) {
        if (w > 0) part[(w - 1) * kWave + l] = acc;
        __syncthreads();
        if (w > 0) return;
#pragma unroll
        for (int s = 1; s < S; ++s) acc += part[(s - 1) * kWave + l];
    }

    if (!tile_ok) return;
    if constexpr (OPS) {  // one row: lanes 0-15 hold channels 16T .. 16T+15
        float v = (float)acc[0] * sa_value;
        v = v * sw;
        const float pv = __shfl_xor(v, 1);
        const bool mine = g == 0 && n < N;
        if (mine) {
            if (acc_out) acc_out[n] = acc[0];
            row_store(in, dst, n, v, pv);
        }
        if (in.arg_keys) row_argmax_key(in.arg_keys, T, v, n, mine);
        return;
    }
    if (n >= N || g != 0) return;
#pragma unroll
    for (int i = 0; i < NI; ++i) {
        if (i < M) {
            const float sa = sa_ptr ? sa_ptr[(size_t)i * sa_stride] : sa_value;
            float v = (float)acc[i] * sa;
            v = v * sw;
            out[(size_t)i * N + n] = v;
            if (acc_out) acc_out[(size_t)i * N + n] = acc[i];
        }
    }
}


struct CfgI8 {
    int s = 0, tpw = 1, d = 4, xr = 0;  // s == 0: unsupported
    bool lazy = false;                    // lap-wise quantization of the fused row
};

size_t lds_i8(int s, int tpw, size_t m, size_t kp, int d = 4, bool lazy = false) {
    return (lazy ? 4 : m) * kp + (size_t)s * tpw * 16 + (size_t)tpw * (s - 1) * kWave * 16 +
           (lazy ? (size_t)(s * tpw + 1) * 64 * d : 0);
}

// Configuration by the number of 16-row tiles (measured on MI355X): about
// 2000-2800 waves and 4-16 MB of weight loads in flight over the whole GPU.
// Many tiles: one wave per tile, 8 tiles per workgroup; otherwise the K
// split keeps enough waves.  The activation staging must fit XR pieces per
// thread (4, 8 or 12 of 16 bytes).
// lazy_ok: the fused row without a quantized-row output, which then takes
// the lap-wise quantization below 1024 tiles (with or without the decode
// step's row operations).  Measured on MI355X (us per call, same box):
// 4096 -> 11008 9.0 -> 8.85, 4096 -> 4096 5.25 -> 5.04, 11008 -> 4096
// 10.4 -> 10.1; 2-8 waves with 4-16 chunks in flight at 688 tiles were
// slower than the configuration below (8.84-10.6 us).  In the INT8 layer's
// decode step (o, down and the 768-tile q/k/v): 83.7 -> 83.05 us per token.
CfgI8 pick_i8(bool fused, size_t n_tiles, size_t m, size_t k, size_t kp, bool lazy_ok = false) {
    CfgI8 c;
    if (n_tiles >= 1024) { c.s = 1; c.tpw = 8; c.d = 8; }
    else if (n_tiles >= 512) { c.s = 4; c.d = 4; }
    else if (kp <= 4096) { c.s = 4; c.d = 8; }
    else { c.s = 8; c.d = 8; }
    const size_t threads = (size_t)c.s * c.tpw * kWave;
    const size_t nx = ceil_div(fused ? k / 4 : m * kp / 16, threads);
    c.xr = nx <= 4 ? 4 : nx <= 8 ? 8 : nx <= 12 ? 12 : 0;
    if (c.xr == 0 || lds_i8(c.s, c.tpw, m, kp) > kMaxLds) c.s = 0;
    if (c.s && fused && lazy_ok && m == 1 && c.tpw == 1 &&
        lds_i8(c.s, c.tpw, m, kp, c.d, true) <= kMaxLds)
        c.lazy = true;
    return c;
}

template <int NI, int S, int TPW, int D, int XR, bool FUSED, bool OPS, bool LAZY = false>
void launch_i8(ActIn in, size_t m, const float *sa_ptr, int sa_stride, float sa_value,
               const QMatrixDev &w, float *out, int32_t *acc_out, hipStream_t st) {
    hipLaunchKernelGGL((k_gemv_int8<NI, S, TPW, D, XR, FUSED, OPS, LAZY>),
                       dim3((unsigned)ceil_div(w.n_tiles, TPW)), dim3(S * TPW * kWave),
                       lds_i8(S, TPW, m, w.kp, D, LAZY), st, in, (int)m, (int)w.kp, sa_ptr,
                       sa_stride,
                       sa_value, reinterpret_cast<const v4i *>(w.tiles), w.scales,
                       (int)w.n_out, (int)w.n_tiles, (int)(w.kp / kChunkK), out, acc_out);
}

template <int NI, bool FUSED, bool OPS = false>
void dispatch_i8(CfgI8 c, ActIn in, size_t m, const float *sa_ptr, int sa_stride,
                 float sa_value, const QMatrixDev &w, float *out, int32_t *acc_out,
                 hipStream_t st) {
    if constexpr (FUSED && NI == 1) {
#define MRI_I8L(S_, D_, XR_)                                                               \
    if (c.s == S_ && c.tpw == 1 && c.d == D_ && c.xr == XR_)                               \
        return launch_i8<1, S_, 1, D_, XR_, true, OPS, true>(in, m, sa_ptr, sa_stride,     \
                                                             sa_value, w, out, acc_out, st);
        if (c.lazy) {
            MRI_I8L(4, 4, 4) MRI_I8L(4, 4, 8) MRI_I8L(4, 4, 12)
            MRI_I8L(4, 8, 4) MRI_I8L(4, 8, 8) MRI_I8L(4, 8, 12)
            MRI_I8L(8, 8, 4) MRI_I8L(8, 8, 8) MRI_I8L(8, 8, 12)
        }
#undef MRI_I8L
    }
#define MRI_I8(S_, TPW_, D_, XR_)                                                          \
    if (c.s == S_ && c.tpw == TPW_ && c.d == D_ && c.xr == XR_)                            \
        return launch_i8<NI, S_, TPW_, D_, XR_, FUSED, OPS>(in, m, sa_ptr, sa_stride,      \
                                                            sa_value, w, out, acc_out, st);
    MRI_I8(1, 8, 8, 4) MRI_I8(1, 8, 8, 8) MRI_I8(1, 8, 8, 12)
    MRI_I8(4, 1, 4, 4) MRI_I8(4, 1, 4, 8) MRI_I8(4, 1, 4, 12)
    MRI_I8(4, 1, 8, 4) MRI_I8(4, 1, 8, 8) MRI_I8(4, 1, 8, 12)
    MRI_I8(8, 1, 8, 4) MRI_I8(8, 1, 8, 8) MRI_I8(8, 1, 8, 12)
#undef MRI_I8
}

}  // namespace

bool gemv_int8_supported(bool fused, size_t m, size_t n_tiles, size_t k, size_t kp) {
    return m >= 1 && m <= (size_t)kMaxM && pick_i8(fused, n_tiles, m, k, kp).s > 0;
}

// The row operations apply to the fused path only, with aligned operands.
bool row_ops_ok(const float *x, const RowOps &o) {
    auto al = [](const float *p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; };
    if (!o.any()) return true;
    const bool rope = o.rope_n == 0 || (o.rope_cos && o.rope_sin && o.hd >= 2 && o.hd % 2 == 0 &&
                                        o.rope_n % 2 == 0);
    const bool segs = (o.seg1 == INT_MAX || o.out1) && (o.seg2 == INT_MAX || o.out2) &&
                      o.seg1 <= o.seg2 && o.seg1 >= 0;
    const bool glu = !o.up || (al(o.up) && !o.norm_w && !o.x_out);
    const bool silu = o.silu_n == 0 || (o.silu_n > 0 && !o.accum && o.rope_n == 0);
    const bool arg = !o.arg_keys || (reinterpret_cast<uintptr_t>(o.arg_keys) & 7) == 0;
    const bool keys = !o.in_keys || ((reinterpret_cast<uintptr_t>(o.in_keys) & 7) == 0 &&
                                     o.n_in_keys > 0 && !o.up);
    return x && al(o.norm_w) && al(o.x_out) && glu && silu && arg && keys && rope && segs;
}

bool gemv_fusable(size_t m, size_t k, const float *x) {
    return m == 1 && k > 0 && k % 4 == 0 && x &&
           (reinterpret_cast<uintptr_t>(x) & 15) == 0;
}

mri_status launch_gemv_int8(const float *x, const int8_t *act, size_t m,
                            const float *sa_ptr, int sa_stride, float sa_value,
                            const QMatrixDev &w, float *out, int8_t *act_q_out,
                            float *scale_out, int32_t *acc_out, hipStream_t st,
                            const RowOps &ops) {
    if (w.n_tiles == 0 || m == 0) return MRI_OK;
    const CfgI8 c = pick_i8(x != nullptr, w.n_tiles, m, w.k_in, w.kp,
                            x && !act_q_out);
    if (c.s == 0) return set_error(MRI_ERR_INVALID_ARGUMENT, "gemv: shape not supported");
    if (!row_ops_ok(x, ops))
        return set_error(MRI_ERR_INVALID_ARGUMENT, "gemv: row operations need the fused path");
    const ActIn in(x, act, (int)w.k_in, act_q_out, scale_out, ops);
    if (ops.any()) {
        dispatch_i8<1, true, true>(c, in, m, nullptr, 0, 0.0f, w, out, acc_out, st);
    } else if (x) {
        dispatch_i8<1, true>(c, in, m, nullptr, 0, 0.0f, w, out, acc_out, st);
    } else {
        if (m == 1) dispatch_i8<1, false>(c, in, m, sa_ptr, sa_stride, sa_value, w, out, acc_out, st);
        else if (m == 2) dispatch_i8<2, false>(c, in, m, sa_ptr, sa_stride, sa_value, w, out, acc_out, st);
        else dispatch_i8<4, false>(c, in, m, sa_ptr, sa_stride, sa_value, w, out, acc_out, st);
    }
    MRI_LAUNCHED("k_gemv_int8");
    return MRI_OK;
}

}  // namespace mri
