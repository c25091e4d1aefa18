// gemv_q8.hip — Q8_0 decode GEMV (M <= 4): matmul_q8_0_direct
// (q8_direct.rs:229-289) on the slab-major MFMA chunks of the quants and
// the slab-major f16 scale groups.
#include "gemv_common.hpp"

namespace mri {
using namespace gemv;
namespace {

// ---------------------------------------------------------------------------
// Q8_0.  One v_mfma_i32_16x16x64_i8 per chunk computes both of its blocks:
// A row m = 2*row + h carries activation row `row` restricted to block
// 2p + h (the other 8 bytes of the lane's 16 are zeroed; the weight chunk
// keeps both blocks), so result register i of lane group g holds the exact
// int32 dot of activation row 2g + i/2 with block 2p + (i & 1) of output
// channel n = 16T + l%16.  MR (1, 2 or 4: rows of the instance) fixes how
// many lane groups hold results.
//
// A workgroup holds TPW tiles of S waves each; its waves share the
// activation staging.  Wave w of a tile sweeps one K segment in laps of one
// scale group (4 chunks = 8 blocks): the MFMAs of the lap's chunks, each
// followed by the refill of its ring slot with the chunk RL laps ahead,
// then the eight terms t_b = ((f32)dot_b * s_a) * d_b (q8_direct.rs:281),
// folded in block order (w == 0) or stored to LDS (w > 0), then the refill
// of the lap's scale slot.  With S > 1, after a barrier wave 0 of the tile
// continues its fold over the later segments in block order; either way the
// f32 result is bit-identical to the sequential reference.
// ---------------------------------------------------------------------------
template <int MR, int S, int TPW, int RL, int XR, bool FUSED, bool DEBUG>
__global__ __launch_bounds__(S * TPW * kWave) void k_gemv_q8_0(
    ActIn in, int M, int kp, const float *__restrict__ sa_rows,
    const v4i *__restrict__ tiles, const v4i *__restrict__ qscales, int N,
    int n_tiles, int G, int nb, float *__restrict__ out,
    int32_t *__restrict__ block_dots) {
    constexpr int NW = S * TPW;               // waves per workgroup
    constexpr int LR = MR == 1 ? 1 : 2;       // rows per result lane
    constexpr int LG = (MR + 1) / 2;          // lane groups holding results
    static_assert(!FUSED || MR == 1, "the fused prologue quantizes one row");
    extern __shared__ v4i s_lds[];
    const int wl = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int tw_ = wl / S;                   // tile of the wave within the WG
    const int w = wl - tw_ * S;               // segment of the wave
    const int T = blockIdx.x * TPW + tw_;
    const bool tile_ok = T < n_tiles;
    const int Tc = tile_ok ? T : n_tiles - 1; // address of a missing tile
    const int l = threadIdx.x & 63;
    const int r = l & 15, g = l >> 4;
    const int q0 = split_lo(G, S, w);
    const int q1 = tile_ok ? split_lo(G, S, w + 1) : q0;
    const int nq = q1 - q0;                   // laps of this wave
    const int c0 = 4 * q0;                    // first chunk of the segment
    const int lastq = max(q1 - 1, 0);
    const int maxq = (G + S - 1) / S;
    const int tstride = 8 * maxq;             // floats per (lane, row) of terms
    const size_t pitch = (size_t)n_tiles * kWave;
    const size_t spitch = (size_t)n_tiles * 16;
    const v4i *wp = tiles + (size_t)Tc * kWave + l;
    const v4i *sp = qscales + (size_t)Tc * 16 + r;
    const int n = T * 16 + r;

    // LDS: [act M*kp][red NW floats][terms TPW x (S-1) x LG x 16 x LR x 8*maxq floats]
    int8_t *s_act = reinterpret_cast<int8_t *>(s_lds);
    float *red = reinterpret_cast<float *>(s_act + (size_t)M * kp);
    float *terms = red + 4 * NW;
    auto term_base = [&](int seg) {  // terms of segment seg >= 1 of this tile, this lane
        return terms + ((size_t)((tw_ * (S - 1) + seg - 1) * LG + (g < LG ? g : 0)) * 16 + r) *
                           LR * tstride;
    };
    float *tl = term_base(w > 0 ? w : 1);

    // A operand: lane (r, g) reads activation row r/2 (16 bytes of lane
    // group g of each chunk) and keeps the half of block 2p + (r & 1).
    const int arow = r >> 1;
    const bool aval = arow < M;
    const int mlo = (aval && !(r & 1)) ? -1 : 0;
    const int mhi = (aval && (r & 1)) ? -1 : 0;
    const v4i *ap = reinterpret_cast<const v4i *>(s_act + (size_t)(aval ? arow : 0) * kp) + g;

    v4i wr[RL][4];
    v4i sr[RL];
    v4i xr[XR];
    const int n16 = FUSED ? in.K / 4 : M * kp / 16;
    stage_load<NW, XR>(FUSED ? reinterpret_cast<const v4i *>(in.x)
                             : reinterpret_cast<const v4i *>(in.act),
                       n16, xr);
    float sa[LR];
    if constexpr (!FUSED) {
#pragma unroll
        for (int j = 0; j < LR; ++j) sa[j] = sa_rows[min(2 * g + j, M - 1)];
    }
    act_begin<NW, XR, FUSED>(in, n16, xr, s_act, red);
    // prime the ring in the steady state's issue order (a lap's quants, then
    // its scales), indices clamped to the segment
#pragma unroll
    for (int u = 0; u < RL; ++u) {
        const int q = min(q0 + u, lastq);
#pragma unroll
        for (int s = 0; s < 4; ++s)
            wr[u][s] = __builtin_nontemporal_load(wp + (size_t)(4 * q + s) * pitch);
        sr[u] = sp[(size_t)q * spitch];
    }
    act_end<NW, XR, FUSED>(in, true, xr, s_act, red, sa[0], blockIdx.x == 0);
    float fs[LR];
#pragma unroll
    for (int j = 0; j < LR; ++j) fs[j] = 0.0f;

    // Lap L of the segment in ring slot U.  REFILL: lap L + RL exists and is
    // loaded into the slot; CHECK: skip padding blocks past nb (only the
    // segment's last laps can hold them).
    auto lap = [&](int L, auto slot, auto w0, bool refill, auto check)
                   __attribute__((always_inline)) {
        constexpr int U = decltype(slot)::value;
        v4i a[4];
#pragma unroll
        for (int s = 0; s < 4; ++s) a[s] = ap[(size_t)(c0 + 4 * L + s) * 4];
        int dt[4][2 * LR];
#pragma unroll
        for (int s = 0; s < 4; ++s) {
            const v4i am = {a[s].x & mlo, a[s].y & mlo, a[s].z & mhi, a[s].w & mhi};
            const v4i d =
                __builtin_amdgcn_mfma_i32_16x16x64_i8(am, wr[U][s], v4i{0, 0, 0, 0}, 0, 0, 0);
#pragma unroll
            for (int i = 0; i < 2 * LR; ++i) dt[s][i] = d[i];
            if (refill)
                wr[U][s] =
                    __builtin_nontemporal_load(wp + (size_t)(c0 + 4 * (L + RL) + s) * pitch);
        }
#pragma unroll
        for (int s = 0; s < 4; ++s) {
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                const int bl = 8 * L + 2 * s + h;   // block within the segment
                const int b = 8 * q0 + bl;
                if (!decltype(check)::value || b < nb) {
                    const unsigned word = (unsigned)sr[U][s];
                    const float d = f16_bits_to_f32(h ? (word >> 16) : (word & 0xFFFFu));
#pragma unroll
                    for (int j = 0; j < LR; ++j) {
                        float t = (float)dt[s][2 * j + h] * sa[j];
                        t = t * d;
                        if constexpr (decltype(w0)::value) fs[j] = fs[j] + t;
                        else if (g < LG) tl[j * tstride + bl] = t;
                    }
                    if constexpr (DEBUG) {
#pragma unroll
                        for (int j = 0; j < LR; ++j) {
                            const int row = 2 * g + j;
                            if (g < LG && row < M && n < N)
                                block_dots[((size_t)row * N + n) * nb + b] = dt[s][2 * j + h];
                        }
                    }
                }
            }
        }
        if (refill) sr[U] = sp[(size_t)(q0 + L + RL) * spitch];
    };

    using T1 = std::true_type;
    using F0 = std::false_type;
    // k full rounds of RL laps; the loop holds the rounds whose refills all
    // exist (branch-free, so the wait counts stay exact); the last full
    // round refills only the remainder's rem laps, which then run last.
    auto sweep = [&](auto w0) __attribute__((always_inline)) {
        const int k = nq / RL, rem = nq - k * RL;
        for (int it = 0; it + 1 < k; ++it)
            static_for<RL>([&](auto u) { lap(it * RL + u, u, w0, true, F0{}); });
        if (k > 0)
            static_for<RL>([&](auto u) { lap((k - 1) * RL + u, u, w0, u < rem, T1{}); });
        static_for<RL>([&](auto u) {
            if (u < rem) lap(k * RL + u, u, w0, false, T1{});
        });
    };
    if (w == 0) sweep(T1{});
    else sweep(F0{});

    if constexpr (S > 1) {
        __syncthreads();
        if (w != 0 || g >= LG) return;
        // continue the block-ordered fold over the later segments; the
        // terms of a segment are contiguous per lane (16-byte reads)
        for (int seg = 1; seg < S; ++seg) {
            const int e0 = split_lo(G, S, seg), e1 = split_lo(G, S, seg + 1);
            const int cnt = max(min(8 * (e1 - e0), nb - 8 * e0), 0);
            const float *ts = term_base(seg);
#pragma unroll
            for (int j = 0; j < LR; ++j) {
                const float4 *t4 = reinterpret_cast<const float4 *>(ts + j * tstride);
                int bl = 0;
                for (; bl + 8 <= cnt; bl += 8) {
                    const float4 u = t4[bl / 4], v = t4[bl / 4 + 1];
                    fs[j] = fs[j] + u.x; fs[j] = fs[j] + u.y; fs[j] = fs[j] + u.z; fs[j] = fs[j] + u.w;
                    fs[j] = fs[j] + v.x; fs[j] = fs[j] + v.y; fs[j] = fs[j] + v.z; fs[j] = fs[j] + v.w;
                }
                for (; bl < cnt; ++bl) fs[j] = fs[j] + ts[j * tstride + bl];
            }
        }
    }
    if (!tile_ok || g >= LG || n >= N) return;
#pragma unroll
    for (int j = 0; j < LR; ++j) {
        const int row = 2 * g + j;
        if (row < M) out[(size_t)row * N + n] = fs[j];
    }
}


struct CfgQ8 {
    int s = 0, tpw = 1, rl = 1, xr = 0;  // s == 0: unsupported
};

// Rows of the Q8_0 kernel instance for m rows: 1, 2 or 4.
inline int mr_of(size_t m) { return m <= 1 ? 1 : m == 2 ? 2 : 4; }

size_t lds_q8(int s, int tpw, size_t m, size_t kp, size_t G) {
    const size_t maxq = (G + s - 1) / s;
    const size_t mr = (size_t)mr_of(m);
    const size_t lr = mr == 1 ? 1 : 2, lg = (mr + 1) / 2;
    return m * kp + (size_t)s * tpw * 16 +
           (size_t)tpw * (s - 1) * lg * 16 * lr * 8 * maxq * 4;
}

// Configuration by the number of 16-row tiles (measured on MI355X).  Many
// tiles: one wave per tile over all of K, two tiles per workgroup, two laps
// in flight; otherwise four waves per tile, with two laps in flight when
// that leaves fewer than about 2000 waves.
CfgQ8 pick_q8(bool fused, size_t n_tiles, size_t m, size_t k, size_t kp, size_t G) {
    CfgQ8 c;
    if (n_tiles >= 1024) { c.s = 1; c.tpw = 2; c.rl = 2; }
    else { c.s = 4; c.rl = n_tiles * 4 >= 2048 ? 1 : 2; }
    const size_t threads = (size_t)c.s * c.tpw * kWave;
    const size_t nx = ceil_div(fused ? k / 4 : m * kp / 16, threads);
    if (c.s == 1) c.xr = nx <= 8 ? 8 : nx <= 24 ? 24 : 0;
    else c.xr = nx <= 4 ? 4 : nx <= 12 ? 12 : 0;
    if (c.xr == 0 || lds_q8(c.s, c.tpw, m, kp, G) > kMaxLds) c.s = 0;
    return c;
}

inline size_t groups_of(const Q8MatrixDev &w) {
    return ((w.n_blocks + 1) / 2 + 3) / 4;  // scale groups holding real blocks
}

template <int MR, int S, int TPW, int RL, int XR, bool FUSED, bool DEBUG>
void launch_q8(ActIn in, size_t m, const float *sa_rows, const Q8MatrixDev &w,
               float *out, int32_t *block_dots, hipStream_t st) {
    const size_t G = groups_of(w);
    hipLaunchKernelGGL((k_gemv_q8_0<MR, S, TPW, RL, XR, FUSED, DEBUG>),
                       dim3((unsigned)ceil_div(w.n_tiles, TPW)), dim3(S * TPW * kWave),
                       lds_q8(S, TPW, m, w.kp, G), st, in, (int)m, (int)w.kp, sa_rows,
                       reinterpret_cast<const v4i *>(w.tiles),
                       reinterpret_cast<const v4i *>(w.scales), (int)w.n_out,
                       (int)w.n_tiles, (int)G, (int)w.n_blocks, out, block_dots);
}

template <int MR, bool FUSED, bool DEBUG>
void dispatch_q8(CfgQ8 c, ActIn in, size_t m, const float *sa_rows, const Q8MatrixDev &w,
                 float *out, int32_t *block_dots, hipStream_t st) {
#define MRI_Q8(S_, TPW_, RL_, XR_)                                                        \
    if (c.s == S_ && c.tpw == TPW_ && c.rl == RL_ && c.xr == XR_)                         \
        return launch_q8<MR, S_, TPW_, RL_, XR_, FUSED, DEBUG>(in, m, sa_rows, w, out,    \
                                                               block_dots, st);
    MRI_Q8(1, 2, 2, 8) MRI_Q8(1, 2, 2, 24)
    MRI_Q8(4, 1, 1, 4) MRI_Q8(4, 1, 1, 12)
    MRI_Q8(4, 1, 2, 4) MRI_Q8(4, 1, 2, 12)
#undef MRI_Q8
}

template <int MR, bool FUSED>
void dispatch_q8_dbg(bool dbg, CfgQ8 c, ActIn in, size_t m, const float *sa_rows,
                     const Q8MatrixDev &w, float *out, int32_t *block_dots, hipStream_t st) {
    if (dbg) dispatch_q8<MR, FUSED, true>(c, in, m, sa_rows, w, out, block_dots, st);
    else dispatch_q8<MR, FUSED, false>(c, in, m, sa_rows, w, out, nullptr, st);
}

}  // namespace

bool gemv_q8_supported(bool fused, size_t m, size_t n_tiles, size_t k, size_t kp) {
    const size_t G = ((k / kQK + 1) / 2 + 3) / 4;
    return m >= 1 && m <= (size_t)kMaxM && pick_q8(fused, n_tiles, m, k, kp, G).s > 0;
}

mri_status launch_gemv_q8_0(const float *x, const int8_t *act, size_t m,
                            const float *sa_rows, const Q8MatrixDev &w, float *out,
                            int32_t *block_dots, float *scales_out, hipStream_t st) {
    if (w.n_tiles == 0 || m == 0) return MRI_OK;
    const CfgQ8 c = pick_q8(x != nullptr, w.n_tiles, m, w.k_in, w.kp, groups_of(w));
    if (c.s == 0) return set_error(MRI_ERR_INVALID_ARGUMENT, "gemv: shape not supported");
    const ActIn in{x, act, (int)w.k_in, nullptr, scales_out};
    const bool dbg = block_dots != nullptr;
    if (x) {
        dispatch_q8_dbg<1, true>(dbg, c, in, m, nullptr, w, out, block_dots, st);
    } else {
        if (m == 1) dispatch_q8_dbg<1, false>(dbg, c, in, m, sa_rows, w, out, block_dots, st);
        else if (m == 2) dispatch_q8_dbg<2, false>(dbg, c, in, m, sa_rows, w, out, block_dots, st);
        else dispatch_q8_dbg<4, false>(dbg, c, in, m, sa_rows, w, out, block_dots, st);
    }
    MRI_LAUNCHED("k_gemv_q8_0");
    return MRI_OK;
}

}  // namespace mri
