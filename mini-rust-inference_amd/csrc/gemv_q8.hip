// gemv_q8.hip — Q8_0 decode GEMV (M <= 4): matmul_q8_0_direct
// (q8_direct.rs:229-289) on the tile-major lap blocks (4 MFMA chunks of
// quants followed by their f16 scales).
#include "gemv_common.hpp"

namespace mri {
using namespace gemv;
namespace {

// ---------------------------------------------------------------------------
// Q8_0 (and, with W4, Q4_0 weights for the W4A8 path: the same computation
// on 4-bit quants).  One v_mfma_i32_16x16x64_i8 per chunk computes both of
// its blocks:
// A row m = 2*row + h carries activation row `row` restricted to block
// 2p + h (the other 8 bytes of the lane's 16 are zeroed; the weight chunk
// keeps both blocks), so result register i of lane group g holds the exact
// int32 dot of activation row 2g + i/2 with block 2p + (i & 1) of output
// channel n = 16T + l%16.  MR (1, 2 or 4: rows of the instance) fixes how
// many lane groups hold results.
//
// A workgroup holds TPW tiles of S waves each; its waves share the
// activation staging.  A tile's K is swept in laps of one scale group
// (4 chunks = 8 blocks) dealt out round-robin: in round R wave w takes lap
// R*S + w, so each round covers S consecutive laps.  Per lap a wave runs
// the MFMAs of its chunks (each followed by the refill of its ring slot
// with the chunk RL laps ahead) and forms the eight terms
// t_b = ((f32)dot_b * s_a) * d_b (q8_direct.rs:281).  Wave 0 adds its own
// terms to the running sum at once; the other waves leave theirs in LDS.
// Every round ends with an LDS-only barrier, after which wave 0 adds the
// round's remaining S-1 laps in block order.  The f32 result is therefore
// bit-identical to the sequential reference, and only the last round's
// terms remain to be added after the sweep.
//
// W4: a lap's quants are two 16-byte loads per lane instead of four; the B
// operand of a chunk is unpacked from two u32 words by moving each nibble
// to the high half of its byte, which gives 16 * quant as int8 (the stored
// nibble is the quant's 4-bit two's complement), so the MFMA's int32 result
// is 16 times the block dot and an arithmetic shift by 4 recovers it.
// ---------------------------------------------------------------------------

// Barrier for LDS traffic only: waits for this wave's LDS operations, not
// for its outstanding global loads (the ring stays in flight).
__device__ inline void lds_barrier() {
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

template <int MR, int S, int TPW, int RL, int XR, bool FUSED, bool OPS, bool DEBUG, bool W4>
__global__ __launch_bounds__(S * TPW * kWave) void k_gemv_q8_0(
    ActIn in, int M, int kp, const float *__restrict__ sa_rows,
    const v4i *__restrict__ laps, int N, int n_tiles, int G, int nb, float *__restrict__ out,
    int32_t *__restrict__ block_dots) {
    constexpr int NW = S * TPW;               // waves per workgroup
    constexpr int LR = MR == 1 ? 1 : 2;       // rows per result lane
    constexpr int LG = (MR + 1) / 2;          // lane groups holding results
    constexpr int TW = 8 * LR;                // terms per result lane per lap
    static_assert(!FUSED || MR == 1, "the fused prologue quantizes one row");
    extern __shared__ v4i s_lds[];
    const int wl = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int tw_ = wl / S;                   // tile of the wave within the WG
    const int w = wl - tw_ * S;               // lap slot of the wave
    const int T = blockIdx.x * TPW + tw_;
    const bool tile_ok = T < n_tiles;
    const int Tc = tile_ok ? T : n_tiles - 1; // address of a missing tile
    const int l = threadIdx.x & 63;
    const int r = l & 15, g = l >> 4;
    const int NR = (G + S - 1) / S;           // rounds
    const int nq = tile_ok && w < G ? (G - w + S - 1) / S : 0;  // laps of this wave
    // lap block q of the tile: quant piece s at v4i offset s * 64 (+ lane),
    // its scales at SO (+ row)
    constexpr size_t LB = (W4 ? kQ4LapBytes : kQ8LapBytes) / 16;
    constexpr int SO = W4 ? 128 : 256;
    constexpr int NP = W4 ? 2 : 4;            // quant pieces per lap and lane
    const v4i *wp = laps + (size_t)Tc * G * LB + l;
    const v4i *sp = laps + (size_t)Tc * G * LB + SO + r;
    const int n = T * 16 + r;

    // LDS: [act M*kp][red NW floats][terms 2 x TPW x (S-1) x LG x 16 x TW floats]
    int8_t *s_act = reinterpret_cast<int8_t *>(s_lds);
    float *red = reinterpret_cast<float *>(s_act + (size_t)M * kp);
    float *terms = red + 4 * NW;
    auto tslot = [&](int par, int ww) {  // terms of wave ww >= 1 in round parity par, this lane
        return terms +
               ((((size_t)(par * TPW + tw_) * (S - 1) + (ww - 1)) * LG + (g < LG ? g : 0)) * 16 + r) * TW;
    };

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
    v4i wn[XR];  // RMS norm weights (row operations)
    if constexpr (FUSED && OPS) {
        if (in.norm_w) stage_load<NW, XR>(reinterpret_cast<const v4i *>(in.norm_w), n16, wn);
    }
    float sa[LR];
    if constexpr (!FUSED) {
#pragma unroll
        for (int j = 0; j < LR; ++j) sa[j] = sa_rows[min(2 * g + j, M - 1)];
    }
    // prime the ring in the steady state's issue order (a lap's quants, then
    // its scales), lap indices clamped to the tile.  The activation loads
    // were issued first, so they return first, and the prologue below waits
    // for them alone while the ring's loads stay in flight.  The scheduling
    // barrier keeps the compiler from moving activation loads after the
    // ring's (it did with 12 pieces per thread, and the prologue then waited
    // for weight loads).
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int u = 0; u < RL; ++u) {
        const int q = min(min(u, max(nq - 1, 0)) * S + w, G - 1);
#pragma unroll
        for (int s = 0; s < NP; ++s)
            wr[u][s] = __builtin_nontemporal_load(wp + (size_t)q * LB + s * 64);
        sr[u] = sp[(size_t)q * LB];
    }
    act_begin<NW, XR, FUSED, OPS>(in, n16, xr, s_act, red);
    act_end<NW, XR, FUSED, OPS>(in, true, xr, wn, s_act, red, sa[0], blockIdx.x == 0);
    float fs[LR];
#pragma unroll
    for (int j = 0; j < LR; ++j) fs[j] = 0.0f;

    // End of round R: wave 0 adds laps R*S+1 .. R*S+S-1 (those that exist)
    // in block order.
    auto round_end = [&](int R) __attribute__((always_inline)) {
        if constexpr (S > 1) {
            lds_barrier();
            if (w == 0) {
                float4 tv[S - 1][TW / 4];
#pragma unroll
                for (int ww = 1; ww < S; ++ww) {
                    const float4 *src = reinterpret_cast<const float4 *>(tslot(R & 1, ww));
#pragma unroll
                    for (int i = 0; i < TW / 4; ++i) tv[ww - 1][i] = src[i];
                }
#pragma unroll
                for (int ww = 1; ww < S; ++ww) {
                    const int cnt = min(nb - 8 * (R * S + ww), 8);  // valid blocks of the lap
#pragma unroll
                    for (int j = 0; j < LR; ++j) {
#pragma unroll
                        for (int i = 0; i < 8; ++i) {
                            const float4 v4 = tv[ww - 1][(8 * j + i) / 4];
                            const int e = i & 3;
                            const float t = e == 0 ? v4.x : e == 1 ? v4.y : e == 2 ? v4.z : v4.w;
                            const float f = fs[j] + t;
                            fs[j] = i < cnt ? f : fs[j];
                        }
                    }
                }
            }
        }
    };

    // Lap L of this wave (round L, lap index L*S + w) in ring slot U.
    // REFILL: lap L + RL exists and is loaded into the slot; CHECK: skip
    // padding blocks past nb (only the tile's last lap can hold them).
    auto lap = [&](int L, auto slot, bool refill, auto check) __attribute__((always_inline)) {
        constexpr int U = decltype(slot)::value;
        const int q = L * S + w;
        v4i a[4];
#pragma unroll
        for (int s = 0; s < 4; ++s) a[s] = ap[(size_t)(4 * q + s) * 4];
        int dt[4][2 * LR];
#pragma unroll
        for (int s = 0; s < 4; ++s) {
            const v4i am = {a[s].x & mlo, a[s].y & mlo, a[s].z & mhi, a[s].w & mhi};
            v4i bw;
            if constexpr (W4) {
                const v4i pc = wr[U][s >> 1];
                const int w0 = (s & 1) ? pc.z : pc.x, w1 = (s & 1) ? pc.w : pc.y;
                constexpr int kHi = (int)0xF0F0F0F0u;
                bw = v4i{(w0 << 4) & kHi, w0 & kHi, (w1 << 4) & kHi, w1 & kHi};
            } else {
                bw = wr[U][s];
            }
            const v4i d = __builtin_amdgcn_mfma_i32_16x16x64_i8(am, bw, v4i{0, 0, 0, 0}, 0, 0, 0);
#pragma unroll
            for (int i = 0; i < 2 * LR; ++i) dt[s][i] = W4 ? d[i] >> 4 : d[i];
            if (refill && (!W4 || (s & 1))) {
                const int pi = W4 ? s >> 1 : s;
                wr[U][pi] = __builtin_nontemporal_load(wp + (size_t)(q + RL * S) * LB + pi * 64);
            }
        }
        float tv[LR][8];
#pragma unroll
        for (int s = 0; s < 4; ++s) {
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                const unsigned word = (unsigned)sr[U][s];
                const float d = f16_bits_to_f32(h ? (word >> 16) : (word & 0xFFFFu));
#pragma unroll
                for (int j = 0; j < LR; ++j) {
                    float t = (float)dt[s][2 * j + h] * sa[j];
                    tv[j][2 * s + h] = t * d;
                }
            }
        }
        if (w == 0) {
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const int b = 8 * q + i;
                if (!decltype(check)::value || b < nb) {
#pragma unroll
                    for (int j = 0; j < LR; ++j) fs[j] = fs[j] + tv[j][i];
                }
            }
        } else if (g < LG) {
            float4 *dst = reinterpret_cast<float4 *>(tslot(L & 1, w));
#pragma unroll
            for (int j = 0; j < LR; ++j) {
                dst[2 * j] = float4{tv[j][0], tv[j][1], tv[j][2], tv[j][3]};
                dst[2 * j + 1] = float4{tv[j][4], tv[j][5], tv[j][6], tv[j][7]};
            }
        }
        if constexpr (DEBUG) {
#pragma unroll
            for (int s = 0; s < 4; ++s) {
#pragma unroll
                for (int h = 0; h < 2; ++h) {
                    const int b = 8 * q + 2 * s + h;
#pragma unroll
                    for (int j = 0; j < LR; ++j) {
                        const int row = 2 * g + j;
                        if (b < nb && g < LG && row < M && n < N)
                            block_dots[((size_t)row * N + n) * nb + b] = dt[s][2 * j + h];
                    }
                }
            }
        }
        if (refill) sr[U] = sp[(size_t)(q + RL * S) * LB];
        round_end(L);
    };

    using T1 = std::true_type;
    using F0 = std::false_type;
    // k full rounds of RL laps; the loop holds the rounds whose refills all
    // exist (branch-free, so the wait counts stay exact); the last full
    // round refills only the remainder's rem laps, which then run last.
    {
        const int k = nq / RL, rem = nq - k * RL;
        for (int it = 0; it + 1 < k; ++it)
            static_for<RL>([&](auto u) { lap(it * RL + u, u, true, F0{}); });
        if (k > 0)
            static_for<RL>([&](auto u) { lap((k - 1) * RL + u, u, u < rem, T1{}); });
        static_for<RL>([&](auto u) {
            if (u < rem) lap(k * RL + u, u, false, T1{});
        });
    }
    // rounds in which this wave has no lap (the barrier count is uniform)
    for (int R = nq; R < NR; ++R) round_end(R);

    if (w != 0 || !tile_ok) return;
    if constexpr (OPS) {  // one row: lanes 0-15 hold channels 16T .. 16T+15
        const float pv = __shfl_xor(fs[0], 1);
        if (g == 0 && n < N) row_store(in, out, n, fs[0], pv);
        return;
    }
    if (g >= LG || n >= N) return;
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
    (void)G;
    const size_t mr = (size_t)mr_of(m);
    const size_t lr = mr == 1 ? 1 : 2, lg = (mr + 1) / 2;
    return m * kp + (size_t)s * tpw * 16 + 2 * (size_t)tpw * (s - 1) * lg * 16 * lr * 8 * 4;
}

// Configuration by the number of 16-row tiles (measured on MI355X): four
// waves per tile, with two laps in flight when that leaves fewer than
// about 2000 waves, else one.
CfgQ8 pick_q8(bool fused, size_t n_tiles, size_t m, size_t k, size_t kp, size_t G) {
    CfgQ8 c;
    c.s = 4;
    c.rl = n_tiles * 4 >= 2048 ? 1 : 2;
    const size_t threads = (size_t)c.s * c.tpw * kWave;
    const size_t nx = ceil_div(fused ? k / 4 : m * kp / 16, threads);
    if (c.s == 1) c.xr = nx <= 8 ? 8 : nx <= 24 ? 24 : 0;
    else c.xr = nx <= 4 ? 4 : nx <= 12 ? 12 : 0;
    if (c.xr == 0 || lds_q8(c.s, c.tpw, m, kp, G) > kMaxLds) c.s = 0;
    return c;
}

inline size_t groups_of(const Q8MatrixDev &w) { return w.laps_per_tile(); }

template <int MR, int S, int TPW, int RL, int XR, bool FUSED, bool OPS, bool DEBUG, bool W4>
void launch_q8(ActIn in, size_t m, const float *sa_rows, const Q8MatrixDev &w,
               float *out, int32_t *block_dots, hipStream_t st) {
    const size_t G = groups_of(w);
    hipLaunchKernelGGL((k_gemv_q8_0<MR, S, TPW, RL, XR, FUSED, OPS, DEBUG, W4>),
                       dim3((unsigned)ceil_div(w.n_tiles, TPW)), dim3(S * TPW * kWave),
                       lds_q8(S, TPW, m, w.kp, G), st, in, (int)m, (int)w.kp, sa_rows,
                       reinterpret_cast<const v4i *>(w.laps), (int)w.n_out,
                       (int)w.n_tiles, (int)G, (int)w.n_blocks, out, block_dots);
}

template <int MR, bool FUSED, bool OPS, bool DEBUG>
void dispatch_q8(CfgQ8 c, ActIn in, size_t m, const float *sa_rows, const Q8MatrixDev &w,
                 float *out, int32_t *block_dots, hipStream_t st) {
#define MRI_Q8(S_, TPW_, RL_, XR_)                                                         \
    if (c.s == S_ && c.tpw == TPW_ && c.rl == RL_ && c.xr == XR_)                          \
        return w.w4 ? launch_q8<MR, S_, TPW_, RL_, XR_, FUSED, OPS, DEBUG, true>(          \
                          in, m, sa_rows, w, out, block_dots, st)                          \
                    : launch_q8<MR, S_, TPW_, RL_, XR_, FUSED, OPS, DEBUG, false>(         \
                          in, m, sa_rows, w, out, block_dots, st);
    MRI_Q8(4, 1, 1, 4) MRI_Q8(4, 1, 1, 12)
    MRI_Q8(4, 1, 2, 4) MRI_Q8(4, 1, 2, 12)
#undef MRI_Q8
}

template <int MR, bool FUSED>
void dispatch_q8_dbg(bool dbg, CfgQ8 c, ActIn in, size_t m, const float *sa_rows,
                     const Q8MatrixDev &w, float *out, int32_t *block_dots, hipStream_t st) {
    if (dbg) dispatch_q8<MR, FUSED, false, true>(c, in, m, sa_rows, w, out, block_dots, st);
    else dispatch_q8<MR, FUSED, false, false>(c, in, m, sa_rows, w, out, nullptr, st);
}

}  // namespace

bool gemv_q8_supported(bool fused, size_t m, size_t n_tiles, size_t k, size_t kp) {
    const size_t G = kp / kQ8LapK;
    return m >= 1 && m <= (size_t)kMaxM && pick_q8(fused, n_tiles, m, k, kp, G).s > 0;
}

mri_status launch_gemv_q8_0(const float *x, const int8_t *act, size_t m,
                            const float *sa_rows, const Q8MatrixDev &w, float *out,
                            int32_t *block_dots, float *scales_out, hipStream_t st,
                            const RowOps &ops) {
    if (w.n_tiles == 0 || m == 0) return MRI_OK;
    const CfgQ8 c = pick_q8(x != nullptr, w.n_tiles, m, w.k_in, w.kp, groups_of(w));
    if (c.s == 0) return set_error(MRI_ERR_INVALID_ARGUMENT, "gemv: shape not supported");
    if (!row_ops_ok(x, ops))
        return set_error(MRI_ERR_INVALID_ARGUMENT, "gemv: row operations need the fused path");
    const ActIn in(x, act, (int)w.k_in, nullptr, scales_out, ops);
    const bool dbg = block_dots != nullptr;
    if (ops.any()) {
        if (dbg) return set_error(MRI_ERR_INVALID_ARGUMENT, "gemv: row operations without debug outputs");
        dispatch_q8<1, true, true, false>(c, in, m, nullptr, w, out, nullptr, st);
    } else if (x) {
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
