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
// One row (MR = 1, the chained form): chunk s of a lap fills rows 2s and
// 2s + 1 of its MFMA's A operand (blocks 2s, 2s + 1) and leaves the other
// rows zero, so the lap's four MFMAs accumulate into one result: lane
// (r, g < 2) holds blocks 4g .. 4g + 3 of the lap for channel r, and each
// lane folds four terms per lap instead of eight terms of which three
// quarters belong to zero rows.  The A operand comes from the masked row
// layout (masked_off), where each lane's 16 bytes are one load with the
// other block's half already zero; lanes without a row in a chunk read a
// zero line.  The accumulator starts at kDotBias, so the block dots read
// as f32 with one subtraction.  The two lane groups' sums are added after
// the sweep.
//
// A workgroup holds TPW tiles of S waves each; its waves share the
// activation staging.  A tile's K is swept in laps of one scale group
// (4 chunks = 8 blocks) dealt out round-robin: in round R wave w takes lap
// R*S + w, so each round covers S consecutive laps.  Per lap a wave runs
// the MFMAs of its chunks (each followed by the refill of its ring slot
// with the chunk RL laps ahead) and adds the eight terms
// t_b = ((f32)dot_b * s_a) * d_b (q8_direct.rs:281) to its own running
// f32 sum, in block order.  After the sweep the S wave sums of a tile are
// added through LDS in wave order (one barrier), so the result is
// deterministic; it differs from the reference's single left-to-right sum
// only in f32 rounding, within 1e-5 * max(|out|, sum_b |t_b|).  The int32
// block dots are exact.  (Keeping the reference's order needed an LDS
// barrier per round and measured ~0.3 us slower at [1,4096]x[4096,11008].)
//
// LAZY (the plain fused row, 512-1023 tiles): the prologue stages the f32
// row in LDS and reduces max|x| (one barrier) without quantizing it; each
// wave then quantizes only the laps it consumes, one lap (4 values a lane,
// the same round-half-away and clamp) into a masked 512-byte area of its own,
// after the previous lap's MFMAs and refills, while the next lap is in
// flight.  Every workgroup re-quantizes the row it uses; quantizing it all
// up front put that VALU work ahead of every wave's first lap.
//
// W4: a lap's quants are two 16-byte loads per lane instead of four; the B
// operand of a chunk is unpacked from two u32 words by moving each nibble
// to the high half of its byte, which gives 16 * quant as int8 (the stored
// nibble is the quant's 4-bit two's complement), so the MFMA's int32 result
// is 16 times the block dot and an arithmetic shift by 4 recovers it.
// ---------------------------------------------------------------------------

template <int MR, int S, int TPW, int RL, int XR, bool FUSED, bool OPS, bool DEBUG, bool W4,
          bool LAZY = false>
__global__ __launch_bounds__(S * TPW * kWave) void k_gemv_q8_0(
    ActIn in, int M, int kp, const float *__restrict__ sa_rows,
    const v4i *__restrict__ laps, int N, int n_tiles, int G, int nb, float *__restrict__ out,
    int32_t *__restrict__ block_dots) {
    constexpr int NW = S * TPW;               // waves per workgroup
    constexpr int LR = MR == 1 ? 1 : 2;       // rows per result lane
    constexpr int LG = (MR + 1) / 2;          // lane groups holding results
    static_assert(!FUSED || MR == 1, "the fused prologue quantizes one row");
    static_assert(!LAZY || FUSED, "lap-wise quantization: the fused row");
    // the plain lap-wise row with one lap in flight and up to four staged
    // pieces quantizes from the staging registers (0-0.06 us faster at
    // [1,4096]x[4096,11008] on two boxes, 2 % at K = 992, same outputs);
    // with two laps in flight the compiler indexed
    // the pieces through scratch memory and the kernels ran 33-50 % slower,
    // so those stage the row in LDS (a fully unrolled lap sequence, which
    // indexes the pieces statically, ran 10.3 against 9.05 us)
    constexpr bool kRegRow = LAZY && !OPS && RL == 1 && XR <= 4;
    static_assert(!kRegRow || TPW == 1, "registers hold this wave's laps only with one tile");
    extern __shared__ v4i s_lds[];
    const int wl = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int tw_ = wl / S;                   // tile of the wave within the WG
    const int w = wl - tw_ * S;               // lap slot of the wave
    const int T = blockIdx.x * TPW + tw_;
    const bool tile_ok = T < n_tiles;
    const int Tc = tile_ok ? T : n_tiles - 1; // address of a missing tile
    const int l = threadIdx.x & 63;
    const int r = l & 15, g = l >> 4;
    const int nq = tile_ok && w < G ? (G - w + S - 1) / S : 0;  // laps of this wave
    // lap block q of the tile: quant piece s at v4i offset s * 64 (+ lane),
    // its scales at SO (+ row)
    constexpr size_t LB = (W4 ? kQ4LapBytes : kQ8LapBytes) / 16;
    constexpr int SO = W4 ? 128 : 256;
    constexpr int NP = W4 ? 2 : 4;            // quant pieces per lap and lane
    const v4i *wp = laps + (size_t)Tc * G * LB + l;
    const int n = T * 16 + r;
    // CH: one row; the four MFMAs of a lap accumulate into one result
    // (scale loads: the 4 f16 scales of blocks 4(g%2) .. + 3 of channel r)
    constexpr bool CH = MR == 1;
    using SR = std::conditional_t<CH, v2i, v4i>;
    const SR *sp = reinterpret_cast<const SR *>(laps + (size_t)Tc * G * LB + SO + r) +
                   (CH ? (g & 1) : 0);
    constexpr size_t LBS = CH ? 2 * LB : LB;  // lap stride in SR units

    // LDS: [act: M*kp int8; CH: the masked row (2*kp bytes) and a 16-byte
    // zero line; LAZY: the f32 row (kp floats)][red NW floats][wave sums TPW
    // x (S-1) x LG x 16 x LR floats][LAZY: one masked lap (512 bytes) and a
    // zero line per wave]
    constexpr int kLapArea = 528;
    int8_t *s_act = reinterpret_cast<int8_t *>(s_lds);
    float *red = reinterpret_cast<float *>(
        s_act + (LAZY ? (size_t)4 * kp : CH ? (size_t)2 * kp + 16 : (size_t)M * kp));
    float *sums = red + 4 * NW;
    int8_t *s_lap = reinterpret_cast<int8_t *>(sums + (size_t)TPW * (S - 1) * LG * 16 * LR) +
                    (size_t)wl * kLapArea;
    auto sslot = [&](int ww) {  // sums of wave ww >= 1 of this tile, this lane
        return sums + ((((size_t)tw_ * (S - 1) + (ww - 1)) * LG + (g < LG ? g : 0)) * 16 + r) * LR;
    };

    // A operand: lane (r, g) reads activation row r/2 (16 bytes of lane
    // group g of each chunk) and keeps the half of block 2p + (r & 1).
    const int arow = r >> 1;
    const bool aval = arow < M;
    const int mlo = (aval && !(r & 1)) ? -1 : 0;
    const int mhi = (aval && (r & 1)) ? -1 : 0;
    const v4i *ap = reinterpret_cast<const v4i *>(LAZY ? s_lap : s_act + (size_t)(aval ? arow : 0) * kp) + g;
    // CH: lane (r, g), r < 8, feeds row r of chunk r/2's MFMA from entry
    // r + 8g of the lap's masked area; every other (lane, MFMA) pair reads
    // the zero line.
    const int own_s = r < 8 ? r >> 1 : -1;
    const int8_t *a_ent = (LAZY ? s_lap : s_act) + 16 * (r + 8 * g);
    const int8_t *a_zero = LAZY ? s_lap + 512 : s_act + 2 * (size_t)kp;

    v4i wr[RL][4];
    SR sr[RL];
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
        sr[u] = sp[(size_t)q * LBS];
    }
    RowDst dst{};  // row operations: wave 0 stores the tile's outputs
    if constexpr (OPS) {
        if (w == 0) dst = row_dst(in, out, n, N);
    }
    if constexpr (CH) {  // zero words of the masked areas, the zero line
        if constexpr (LAZY) {
            *reinterpret_cast<int *>(s_lap + (masked_off(4 * l) ^ 8)) = 0;
            if (l < 4) reinterpret_cast<int *>(s_lap + 512)[l] = 0;
        } else {
            if (threadIdx.x < 4) reinterpret_cast<int *>(s_act + 2 * (size_t)kp)[threadIdx.x] = 0;
        }
    }
    if constexpr (FUSED && OPS) {
        if (in.up) act_swiglu<NW, XR>(in, xr, wn);
    }
    float inv = 0.0f;  // LAZY: 1 / scale of the row
    if constexpr (LAZY) {
        // the row and its scale as act_begin / act_end compute them, the
        // f32 row staged in LDS; each wave quantizes the laps it consumes
        // (quant_lap)
        act_begin<NW, XR, FUSED, OPS>(in, n16, xr, s_act, red);
        inv = act_end_lazy<NW, XR, OPS, !kRegRow>(in, xr, wn, reinterpret_cast<float *>(s_act),
                                                  red, sa[0], blockIdx.x == 0);
    } else {
        act_begin<NW, XR, FUSED, OPS, CH>(in, n16, xr, s_act, red);
        act_end<NW, XR, FUSED, OPS>(in, CH ? kLayMasked : kLayPerm, xr, wn, s_act, red, sa[0],
                                    blockIdx.x == 0);
    }
    // LAZY: quantize lap q = L * S + w of the row (lane l: elements
    // 256q + 4l .. + 3, zero past K) into this wave's 256-byte area,
    // chunk-permuted.  kRegRow: those elements are this thread's staged
    // piece L (piece e of thread 64w + l is float4 64 (w + S e) + l), so
    // they come from registers instead of LDS.
    auto quant_lap = [&](int L) __attribute__((always_inline)) {
        const int q = L * S + w;
        const int kk = 256 * q + 4 * l;
        float4 v = float4{0.0f, 0.0f, 0.0f, 0.0f};
        if constexpr (kRegRow) {
            v4i pc = xr[0];
#pragma unroll
            for (int e = 1; e < XR; ++e) pc = L == e ? xr[e] : pc;
            if (kk < in.K) v = __builtin_bit_cast(float4, pc);
        } else {
            if (kk < in.K) v = reinterpret_cast<const float4 *>(s_act)[kk >> 2];
        }
        // the data word of elements 4l .. 4l + 3 of the lap (its zero word
        // was written once)
        *reinterpret_cast<int *>(s_lap + masked_off(4 * l)) = quant4_packed(v, inv);
    };
    if constexpr (LAZY) {
        if (nq > 0) quant_lap(0);
    }
    float fs[LR];
#pragma unroll
    for (int j = 0; j < LR; ++j) fs[j] = 0.0f;

    // Lap L of this wave (round L, lap index L*S + w) in ring slot U.
    // REFILL: lap L + RL exists and is loaded into the slot; CHECK: skip
    // padding blocks past nb (only the tile's last lap can hold them).
    auto lap = [&](int L, auto slot, bool refill, auto check) __attribute__((always_inline)) {
        constexpr int U = decltype(slot)::value;
        const int q = L * S + w;
        if constexpr (CH) {
            // rows 2s, 2s + 1 of MFMA s are blocks 2s, 2s + 1 of the lap and
            // its other rows are zero, so one accumulator collects the lap:
            // lane (r, g < 2) ends with blocks 4g .. 4g + 3 of channel r in
            // registers 0-3, each as the bits of kDotBiasF + dot
            const int8_t *ent = a_ent + (LAZY ? 0 : (size_t)512 * q);
            v4i a[4];
#pragma unroll
            for (int s = 0; s < 4; ++s)
                a[s] = *reinterpret_cast<const v4i *>(s == own_s ? ent : a_zero);
            v4i c = v4i{kDotBias, kDotBias, kDotBias, kDotBias};
#pragma unroll
            for (int s = 0; s < 4; ++s) {
                v4i bw;
                if constexpr (W4) {
                    const v4i pc = wr[U][s >> 1];
                    const int w0 = (s & 1) ? pc.z : pc.x, w1 = (s & 1) ? pc.w : pc.y;
                    constexpr int kHi = (int)0xF0F0F0F0u;
                    bw = v4i{(w0 << 4) & kHi, w0 & kHi, (w1 << 4) & kHi, w1 & kHi};
                } else {
                    bw = wr[U][s];
                }
                c = __builtin_amdgcn_mfma_i32_16x16x64_i8(a[s], bw, c, 0, 0, 0);
                if (refill && (!W4 || (s & 1))) {
                    const int pi = W4 ? s >> 1 : s;
                    wr[U][pi] = __builtin_nontemporal_load(wp + (size_t)(q + RL * S) * LB + pi * 64);
                }
            }
            // t_b = ((f32)dot_b * s_a) * d_b (q8_direct.rs:281), in block order
            // per lane (W4: the MFMA holds 16 * dot, and (f32)(16 dot) / 16 is
            // exact)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                // (a copy first: __builtin_bit_cast of the element expression
                // c[i] read element 0 for every i)
                const int ci = c[i];
                float dv = __builtin_bit_cast(float, ci) - kDotBiasF;
                if constexpr (W4) dv = dv * 0.0625f;
                const unsigned word = (unsigned)sr[U][i >> 1];
                const float d = f16_bits_to_f32((i & 1) ? (word >> 16) : (word & 0xFFFFu));
                float t = dv * sa[0];
                t = t * d;
                if (!decltype(check)::value || 8 * q + 4 * g + i < nb) fs[0] = fs[0] + t;
            }
            if constexpr (DEBUG) {
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const int b = 8 * q + 4 * g + i;
                    if (b < nb && g < 2 && n < N)
                        block_dots[(size_t)n * nb + b] =
                            W4 ? (c[i] - kDotBias) >> 4 : c[i] - kDotBias;
                }
            }
        } else {
        v4i a[4];
#pragma unroll
        for (int s = 0; s < 4; ++s) a[s] = ap[(size_t)((LAZY ? 0 : 4 * q) + s) * 4];
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
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const int b = 8 * q + i;
            if (!decltype(check)::value || b < nb) {
#pragma unroll
                for (int j = 0; j < LR; ++j) fs[j] = fs[j] + tv[j][i];
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
        }
        if (refill) sr[U] = sp[(size_t)(q + RL * S) * LBS];
        if constexpr (LAZY) {
            if (L + 1 < nq) quant_lap(L + 1);  // while the next laps are in flight
        }
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
    // CH: lane group 1 holds blocks 4-7 of every lap
    if constexpr (CH) fs[0] = fs[0] + __shfl_xor(fs[0], 16);
    // the wave sums of the tile, added in wave order
    if constexpr (S > 1) {
        if (w != 0 && g < LG) {
#pragma unroll
            for (int j = 0; j < LR; ++j) sslot(w)[j] = fs[j];
        }
        __syncthreads();
        if (w == 0 && g < LG) {
            const int sw = min(S, G);  // waves past G hold no lap
            for (int ww = 1; ww < sw; ++ww) {
#pragma unroll
                for (int j = 0; j < LR; ++j) fs[j] = fs[j] + sslot(ww)[j];
            }
        }
    }
    if (w != 0 || !tile_ok) return;
    if constexpr (OPS) {  // one row: lanes 0-15 hold channels 16T .. 16T+15
        const float pv = __shfl_xor(fs[0], 1);
        if (g == 0 && n < N) row_store(in, dst, n, fs[0], pv);
        if (in.arg_keys) row_argmax_key(in.arg_keys, T, fs[0], n, g == 0 && n < N);
        return;
    }
    if (g >= LG || n >= N) return;
#pragma unroll
    for (int j = 0; j < LR; ++j) {
        const int row = 2 * g + j;
        if (row < M) out[(size_t)row * N + n] = fs[j];
    }
}


// ---------------------------------------------------------------------------
// Q4_0 with f32 activations (W4A32, matmul_q4_0_dequant, q4_0.rs:94-181) on
// the same 4-bit lap blocks and GEMV skeleton: x is staged in LDS as f32
// (no quantization), each lane dequantizes its 8 elements of each block in
// registers (nibble -> signed int -> f32, the reference's (nibble - 8) as
// the stored nibble is its 4-bit two's complement) and accumulates
// d_b * sum_i x_i * q_i with FMAs.  Lane groups g = l / 16 hold the four
// 8-element slices of a block for row 16T + l % 16; after the sweep they
// are added across lanes (fixed shuffle order) and the S wave sums through
// LDS in wave order.  The reference adds x_k * w_k sequentially over all k;
// the result differs only in f32 rounding (within
// 1e-5 * max(|out|, sum_k |x_k w_k|)).  Word j of lap piece u is block
// 8q + 4u + j; byte i of a word holds elements 8g + i (low nibble) and
// 8g + 4 + i (high nibble).
// ---------------------------------------------------------------------------
template <int MR, int S, int RL, int XR>
__global__ __launch_bounds__(S * kWave) void k_gemv_w4a32(
    const float *__restrict__ x, int M, int K, int kp, const v4i *__restrict__ laps, int N,
    int n_tiles, int G, int nb, float *__restrict__ out) {
    extern __shared__ v4i s_lds[];
    const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int T = blockIdx.x;
    const int l = threadIdx.x & 63;
    const int r = l & 15, g = l >> 4;
    const int nq = w < G ? (G - w + S - 1) / S : 0;  // laps of this wave
    constexpr size_t LB = kQ4LapBytes / 16;
    const v4i *wp = laps + (size_t)T * G * LB + l;
    const v4i *sp = laps + (size_t)T * G * LB + 128 + r;
    // LDS: x rows [MR][kp] f32 (zero past K), then the wave sums
    float *s_x = reinterpret_cast<float *>(s_lds);
    float *sums = s_x + (size_t)MR * kp;

    v4i wr[RL][2];
    v4i sr[RL];
    v4i xr[XR];
    const int k4 = K / 4, kp4 = kp / 4;
    const int n4 = M * kp4;  // float4s of the staged rows
#pragma unroll
    for (int e = 0; e < XR; ++e) {
        const int i = min((int)threadIdx.x + S * kWave * e, n4 - 1);
        const int row = i / kp4, c = i - row * kp4;
        xr[e] = c < k4 ? reinterpret_cast<const v4i *>(x + (size_t)row * K)[c] : v4i{0, 0, 0, 0};
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int u = 0; u < RL; ++u) {
        const int q = min(min(u, max(nq - 1, 0)) * S + w, G - 1);
        wr[u][0] = __builtin_nontemporal_load(wp + (size_t)q * LB);
        wr[u][1] = __builtin_nontemporal_load(wp + (size_t)q * LB + 64);
        sr[u] = sp[(size_t)q * LB];
    }
#pragma unroll
    for (int e = 0; e < XR; ++e) {
        const int i = (int)threadIdx.x + S * kWave * e;
        if (i < n4) reinterpret_cast<v4i *>(s_x)[i] = xr[e];
    }
    __builtin_amdgcn_sched_barrier(0);
    __syncthreads();
    float acc[MR];
#pragma unroll
    for (int j = 0; j < MR; ++j) acc[j] = 0.0f;

    auto lap = [&](int L, auto slot, bool refill) __attribute__((always_inline)) {
        constexpr int U = decltype(slot)::value;
        const int q = L * S + w, qn = q + RL * S;
        const v4i p0 = wr[U][0], p1 = wr[U][1], sc = sr[U];
        if (refill) {
            wr[U][0] = __builtin_nontemporal_load(wp + (size_t)qn * LB);
            wr[U][1] = __builtin_nontemporal_load(wp + (size_t)qn * LB + 64);
            sr[U] = sp[(size_t)qn * LB];
        }
#pragma unroll
        for (int jb = 0; jb < 8; ++jb) {  // block 8q + jb: word jb % 4 of piece jb / 4
            const int b = 8 * q + jb;
            const v4i pc = jb < 4 ? p0 : p1;
            const int wd = pc[jb & 3];
            const unsigned sw = (unsigned)sc[jb >> 1];
            const float d = f16_bits_to_f32((jb & 1) ? (sw >> 16) : (sw & 0xFFFFu));
            float qv[8];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                qv[i] = (float)((wd << (28 - 8 * i)) >> 28);      // low nibble of byte i
                qv[4 + i] = (float)((wd << (24 - 8 * i)) >> 28);  // high nibble
            }
#pragma unroll
            for (int j = 0; j < MR; ++j) {
                const float4 *xa = reinterpret_cast<const float4 *>(
                    s_x + (size_t)j * kp + 32 * b + 8 * g);
                const float4 lo = xa[0], hi = xa[1];
                float p = lo.x * qv[0];
                p = fmaf(lo.y, qv[1], p);
                p = fmaf(lo.z, qv[2], p);
                p = fmaf(lo.w, qv[3], p);
                p = fmaf(hi.x, qv[4], p);
                p = fmaf(hi.y, qv[5], p);
                p = fmaf(hi.z, qv[6], p);
                p = fmaf(hi.w, qv[7], p);
                const float a = fmaf(d, p, acc[j]);
                acc[j] = b < nb ? a : acc[j];
            }
        }
    };
    {
        const int k = nq / RL, rem = nq - k * RL;
        for (int it = 0; it + 1 < k; ++it)
            static_for<RL>([&](auto u) { lap(it * RL + u, u, true); });
        if (k > 0) static_for<RL>([&](auto u) { lap((k - 1) * RL + u, u, u < rem); });
        static_for<RL>([&](auto u) {
            if (u < rem) lap(k * RL + u, u, false);
        });
    }
    // lane groups (fixed order), then waves (in order)
#pragma unroll
    for (int j = 0; j < MR; ++j) {
        float v = acc[j] + __shfl_xor(acc[j], 16);
        acc[j] = v + __shfl_xor(v, 32);
    }
    if constexpr (S > 1) {
        if (w != 0 && l < 16) {
#pragma unroll
            for (int j = 0; j < MR; ++j) sums[((w - 1) * MR + j) * 16 + l] = acc[j];
        }
        __syncthreads();
        if (w != 0) return;
        const int sw_ = min(S, G);
        for (int ww = 1; ww < sw_; ++ww) {
#pragma unroll
            for (int j = 0; j < MR; ++j) acc[j] = acc[j] + sums[((ww - 1) * MR + j) * 16 + r];
        }
    }
    const int n = T * 16 + l;
    if (l < 16 && n < N) {
#pragma unroll
        for (int j = 0; j < MR; ++j)
            if (j < M) out[(size_t)j * N + n] = acc[j];
    }
}

// Lap-wise quantization of the fused row (k_gemv_q8_0's LAZY instances):
// waves per tile and laps in flight by tile count and laps per tile G, from
// A/B runs on one box (us per call, against the row quantized into LDS up
// front): 512-1023 tiles, 4 waves x 1 lap (688 tiles, [1,4096]x[4096,11008]:
// 9.07-9.11 against 9.30-9.34; 8 waves 9.7-9.9, 16 waves 11.1); below 512
// tiles 4 waves x 2 laps at G <= 16 (256 tiles, 4096 -> 4096: 5.07 against
// 5.70) and 8 waves x 2 laps above (11008 -> 4096: 10.07-10.16 against
// 10.62-10.78; 16 waves x 1 lap 10.05).  From 1024 tiles the up-front form
// stays (2000 tiles, 4096 -> 32000: 22.3 against 21.6 with 4 x 1).  The
// row-operation instances of the decode step take it below 512 tiles (the
// o projection with its residual add, down with the SwiGLU prologue: 80.7-
// 80.9 against 81.4 us per token) and, with the one-row chained form, also
// from 512 tiles (q/k/v and gate/up with the RMSNorm prologue, and the W4A8
// lm_head): Q8_0 81.75-82.2 -> 81.1-81.2, W4A8 65.8-66.4 -> 62.3-62.4 us per
// token.  The Q8_0 lm_head (2000 tiles) keeps the up-front form, like the
// matmul entry points from 1024 tiles: lap-wise it took 24.2 against 23.3
// us (rocprof), and the step 81.3 against 80.9-81.1.
constexpr size_t kLazyMaxTiles = 1024;
constexpr size_t kLazyMaxOpsTiles = 1536;  // Q8_0 row operations; W4A8: every count

struct CfgQ8 {
    int s = 0, tpw = 1, rl = 1, xr = 0;  // s == 0: unsupported
    bool lazy = false;                    // lap-wise quantization of the fused row
};

// Rows of the Q8_0 kernel instance for m rows: 1, 2 or 4.
inline int mr_of(size_t m) { return m <= 1 ? 1 : m == 2 ? 2 : 4; }

size_t lds_q8(int s, int tpw, size_t m, size_t kp, size_t G, bool lazy = false) {
    (void)G;
    const size_t mr = (size_t)mr_of(m);
    const size_t lr = mr == 1 ? 1 : 2, lg = (mr + 1) / 2;
    const size_t act = lazy ? 4 * kp : mr == 1 ? 2 * kp + 16 : m * kp;
    return act + (size_t)s * tpw * 16 + (size_t)tpw * (s - 1) * lg * 16 * lr * 4 +
           (lazy ? (size_t)s * tpw * 528 : 0);
}

// Activation pieces per thread of the instances with S waves per tile.
inline int xr_small(int s) { return 16 / s; }
inline int xr_large(int s) { return 48 / s; }

// Configuration by the number of 16-row tiles (measured on MI355X at
// K = 4096 and 11008): four waves per tile and one lap in flight per wave
// from 512 tiles up; below, more waves per tile (8 at K <= 4096, 16 above)
// with two laps in flight, so that the launch still has >= 2048 waves.
CfgQ8 pick_q8(bool fused, size_t n_tiles, size_t m, size_t k, size_t kp, size_t G,
              bool ops = false, bool w4 = false) {
    CfgQ8 c;
    if (fused && m == 1 &&
        n_tiles < (ops ? (w4 ? SIZE_MAX : kLazyMaxOpsTiles) : kLazyMaxTiles)) {
        CfgQ8 z;
        z.s = n_tiles >= 512 || G <= 16 ? 4 : 8;
        // the 4-bit laps of the decode step's row operations: two in flight
        // (half the bytes of a Q8_0 lap; W4A8 layer decode 62.1-62.6 -> 61.2-
        // 61.3 us per token, where Q8_0 took 81.0 -> 81.4-81.9)
        z.rl = n_tiles >= 512 && !(ops && w4) ? 1 : 2;
        z.lazy = true;
        const size_t nx = ceil_div(k / 4, (size_t)z.s * kWave);
        z.xr = nx <= (size_t)xr_small(z.s) ? xr_small(z.s) : nx <= (size_t)xr_large(z.s) ? xr_large(z.s) : 0;
        if (z.xr != 0 && lds_q8(z.s, z.tpw, m, kp, G, true) <= kMaxLds) return z;
    }
    // Below 512 tiles: the waves and laps of the lap-wise form above, so the
    // two-kernel path adds the wave sums in the same order as the fused row
    // (identical results; also faster at 4096 -> 4096, 5.51 against 5.72 us).
    // Row operations that cannot take the lap-wise form keep 8 or 16 waves
    // (in the decode step's up-front form they measured 1.6 us per token
    // faster than 4 or 8).
    if (n_tiles >= 512) {
        c.s = 4;
        c.rl = 1;
    } else if (ops) {
        c.s = G > 16 ? 16 : 8;
        c.rl = 2;
    } else {
        c.s = G > 16 ? 8 : 4;
        c.rl = 2;
    }
    const size_t threads = (size_t)c.s * c.tpw * kWave;
    const size_t nx = ceil_div(fused ? k / 4 : m * kp / 16, threads);
    const size_t xs = (size_t)xr_small(c.s), xl = (size_t)xr_large(c.s);
    c.xr = nx <= xs ? (int)xs : nx <= xl ? (int)xl : 0;
    if (c.xr == 0 || lds_q8(c.s, c.tpw, m, kp, G) > kMaxLds) c.s = 0;
    return c;
}

inline size_t groups_of(const Q8MatrixDev &w) { return w.laps_per_tile(); }

template <int MR, int S, int TPW, int RL, int XR, bool FUSED, bool OPS, bool DEBUG, bool W4,
          bool LAZY = false>
void launch_q8(ActIn in, size_t m, const float *sa_rows, const Q8MatrixDev &w,
               float *out, int32_t *block_dots, hipStream_t st) {
    const size_t G = groups_of(w);
    hipLaunchKernelGGL((k_gemv_q8_0<MR, S, TPW, RL, XR, FUSED, OPS, DEBUG, W4, LAZY>),
                       dim3((unsigned)ceil_div(w.n_tiles, TPW)), dim3(S * TPW * kWave),
                       lds_q8(S, TPW, m, w.kp, G, LAZY), st, in, (int)m, (int)w.kp, sa_rows,
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
    if constexpr (FUSED && MR == 1) {
#define MRI_Q8L(S_, RL_, XR_)                                                              \
    if (c.s == S_ && c.rl == RL_ && c.xr == XR_)                                           \
        return w.w4 ? launch_q8<1, S_, 1, RL_, XR_, true, OPS, DEBUG, true, true>(         \
                          in, m, sa_rows, w, out, block_dots, st)                          \
                    : launch_q8<1, S_, 1, RL_, XR_, true, OPS, DEBUG, false, true>(        \
                          in, m, sa_rows, w, out, block_dots, st);
        if (c.lazy) {
            MRI_Q8L(4, 1, 4) MRI_Q8L(4, 1, 12)
            MRI_Q8L(4, 2, 4) MRI_Q8L(4, 2, 12)
            MRI_Q8L(8, 2, 2) MRI_Q8L(8, 2, 6)
        }
#undef MRI_Q8L
    }
    MRI_Q8(4, 1, 1, 4) MRI_Q8(4, 1, 1, 12)
    MRI_Q8(4, 1, 2, 4) MRI_Q8(4, 1, 2, 12)
    MRI_Q8(8, 1, 2, 2) MRI_Q8(8, 1, 2, 6)
    MRI_Q8(16, 1, 2, 1) MRI_Q8(16, 1, 2, 3)
#undef MRI_Q8
}

template <int MR, bool FUSED>
void dispatch_q8_dbg(bool dbg, CfgQ8 c, ActIn in, size_t m, const float *sa_rows,
                     const Q8MatrixDev &w, float *out, int32_t *block_dots, hipStream_t st) {
    if (dbg) dispatch_q8<MR, FUSED, false, true>(c, in, m, sa_rows, w, out, block_dots, st);
    else dispatch_q8<MR, FUSED, false, false>(c, in, m, sa_rows, w, out, nullptr, st);
}

// W4A32 on 4-bit lap blocks: rows in groups of up to four per launch,
// four waves per tile from 512 tiles up (one lap in flight: two took 8.51
// against 8.07 us at 4096 -> 11008, 18.4 against 17.0 at 4096 -> 32000),
// else 8 (K <= 4096) or 16.  LDS:
// the MR f32 rows (at most kMaxLds) plus S - 1 waves' partial sums of MR x
// 16 outputs (at most 3.75 KiB), so an instance may take more than 64 KiB
// and declares its maximum once per device.
template <int MR, int S>
constexpr size_t w4a32_sum_bytes() { return (size_t)(S - 1) * MR * 16 * 4; }

template <int MR, int S, int RL, int XR>
mri_status launch_w4a32_inst(const float *x, size_t m, size_t k, const Q8MatrixDev &w,
                             float *out, hipStream_t st) {
    const size_t lds = (size_t)MR * w.kp * 4 + w4a32_sum_bytes<MR, S>();
    static DeviceOnce attr;
    MRI_HIP(attr.run([](int) {
        return hipFuncSetAttribute(reinterpret_cast<const void *>(&k_gemv_w4a32<MR, S, RL, XR>),
                                   hipFuncAttributeMaxDynamicSharedMemorySize,
                                   (int)(kMaxLds + w4a32_sum_bytes<MR, S>()));
    }));
    hipLaunchKernelGGL((k_gemv_w4a32<MR, S, RL, XR>), dim3((unsigned)w.n_tiles), dim3(S * kWave),
                       lds, st, x, (int)m, (int)k, (int)w.kp, reinterpret_cast<const v4i *>(w.laps),
                       (int)w.n_out, (int)w.n_tiles, (int)groups_of(w), (int)w.n_blocks, out);
    return MRI_OK;
}

// MRI_ERR_UNSUPPORTED when the MR f32 rows exceed kMaxLds.
template <int MR>
mri_status launch_w4a32_rows(const float *x, size_t m, size_t k, const Q8MatrixDev &w,
                             float *out, hipStream_t st) {
    const size_t G = groups_of(w);
    const int s = w.n_tiles >= 512 ? 4 : G > 16 ? 16 : 8;
    const size_t n4 = (size_t)MR * w.kp / 4;
    const size_t per = ceil_div(n4, (size_t)s * kWave);  // float4s per thread
    if ((size_t)MR * w.kp * 4 <= kMaxLds) {
#define MRI_W4A32(S_, RL_, XR_) \
    if (s == S_ && per <= XR_) return launch_w4a32_inst<MR, S_, RL_, XR_>(x, m, k, w, out, st);
        MRI_W4A32(4, 1, 4) MRI_W4A32(4, 1, 16)
        MRI_W4A32(8, 2, 2) MRI_W4A32(8, 2, 8)
        MRI_W4A32(16, 2, 1) MRI_W4A32(16, 2, 4)
#undef MRI_W4A32
    }
    return set_error(MRI_ERR_UNSUPPORTED, "w4a32: K too large for the LDS staging");
}

}  // namespace

// W4A32 matmul on a device-resident Q4_0 handle (x f32 [m][k], 16-byte
// aligned rows, k % 4 == 0): four rows per launch.
mri_status launch_gemv_w4a32(const float *x, size_t m, size_t k, const Q8MatrixDev &w,
                             float *out, hipStream_t st) {
    if (w.n_tiles == 0 || m == 0) return MRI_OK;
    if (!w.w4 || k != w.k_in || k % 4 || (reinterpret_cast<uintptr_t>(x) & 15))
        return set_error(MRI_ERR_INVALID_ARGUMENT, "w4a32: unsupported input");
    for (size_t m0 = 0; m0 < m; m0 += 4) {
        const size_t mc = std::min<size_t>(4, m - m0);
        const float *xs = x + m0 * k;
        float *os = out + m0 * w.n_out;
        const mri_status r = mc == 1   ? launch_w4a32_rows<1>(xs, mc, k, w, os, st)
                             : mc == 2 ? launch_w4a32_rows<2>(xs, mc, k, w, os, st)
                                       : launch_w4a32_rows<4>(xs, mc, k, w, os, st);
        if (r) return r;
        MRI_LAUNCHED("k_gemv_w4a32");
    }
    return MRI_OK;
}

bool gemv_q8_supported(bool fused, size_t m, size_t n_tiles, size_t k, size_t kp) {
    const size_t G = kp / kQ8LapK;
    return m >= 1 && m <= (size_t)kMaxM && pick_q8(fused, n_tiles, m, k, kp, G).s > 0;
}

mri_status launch_gemv_q8_0(const float *x, const int8_t *act, size_t m,
                            const float *sa_rows, const Q8MatrixDev &w, float *out,
                            int32_t *block_dots, float *scales_out, hipStream_t st,
                            const RowOps &ops) {
    if (w.n_tiles == 0 || m == 0) return MRI_OK;
    const CfgQ8 c =
        pick_q8(x != nullptr, w.n_tiles, m, w.k_in, w.kp, groups_of(w), ops.any(), w.w4);
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
