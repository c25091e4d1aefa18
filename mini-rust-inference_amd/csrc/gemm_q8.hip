// gemm_q8.hip — prefill-sized matmul_q8_0_direct (q8_direct.rs:229-289):
// Q8_0 weights (32-element blocks, one f16 scale each) times activation
// rows quantized per row to int8, on LDS-staged CDNA4 MFMA tiles.
//
//   dot[m, n, b] = sum_{k in block b} act_q[m, k] * w_q[n, k]     (exact int32)
//   out[m, n]    = s_a[m] * sum_b (f32)dot[m, n, b] * d[n, b]       (f32)
//
// The per-block f32 fold is the work that bounds this product: one term
// per (row, channel, block), against one MFMA per 16 x 16 x 32 block.  The
// reference rounds ((f32)dot * s_a) * d per block and adds in block order
// (two multiplies and an add); here each term is one fused multiply-add
// onto the running sum (the dot's f32 value and an FMA) and s_a multiplies
// once at the end.  The int32 block dots are exact; the f32 result differs from the
// reference's only by those roundings, within 1e-5 * max(|out|, sum |t_b|)
// of it.  Half the VALU work of the reference's order is what makes this
// kernel twice as fast as keeping that order would be.
//
// Operands.  Both are used in the layouts the decode kernels read:
//   * activations: rows [M][kp] (kp = K padded to 256) with each 64-byte
//     chunk permuted so that lane group g's 16 bytes are [block 2p, k 8g..+8 |
//     block 2p+1, k 8g..+8], i.e. the 8-byte A operands of
//     v_mfma_i32_16x16x32_i8 for both blocks of the chunk;
//   * weights: lap blocks of 16 channels x 256 k (4 chunks of 1 KiB in the
//     same permutation, then 16 rows x 8 f16 scales), tile-major.
// A workgroup computes BM rows x BN channels (128 x 64: 4 x 2 sub-tiles of
// 32 x 32); each ring stage is half a lap (4 blocks): per stage it stages
// BM x 128 bytes of activation fragments, BN x 128 bytes of weight chunks
// and the lap's scales in LDS by global_load_lds (16 bytes per lane, each
// lane its own address, so a fragment of 16 rows x 64 bytes is gathered
// straight from the row-major activations), NS stages deep: the loads of
// the next stages fly while one is folded.  Each of the 8 waves (4 x 2) owns
// 32 rows x 32 channels; two workgroups share a CU, four waves per SIMD, and
// the MFMA results, sums and operands all stay in VGPRs.
//
// Per block, v_mfma_i32_32x32x32_i8 gives the exact dots of 32 rows x 32
// channels; its output register e of lane l holds row 8 * (e / 4) +
// 4 * (l / 32) + e % 4 and channel l % 32.
#include <hip/hip_runtime.h>

#include <type_traits>
#include <utility>

#include "gemv_common.hpp"

namespace mri {
using namespace gemv;
namespace {

typedef int v16i __attribute__((ext_vector_type(16)));

constexpr int kQWave = 64;
constexpr int kQWaitVm0 = 0x0F70;  // s_waitcnt vmcnt(0), others untouched
constexpr int kQXcds = 8;
template <typename F, int... I>
__device__ inline void q_static_for_impl(F &&f, std::integer_sequence<int, I...>) {
    (f(std::integral_constant<int, I>{}), ...);
}
template <int N, typename F>
__device__ inline void q_static_for(F &&f) {
    q_static_for_impl(f, std::make_integer_sequence<int, N>{});
}

#pragma clang diagnostic ignored "-Winline-asm"
// 16 bytes per lane from g into LDS at byte address lds + 16 * lane (the
// loads write M0 themselves; s_nop 0 covers the M0 -> LDS DMA hazard).
__device__ inline void q_dma16(const void *g, unsigned lds) {
    asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off"
                 :
                 : "v"(g), "s"(lds)
                 : "memory", "m0");
}
__device__ inline void q_dma16_nt(const void *g, unsigned lds) {
    asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off nt"
                 :
                 : "v"(g), "s"(lds)
                 : "memory", "m0");
}

// 4 bytes per lane from g into LDS at byte address lds + 4 * lane.
__device__ inline void q_dma4_nt(const void *g, unsigned lds) {
    asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dword %0, off nt"
                 :
                 : "v"(g), "s"(lds)
                 : "memory", "m0");
}

// s_waitcnt lgkmcnt(0) that the compiler sees reading and writing every
// operand quad read by inline ds_read2_b64, so that none of their uses is
// scheduled before it.
template <int RG, int TT>
__device__ inline void q8_wait_lds(v4i (&a)[2][RG][2], v4i (&b)[2][TT][2]) {
    if constexpr (RG == 2 && TT == 1) {
        asm volatile("s_waitcnt lgkmcnt(0)"
                     : "+v"(a[0][0][0]), "+v"(a[0][0][1]), "+v"(a[0][1][0]), "+v"(a[0][1][1]),
                       "+v"(a[1][0][0]), "+v"(a[1][0][1]), "+v"(a[1][1][0]), "+v"(a[1][1][1]),
                       "+v"(b[0][0][0]), "+v"(b[0][0][1]), "+v"(b[1][0][0]), "+v"(b[1][0][1]));
    } else if constexpr (RG == 1 && TT == 1) {
        asm volatile("s_waitcnt lgkmcnt(0)"
                     : "+v"(a[0][0][0]), "+v"(a[0][0][1]), "+v"(a[1][0][0]), "+v"(a[1][0][1]),
                       "+v"(b[0][0][0]), "+v"(b[0][0][1]), "+v"(b[1][0][0]), "+v"(b[1][0][1]));
    } else if constexpr (RG == 1 && TT == 2) {
        asm volatile("s_waitcnt lgkmcnt(0)"
                     : "+v"(a[0][0][0]), "+v"(a[0][0][1]), "+v"(a[1][0][0]), "+v"(a[1][0][1]),
                       "+v"(b[0][0][0]), "+v"(b[0][0][1]), "+v"(b[0][1][0]), "+v"(b[0][1][1]),
                       "+v"(b[1][0][0]), "+v"(b[1][0][1]), "+v"(b[1][1][0]), "+v"(b[1][1][1]));
    } else {
        static_assert(RG == 2 && TT == 2, "wave tile");
        asm volatile("s_waitcnt lgkmcnt(0)"
                     : "+v"(a[0][0][0]), "+v"(a[0][0][1]), "+v"(a[0][1][0]), "+v"(a[0][1][1]),
                       "+v"(a[1][0][0]), "+v"(a[1][0][1]), "+v"(a[1][1][0]), "+v"(a[1][1][1]),
                       "+v"(b[0][0][0]), "+v"(b[0][0][1]), "+v"(b[0][1][0]), "+v"(b[0][1][1]),
                       "+v"(b[1][0][0]), "+v"(b[1][0][1]), "+v"(b[1][1][0]), "+v"(b[1][1][1]));
    }
}

// Scale fragments of a stage: one per 16-channel weight tile, at least one
// per wave (every wave issues the same loads; waves past the tile count
// reload the last tile's scales into a slot nothing reads).
template <int BN, int NW>
constexpr int q8_scale_slots() {
    return BN / 16 > NW ? BN / 16 : NW;
}

// Weight fragments (1 KiB each) of a stage: Q8_0, one per 16-channel tile
// and chunk; W4, one quant piece (the half lap's two chunks) per tile, at
// least one per wave (waves past the tile count reload the last tile's
// piece into a slot nothing reads).
template <int BN, int NW, bool W4>
constexpr int q8_b_slots() {
    return W4 ? (BN / 16 > NW ? BN / 16 : NW) : BN / 8;
}

// The same wait for the W4 instance (RG = TT = 1): the activation quads and
// the weight quant pieces.
__device__ inline void q8_wait_lds_w4(v4i (&a)[2][1][2], v4i (&bw)[1][2]) {
    asm volatile("s_waitcnt lgkmcnt(0)"
                 : "+v"(a[0][0][0]), "+v"(a[0][0][1]), "+v"(a[1][0][0]), "+v"(a[1][0][1]),
                   "+v"(bw[0][0]), "+v"(bw[0][1]));
}

// Bytes of one ring stage (half a lap: 2 chunks, 4 blocks) of a BM x BN tile:
// activation fragments, weight chunks, and the lap's weight scales.
template <int BM, int BN, int NW, bool W4>
constexpr int q8_stage_bytes() {
    return BM * 128 + q8_b_slots<BN, NW, W4>() * 1024 + q8_scale_slots<BN, NW>() * 256;
}

template <int BM, int BN, int WM, int WN, int NS, bool W4>
__global__ __launch_bounds__(WM * WN * kQWave) void k_gemm_q8_0(
    const int8_t *__restrict__ act, int M, int kp, const float *__restrict__ sa_rows,
    const int8_t *__restrict__ laps, int N, int n_tiles, int G, int n_mt, int n_total, int ks,
    float *__restrict__ out, float *__restrict__ part, int *__restrict__ cnt) {
    constexpr int NW = WM * WN;
    constexpr int RG = BM / 32 / WM, TT = BN / 32 / WN;  // 32 x 32 sub-tiles per wave
    constexpr int FA = BM / 8, FB = q8_b_slots<BN, NW, W4>(), FS = q8_scale_slots<BN, NW>();
    constexpr int LA = FA / NW, LB = FB / NW, LS = FS / NW;  // ... per wave
    static_assert(RG >= 1 && TT >= 1 && FA % NW == 0 && FB % NW == 0 && FS % NW == 0,
                  "wave split");
    static_assert(NS >= 2, "ring depth");
    constexpr int L = LA + LB + LS;  // loads per wave and stage, the same for every wave
    constexpr int SA = BM * 128, SB = FB * 1024;
    constexpr int STAGE = q8_stage_bytes<BM, BN, NW, W4>();
    extern __shared__ v4i s_buf[];

    // XCD-aware tile index: workgroups go to the 8 XCDs round-robin; the M
    // tiles of one weight column block run on one XCD and share its L2.
    // With a K split the ks parts of a tile are adjacent items, each a
    // contiguous range [s0, s1) of the K steps.
    const int per_xcd = (int)(gridDim.x / kQXcds);
    const int item = (int)(blockIdx.x % kQXcds) * per_xcd + (int)(blockIdx.x / kQXcds);
    if (item >= n_total * ks) return;
    const int tile = item / ks, kpart = item - tile * ks;
    const int mt = tile % n_mt, nt = tile / n_mt;

    const int t = threadIdx.x;
    const int wv = __builtin_amdgcn_readfirstlane(t >> 6), l = t & 63;
    const int wm = wv / WN, wn = wv % WN;
    const unsigned lds0 = __builtin_amdgcn_readfirstlane((unsigned)(size_t)s_buf);
    const int S = 2 * G;  // ring steps: half laps
    const int s0 = split_lo(S, ks, kpart), s1 = split_lo(S, ks, kpart + 1);

    // This wave's loads of a stage.  Fragment f = wv + NW * j of the A
    // region: 16-row group f / 2, chunk f % 2 of the half lap; rows past M
    // read row M - 1 (their outputs are not stored).  Fragment f of the B
    // region: weight tile f / 2, chunk f % 2; tiles past the end read the
    // last.  Scales: tile wv + NW * j (waves past the tile count: the last
    // tile, into a slot nothing reads), 4 bytes per lane (its 256 bytes).
    // Step s adds 128 s bytes to an activation source, and lap s / 2 (plus
    // 2 KiB for the second half) to a weight source.
    const int8_t *a_src[LA];
    const int8_t *b_src[LB];
    const int8_t *s_src[LS];
    const size_t lap_bytes = W4 ? kQ4LapBytes : kQ8LapBytes;
    constexpr int kScaleOff = W4 ? 2048 : 4096;  // the lap's scales in its block
#pragma unroll
    for (int j = 0; j < LA; ++j) {
        const int f = wv + NW * j;
        const int row = min(BM * mt + 16 * (f >> 1) + (l & 15), M - 1);
        a_src[j] = act + (size_t)row * kp + 64 * (f & 1) + 16 * (l >> 4);
    }
#pragma unroll
    for (int j = 0; j < LB; ++j) {
        const int f = wv + NW * j;
        if constexpr (W4) {  // the tile's quant piece of the half lap
            const int T = min(BN / 16 * nt + min(f, BN / 16 - 1), n_tiles - 1);
            b_src[j] = laps + (size_t)T * G * lap_bytes + 16 * l;
        } else {
            const int T = min(BN / 16 * nt + (f >> 1), n_tiles - 1);
            b_src[j] = laps + (size_t)T * G * lap_bytes + 1024 * (f & 1) + 16 * l;
        }
    }
#pragma unroll
    for (int j = 0; j < LS; ++j) {
        const int T = min(BN / 16 * nt + min(wv + NW * j, BN / 16 - 1), n_tiles - 1);
        s_src[j] = laps + (size_t)T * G * lap_bytes + kScaleOff + 4 * l;
    }
    // loads of step s (clamped to the last: the loads past the end re-read
    // it into a stage no later step reads, so every wait count is constant)
    auto issue = [&](int s) __attribute__((always_inline)) {
        const int sc = min(s, s1 - 1);
        const unsigned base = lds0 + (unsigned)((s % NS) * STAGE);
        const size_t ao = (size_t)sc * 128;
        const size_t bo = (size_t)(sc >> 1) * lap_bytes + (size_t)(sc & 1) * (W4 ? 1024 : 2048);
        const size_t so = (size_t)(sc >> 1) * lap_bytes;
#pragma unroll
        for (int j = 0; j < LA; ++j) q_dma16(a_src[j] + ao, base + (wv + NW * j) * 1024);
#pragma unroll
        for (int j = 0; j < LB; ++j) q_dma16_nt(b_src[j] + bo, base + SA + (wv + NW * j) * 1024);
#pragma unroll
        for (int j = 0; j < LS; ++j)
            q_dma4_nt(s_src[j] + so, base + SA + SB + (wv + NW * j) * 256);
    };

    // v_mfma_i32_32x32x32_i8 operands: lane l holds row (or channel) l % 32
    // and 16 k-bytes, k-half u = l / 32 of the block.  A staged fragment
    // holds 16 rows x 64 bytes with lane' = 16 g + r owning row r and bytes
    // [block 2c, k 8g..+8 | block 2c+1, k 8g..+8], so lane l gathers lane's
    // 32u + l % 16 and 32u + 16 + l % 16 of its 16-row group: the low 8
    // bytes of both are its operand for block 2c, the high 8 for block
    // 2c + 1.  A and B are gathered alike, so the int32 dots are the same
    // sums over the same k.
    const int r16 = l & 15, half = (l >> 4) & 1, u = l >> 5;
    float fs[RG][TT][16];
#pragma unroll
    for (int i = 0; i < RG; ++i)
#pragma unroll
        for (int j = 0; j < TT; ++j)
#pragma unroll
            for (int e = 0; e < 16; ++e) fs[i][j][e] = 0.0f;
    // Each block's MFMAs start from the bits of 1.5 * 2^23 rather than from
    // zero, so that an output register, read as f32, is 12582912 + dot
    // exactly (|dot| <= 32 * 128 * 127 < 2^22 keeps it in [2^23, 2^24),
    // where the f32 spacing is 1): one full-rate subtract then gives
    // (f32)dot, where v_cvt_f32_i32 issues at half rate.
    v16i bias;
#pragma unroll
    for (int e = 0; e < 16; ++e) bias[e] = kDotBias;

#pragma unroll
    for (int s = s0; s < s0 + NS - 1; ++s) issue(s);
    // Step s: wait for its loads and for every wave to be done with step
    // s - 1, whose stage the loads of step s + NS - 1 refill; then its 4
    // blocks, software-pipelined: the MFMAs of block k + 1 (into registers
    // of their own) are issued before the fold of block k, so the MFMA pipe
    // and the VALU work side by side.
    for (int s = s0; s < s1; ++s) {
        asm volatile("s_waitcnt vmcnt(%0)\n\ts_barrier" : : "n"((NS - 2) * L) : "memory");
        issue(s + NS - 1);
        const v4i *ss_ = s_buf + ((size_t)(s % NS) * STAGE + SA + SB) / 16;
        const int hh = s & 1;  // which half of the lap: its blocks 4 hh .. 4 hh + 3
        v4i sc[TT];  // the lap's 8 f16 scales of this lane's channel in sub-tile j
#pragma unroll
        for (int j = 0; j < TT; ++j) sc[j] = ss_[(2 * (wn * TT + j) + half) * 16 + r16];
        // Operands of chunk c: [sub-tile][block h of the chunk], each one
        // ds_read2_b64 of lane' (offset h) and lane' + 16 (offset 32 + h, in
        // 8-byte units) straight into a register quad.  The reads are issued
        // here for the whole half lap and waited for once, by an s_waitcnt
        // that takes every operand as its own in-out operand, so that no use
        // can be scheduled before it.
        v4i a[2][RG][2], b[2][TT][2];
        v4i bw[TT][2];  // W4: the quant pieces of lane' and lane' + 16
        const unsigned st = lds0 + (unsigned)((s % NS) * STAGE) + (unsigned)(16 * (32 * u + r16));
#pragma unroll
        for (int c = 0; c < 2; ++c) {
#pragma unroll
            for (int i = 0; i < RG; ++i) {
                const unsigned ad = st + (unsigned)(((2 * (wm * RG + i) + half) * 2 + c) * 1024);
                asm volatile("ds_read2_b64 %0, %1 offset1:32" : "=v"(a[c][i][0]) : "v"(ad));
                asm volatile("ds_read2_b64 %0, %1 offset0:1 offset1:33" : "=v"(a[c][i][1]) : "v"(ad));
            }
#pragma unroll
            for (int j = 0; j < TT; ++j) {
                if constexpr (W4) {
                    // one 16-byte piece per lane' holds the half lap's 4
                    // block words: read it once, at c = 0
                    if (c == 0) {
                        const unsigned ad = st + (unsigned)(SA + (2 * (wn * TT + j) + half) * 1024);
                        asm volatile("ds_read_b128 %0, %1" : "=v"(bw[j][0]) : "v"(ad));
                        asm volatile("ds_read_b128 %0, %1 offset:256" : "=v"(bw[j][1]) : "v"(ad));
                    }
                } else {
                    const unsigned ad =
                        st + (unsigned)(SA + ((2 * (wn * TT + j) + half) * 2 + c) * 1024);
                    asm volatile("ds_read2_b64 %0, %1 offset1:32" : "=v"(b[c][j][0]) : "v"(ad));
                    asm volatile("ds_read2_b64 %0, %1 offset0:1 offset1:33"
                                 : "=v"(b[c][j][1])
                                 : "v"(ad));
                }
            }
        }
        static_assert(RG * 4 + TT * 4 <= 24, "operands of the wait");
        if constexpr (W4) {
            static_assert(RG == 1 && TT == 1, "W4 wave tile");
            q8_wait_lds_w4(a, bw);
        } else {
            q8_wait_lds(a, b);
        }
        v16i d[2][RG][TT];  // block dots of block k in set k % 2
        auto dots = [&](auto kk) __attribute__((always_inline)) {
            constexpr int k = decltype(kk)::value, c = k / 2, h = k % 2;
#pragma unroll
            for (int i = 0; i < RG; ++i)
#pragma unroll
                for (int j = 0; j < TT; ++j) {
                    v4i bv;
                    if constexpr (W4) {
                        // word 2c + h of each piece: block h of chunk c, 8
                        // elements as nibbles; each moved to the high half of
                        // its byte reads as 16 * quant (k order as in Q8_0)
                        constexpr int kHi = (int)0xF0F0F0F0u;
                        const int w0 = bw[j][0][2 * c + h], w1 = bw[j][1][2 * c + h];
                        bv = v4i{(w0 << 4) & kHi, w0 & kHi, (w1 << 4) & kHi, w1 & kHi};
                    } else {
                        bv = b[c][j][h];
                    }
                    d[k % 2][i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a[c][i][h], bv, bias,
                                                                         0, 0, 0);
                }
        };
        auto fold = [&](auto kk) __attribute__((always_inline)) {
            constexpr int k = decltype(kk)::value, c = k / 2, h = k % 2;
#pragma unroll
            for (int j = 0; j < TT; ++j) {
                // block 4 hh + k of the lap: f16 number 4 hh + k of the row's 8
                const unsigned word = (unsigned)(hh ? sc[j][2 + c] : sc[j][c]);
                // converted once here (v_cvt_f32_f16), so that each term is a
                // full-rate v_fma_f32 rather than a mixed-precision FMA
                float ds;
                asm("v_cvt_f32_f16_e32 %0, %1" : "=v"(ds) : "v"(h ? (word >> 16) : word));
                // W4: the dots are 16 * dot (exact, < 2^22), so the scale
                // takes the 1/16 (exact: a power of two on a normal f32), and
                // fma(16 dot, d / 16, s) == fma(dot, d, s) bit for bit
                if constexpr (W4) ds = ds * 0.0625f;
#pragma unroll
                for (int i = 0; i < RG; ++i)
#pragma unroll
                    for (int e = 0; e < 16; ++e) {
                        const int biased = d[k % 2][i][j][e];
                        fs[i][j][e] = __builtin_fmaf(__int_as_float(biased) - kDotBiasF, ds,
                                                     fs[i][j][e]);
                    }
            }
        };
        dots(std::integral_constant<int, 0>{});
        q_static_for<4>([&](auto kk) {
            constexpr int k = decltype(kk)::value;
            if constexpr (k + 1 < 4) dots(std::integral_constant<int, k + 1>{});
            fold(kk);
        });
    }
    // the clamped loads past the end may still be writing LDS
    asm volatile("s_waitcnt vmcnt(0)" : : : "memory");

    if (ks > 1) {
        // K split: every part but the last to arrive leaves its partial sums
        // in its slot (register e of sub-tile (i, j) of wave wv at word
        // ((wv * RG * TT + i * TT + j) * 16 + e) * 64 + l) and counts itself
        // on the tile's counter; the last adds the parts in part order, so
        // the result does not depend on the order of arrival.  The slots are
        // written with device-scope (sc1) stores, complete at vmcnt(0)
        // before the barrier and the count, and read with device-scope
        // loads, which do not hit lines this XCD's L2 cached before.
        __shared__ int s_last;
        const size_t wbase = (size_t)wv * RG * TT * 16 * 64 + l;
        float *mine = part + ((size_t)tile * ks + kpart) * (BM * BN) + wbase;
#pragma unroll
        for (int i = 0; i < RG; ++i)
#pragma unroll
            for (int j = 0; j < TT; ++j)
#pragma unroll
                for (int e = 0; e < 16; ++e)
                    __hip_atomic_store(mine + ((i * TT + j) * 16 + e) * 64, fs[i][j][e],
                                       __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __builtin_amdgcn_s_waitcnt(kQWaitVm0);
        __syncthreads();
        if (t == 0)
            s_last = __hip_atomic_fetch_add(&cnt[tile], 1, __ATOMIC_RELAXED,
                                            __HIP_MEMORY_SCOPE_AGENT) == ks - 1;
        __syncthreads();
        if (!s_last) return;
        float tot[RG][TT][16];
        for (int p = 0; p < ks; ++p) {
            const float *src = part + ((size_t)tile * ks + p) * (BM * BN) + wbase;
#pragma unroll
            for (int i = 0; i < RG; ++i)
#pragma unroll
                for (int j = 0; j < TT; ++j)
#pragma unroll
                    for (int e = 0; e < 16; ++e) {
                        const float v = p == kpart ? fs[i][j][e]
                                                   : __hip_atomic_load(
                                                         src + ((i * TT + j) * 16 + e) * 64,
                                                         __ATOMIC_RELAXED,
                                                         __HIP_MEMORY_SCOPE_AGENT);
                        tot[i][j][e] = p == 0 ? v : tot[i][j][e] + v;
                    }
        }
#pragma unroll
        for (int i = 0; i < RG; ++i)
#pragma unroll
            for (int j = 0; j < TT; ++j)
#pragma unroll
                for (int e = 0; e < 16; ++e) fs[i][j][e] = tot[i][j][e];
        if (t == 0)  // ready for the next call on this stream
            __hip_atomic_store(&cnt[tile], 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }

    // register e of sub-tile (i, j): row 32 i + 8 (e / 4) + 4 u + e % 4 of the
    // wave's rows, channel 32 j + l % 32 of its channels
#pragma unroll
    for (int i = 0; i < RG; ++i) {
        const int m0 = BM * mt + 32 * (wm * RG + i) + 4 * u;
        float sa[16];
#pragma unroll
        for (int e = 0; e < 16; ++e) sa[e] = sa_rows[min(m0 + 8 * (e >> 2) + (e & 3), M - 1)];
#pragma unroll
        for (int j = 0; j < TT; ++j) {
            const int n = BN * nt + 32 * (wn * TT + j) + (l & 31);
            if (n >= N) continue;
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                const int m = m0 + 8 * (e >> 2) + (e & 3);
                if (m < M) out[(size_t)m * N + n] = fs[i][j][e] * sa[e];
            }
        }
    }
}

constexpr int kQ8BM = 128, kQ8BN = 64;  // the tile of the launched instance

// Tiles of the launched instance for m rows, and its K split: 2-way when
// the tiles fill at most one of the two workgroup slots of every CU, each
// part keeping at least 8 half-lap steps.  (The GEMM's range, m * n > 2^20,
// always has more than 128 tiles of 128 x 64, so a 4-way split would leave
// CUs idle no less.)
size_t q8_tiles(size_t m, const Q8MatrixDev &w) {
    return ((m + kQ8BM - 1) / kQ8BM) * ((w.n_tiles + kQ8BN / 16 - 1) / (kQ8BN / 16));
}
int q8_ks(size_t m, const Q8MatrixDev &w) {
    const size_t cus = (size_t)std::max(device_cus(), 0), tiles = q8_tiles(m, w);
    const size_t S = 2 * w.laps_per_tile();
    int ks = 1;
    if (cus > 0 && tiles <= cus && S >= 16) ks = 2;
    if (tiles * (size_t)ks > (size_t)kGemmWsCounters) ks = 1;
    return ks;
}

template <int BM, int BN, int WM, int WN, int NS, bool W4>
mri_status launch_q8_inst(const int8_t *act, size_t m, const float *sa_rows,
                          const Q8MatrixDev &w, float *out, void *ws, hipStream_t s) {
    constexpr size_t lds = (size_t)NS * q8_stage_bytes<BM, BN, WM * WN, W4>();
    static DeviceOnce attr;
    MRI_HIP(attr.run([&](int) {
        return hipFuncSetAttribute(
            reinterpret_cast<const void *>(&k_gemm_q8_0<BM, BN, WM, WN, NS, W4>),
            hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    }));
    const size_t n_mt = (m + BM - 1) / BM;
    const size_t n_nt = (w.n_tiles + BN / 16 - 1) / (BN / 16);
    const size_t total = n_mt * n_nt;
    const int ks = ws ? q8_ks(m, w) : 1;
    int *cnt = static_cast<int *>(ws);
    float *part = ws ? reinterpret_cast<float *>(cnt + kGemmWsCounters) : nullptr;
    const size_t grid = (total * ks + kQXcds - 1) / kQXcds * kQXcds;
    hipLaunchKernelGGL((k_gemm_q8_0<BM, BN, WM, WN, NS, W4>), dim3((unsigned)grid),
                       dim3(WM * WN * kQWave), lds, s, act, (int)m, (int)w.kp, sa_rows, w.laps,
                       (int)w.n_out, (int)w.n_tiles, (int)w.laps_per_tile(), (int)n_mt,
                       (int)total, ks, out, part, cnt);
    MRI_LAUNCHED("k_gemm_q8_0");
    return MRI_OK;
}

}  // namespace

// Where this kernel is used instead of the skinny kernel (which keeps the
// reference's per-block rounding bit for bit): from 128 rows once the
// product has more than 2^20 outputs.  The skinny kernel's waves then no
// longer fit one pass of the SIMDs, while this kernel's time has a floor of
// its K loop's latency (about 39 us at K = 4096).  Measured at K = 4096
// (us, skinny / this kernel): 64 x 4096 31.0 / 38.7, 128 x 4096 33.0 /
// 39.5, 256 x 4096 35.6 / 41.0, 512 x 2048 36.7 / 42.5 (all 2^20 outputs or
// fewer); 128 x 11008 58.5 / 42.2, 256 x 11008 57.5 / 57.7, 512 x 4096
// 61.5 / 45.0, 512 x 12288 155 / 101.7, 512 x 22016 258 / 171; at
// K = 11008, 512 x 4096 148.7 / 108 and 256 x 4096 80 / 112.
bool gemm_q8_supported(size_t m, const Q8MatrixDev &w) {
    return m >= 128 && m * w.n_out > (1ull << 20) && m * w.kp < (1ull << 31) &&
           m * w.n_out < (1ull << 31);
}

// act: quantized rows [m][w.kp], chunk-permuted (launch_quantize_rows with
// the Q8_0 layout); sa_rows: their scales.
// Tiles of 128 rows x 64 channels, 8 waves of 32 x 32, two LDS stages
// (about 52 KiB; the 126 VGPRs hold two workgroups per CU, four waves per
// SIMD, either way).  Three stages took 1-2 % longer (M = 512, K = 4096:
// N = 12288 86.5 against 88.2 us, N = 32000 204.5 against 208.1, N = 4096
// 39.5 against 40.1; K = 11008 79.9 against 81.6; bit-identical).  With
// the MFMA results in
// VGPRs (see the build flags) 128 x 64 tiles beat 128 x 128 tiles of 8
// waves at every N measured (M = 512, K = 4096: 164.5 against 176.4 us at
// N = 22016, 223.5 against 234 at N = 32000); 8 waves of 32 x 32 rather
// than 4 of 64 x 32 halve each wave's serial fold per step and took the
// latency floor from 43 to 39 us (512 x 11008 -> 4096: 108 against 117).
mri_status launch_gemm_q8_0(const int8_t *act, size_t m, const float *sa_rows,
                            const Q8MatrixDev &w, float *out, void *ws, hipStream_t s) {
    if (w.w4) return launch_q8_inst<kQ8BM, kQ8BN, 4, 2, 2, true>(act, m, sa_rows, w, out, ws, s);
    return launch_q8_inst<kQ8BM, kQ8BN, 4, 2, 2, false>(act, m, sa_rows, w, out, ws, s);
}

// [tile counters (kGemmWsCounters ints, shared with the INT8 GEMM's)]
// [f32 partial tiles: ks slots per tile]; 0 without a K split.
size_t gemm_q8_ws_bytes(size_t m, const Q8MatrixDev &w) {
    const int ks = q8_ks(m, w);
    if (ks == 1) return 0;
    return (size_t)kGemmWsCounters * sizeof(int) +
           q8_tiles(m, w) * (size_t)ks * kQ8BM * kQ8BN * sizeof(float);
}

}  // namespace mri
