// gemm.hip — prefill-sized per-channel INT8 matmul (matmul_int8,
// int8.rs:61-98, and its parallel form parallel.rs:308-346) as a dense
// contraction on CDNA4 int8 MFMA.
//
//   acc[m, n] = sum_k act_q[m, k] * w[n, k]            (exact int32)
//   out[m, n] = ((f32)acc[m, n] * s_a[m]) * s_w[n]      (int8.rs:93)
//
// Tiling: a workgroup of WM x WN waves computes a BM x BN output tile; wave
// (wm, wn) owns a (BM/WM) x (BN/WN) block of 32 x 32 MFMA tiles and runs
// two v_mfma_i32_32x32x32_i8 per tile per K step of 64 (one per k half).
// The 32x32x32 form keeps the int8 pipe full with a few accumulators per
// wave, where 16x16x64 needs many.  Both operands are staged through LDS
// in the MFMA fragment layout: a 32-row x 32-k fragment is 1 KiB with lane
// l's 16 bytes at l * 16 (row l % 32, k 16*(l/32)..+16), so every LDS read
// is one contiguous, conflict-free ds_read_b128 per wave.
//
// Loads: gfx950's global_load_lds_dwordx4 moves 16 bytes per lane from
// global memory straight into LDS at M0 + 16 * lane, i.e. one 1 KiB
// fragment per wave instruction, without passing through registers; each
// lane supplies its own source address.  An activation lane points at its
// row.  A weight fragment (32 rows) gathers its 16-byte pieces from the two
// stored 16-row chunks of the slab, which are adjacent in the slab-major
// layout, so a workgroup's weight loads of one K slab stay within one
// contiguous block.  An NS-stage LDS ring keeps NS - 1 K steps in flight.
//
// Ordering: the loads are issued from inline assembly, outside the
// compiler's wait-count tracking, and every step waits explicitly: the
// wave's own loads of the step (s_waitcnt vmcnt(N)), then one s_barrier,
// after which all waves' loads of the step are in LDS and all reads of the
// previous step are done, so its buffer can be refilled.
//
// Workgroup -> tile mapping is XCD-aware: workgroups are dispatched to the
// eight XCDs round-robin, and the M tiles that share a weight column block
// are placed on the same XCD, so they share its L2.
#include <hip/hip_runtime.h>

#include "common.hpp"

namespace mri {
namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));
constexpr int kWave = 64;
constexpr int kXcds = 8;
#ifndef DMA_B
#define DMA_B dma16_nt
#endif

// The loads below write M0 themselves; no code of this file keeps a value
// in M0 across them (gfx9 LDS instructions do not use it), so clobbering
// the reserved register is safe here.  s_nop 0 covers the M0 -> LDS DMA
// hazard, which the compiler cannot see inside the assembly.
#pragma clang diagnostic ignored "-Winline-asm"

// 16 bytes per lane from g into LDS at byte address lds + 16 * lane.
__device__ inline void dma16(const void *g, unsigned lds) {
    asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off"
                 :
                 : "v"(g), "s"(lds)
                 : "memory", "m0");
}
// The same with the streaming (non-temporal) hint: for data read once, so
// that it does not evict the operand that every workgroup re-reads from L2.
__device__ inline void dma16_nt(const void *g, unsigned lds) {
    asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off nt"
                 :
                 : "v"(g), "s"(lds)
                 : "memory", "m0");
}

// Wait until at most N of this wave's loads are outstanding, then barrier.
template <int N>
__device__ inline void wait_barrier() {
    asm volatile("s_waitcnt vmcnt(%0)\n\ts_barrier" : : "n"(N) : "memory");
}

template <int BM, int BN, int WM, int WN, int NSA, int NSB>
__global__ __launch_bounds__(WM * WN * kWave) void k_gemm_int8(
    const int8_t *__restrict__ act, int mg, const float *__restrict__ sa_ptr, int sa_stride,
    float sa_value, const int8_t *__restrict__ tiles, const float *__restrict__ wscales,
    int M, int N, int n_tiles, int P, int n_mt, int n_tiles_total, float *__restrict__ out,
    int32_t *__restrict__ acc_out) {
    constexpr int NW = WM * WN;                // waves
    constexpr int FA = BM / 32 * 2, FB = BN / 32 * 2;  // fragments per K step (2 k halves)
    constexpr int TM = BM / WM / 32, TN = BN / WN / 32;  // MFMA tiles per wave
    constexpr int LA = FA / NW, LB = FB / NW;  // fragment loads per wave per step
    static_assert(FA % NW == 0 && FB % NW == 0, "load split");
    constexpr int SA = FA * 1024, SB = FB * 1024;  // bytes of one A / B stage
    static_assert(NSA >= 3 && NSB >= 3, "ring depths");
    // Issue order per step q: A(q + NSA - 1), then B(q + NSB - 1).  Step p
    // of the loop needs the data of step p + 1 (its fragments are read into
    // registers while step p's MFMAs run); the younger of A(p+1), B(p+1) is
    // A(p+1) when NSB > NSA, else B(p+1).  The loads younger than it are,
    // respectively, B of its step plus NSA - 3 whole later steps, or NSB - 3
    // whole later steps.  WAIT0 is the same count for step 0 before the loop.
    constexpr int WAIT = NSB > NSA ? LB + (NSA - 3) * (LA + LB) : (NSB - 3) * (LA + LB);
    constexpr int WAIT0 = WAIT + LA + LB;
    constexpr int NMX = NSA > NSB ? NSA : NSB;
    extern __shared__ v4i s_buf[];

    // XCD-aware tile index: this workgroup runs on XCD blockIdx % 8.
    const int per_xcd = (int)(gridDim.x / kXcds);
    const int tile = (int)(blockIdx.x % kXcds) * per_xcd + (int)(blockIdx.x / kXcds);
    if (tile >= n_tiles_total) return;
    const int mt = tile % n_mt, nt = tile / n_mt;
    const int m0 = mt * BM, T0 = nt * (BN / 16);  // first row, first 16-row weight tile

    const int t = threadIdx.x;
    const int wv = __builtin_amdgcn_readfirstlane(t >> 6), l = t & 63;
    const int wm = wv / WN, wn = wv % WN;
    const unsigned ldsA = __builtin_amdgcn_readfirstlane((unsigned)(size_t)s_buf);
    const unsigned ldsB = ldsA + NSA * SA;

    // This wave's loads.  Fragment f = wv + NW*j holds row group f/2, k half
    // f%2.  Activations are packed (see pack layout): fragment (p, g, h) is
    // 1 KiB at ((p * mg + g) * 2 + h) KiB, so the workgroup's BM/32 row
    // groups of one K step are contiguous.  Weight lane: row 32*(f/2) + l%32
    // of the block, i.e. stored chunk T0 + 2*(f/2) + (l%32)/16 (clamped: rows
    // past N feed only discarded outputs), piece (2*(f%2) + l/32)*16 + l%16.
    const int8_t *a_src[LA];
    const int8_t *b_src[LB];
#pragma unroll
    for (int j = 0; j < LA; ++j) {
        const int f = wv + NW * j;
        const int g = min(m0 / 32 + (f >> 1), mg - 1);  // clamped: rows past M
        a_src[j] = act + ((size_t)(2 * g + (f & 1)) * kWave + l) * 16;
    }
#pragma unroll
    for (int j = 0; j < LB; ++j) {
        const int f = wv + NW * j;
        const int T = min(T0 + 2 * (f >> 1) + ((l & 31) >> 4), n_tiles - 1);
        const int piece = (2 * (f & 1) + (l >> 5)) * 16 + (l & 15);
        b_src[j] = tiles + ((size_t)T * kWave + piece) * 16;
    }
    const size_t a_pitch = (size_t)mg * 2 * 1024;   // bytes per K step
    const size_t b_pitch = (size_t)n_tiles * 1024;  // bytes per K slab

    // Step indices are clamped to P - 1: the loads past the end re-read the
    // last step (cached) into buffers no later step reads, which keeps the
    // number of loads per step, and so every wait count, constant.
    auto issue_a = [&](int p) __attribute__((always_inline)) {
        const unsigned st = ldsA + (unsigned)((p % NSA) * SA);
        const size_t off = (size_t)min(p, P - 1) * a_pitch;
#pragma unroll
        for (int j = 0; j < LA; ++j) dma16(a_src[j] + off, st + (wv + NW * j) * 1024);
    };
    auto issue_b = [&](int p) __attribute__((always_inline)) {
        const unsigned st = ldsB + (unsigned)((p % NSB) * SB);
        const size_t off = (size_t)min(p, P - 1) * b_pitch;
#pragma unroll
        for (int j = 0; j < LB; ++j) DMA_B(b_src[j] + off, st + (wv + NW * j) * 1024);
    };

    v16i acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) acc[i][j] = v16i{};

    // Fragments of a step in registers, two sets (current, next).
    v4i fa[2][2][TM], fb[2][2][TN];  // [set][k half][tile]
    auto lds_read = [&](auto set, int p) __attribute__((always_inline)) {
        constexpr int S = decltype(set)::value;
        const v4i *sa_ = s_buf + (size_t)(p % NSA) * (SA / 16) + l;
        const v4i *sb_ = s_buf + (size_t)(NSA * SA + (p % NSB) * SB) / 16 + l;
#pragma unroll
        for (int h = 0; h < 2; ++h) {
#pragma unroll
            for (int i = 0; i < TM; ++i) fa[S][h][i] = sa_[(2 * (wm * TM + i) + h) * kWave];
#pragma unroll
            for (int j = 0; j < TN; ++j) fb[S][h][j] = sb_[(2 * (wn * TN + j) + h) * kWave];
        }
    };
    auto mfmas = [&](auto set) __attribute__((always_inline)) {
        constexpr int S = decltype(set)::value;
#pragma unroll
        for (int h = 0; h < 2; ++h)
#pragma unroll
            for (int i = 0; i < TM; ++i)
#pragma unroll
                for (int j = 0; j < TN; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(fa[S][h][i], fb[S][h][j],
                                                                      acc[i][j], 0, 0, 0);
    };

    // The prologue replays the steady-state issue order for the steps
    // q = -(NMX-1) .. -1 (skipping loads of steps below 0), so the wait
    // count of every step is the same constant.
    for (int q = -(NMX - 1); q < 0; ++q) {
        if (q + NSA - 1 >= 0) issue_a(q + NSA - 1);
        if (q + NSB - 1 >= 0) issue_b(q + NSB - 1);
    }
    wait_barrier<WAIT0>();
    lds_read(std::integral_constant<int, 0>{}, 0);
    // Step p: wait for step p + 1's loads and barrier (all waves are past
    // step p - 1, whose buffers are refilled next), issue step p + NS - 1,
    // read step p + 1's fragments into the other register set, then the
    // MFMAs of step p (which run on while the next step waits).  The reads
    // past the last step touch a buffer no step reads; they are unused.
    auto step = [&](int p, auto cur, auto nxt) __attribute__((always_inline)) {
        wait_barrier<WAIT>();
        issue_a(p + NSA - 1);
        issue_b(p + NSB - 1);
        lds_read(nxt, p + 1);
        mfmas(cur);
    };
    using S0 = std::integral_constant<int, 0>;
    using S1 = std::integral_constant<int, 1>;
    int p = 0;
    for (; p + 1 < P; p += 2) {
        step(p, S0{}, S1{});
        step(p + 1, S1{}, S0{});
    }
    if (p < P) step(p, S0{}, S1{});
    // no load may still be writing LDS when the workgroup ends
    asm volatile("s_waitcnt vmcnt(0)" : : : "memory");

    // epilogue: lane l, register r of tile (i, j) holds row
    // m0 + 32*(wm*TM + i) + 8*(r/4) + 4*(l/32) + r%4 and column
    // n = 16*T0 + 32*(wn*TN + j) + l%32
#pragma unroll
    for (int j = 0; j < TN; ++j) {
        const int n = 16 * T0 + 32 * (wn * TN + j) + (l & 31);
        if (n >= N) continue;
        const float sw = wscales[n];
#pragma unroll
        for (int i = 0; i < TM; ++i) {
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int m = m0 + 32 * (wm * TM + i) + 8 * (r >> 2) + 4 * (l >> 5) + (r & 3);
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

template <int BM, int BN, int WM, int WN, int NSA, int NSB>
mri_status launch(const int8_t *act_packed, size_t m, const float *sa_ptr, int sa_stride,
                  float sa_value, const QMatrixDev &w, float *out, int32_t *acc_out,
                  hipStream_t s) {
    constexpr size_t lds = ((size_t)NSA * (BM / 32) + (size_t)NSB * (BN / 32)) * 2 * 1024;
    static bool attr_set = false;  // the attribute belongs to the function
    if (!attr_set) {
        MRI_HIP(hipFuncSetAttribute(
            reinterpret_cast<const void *>(&k_gemm_int8<BM, BN, WM, WN, NSA, NSB>),
            hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds));
        attr_set = true;
    }
    const size_t n_mt = (m + BM - 1) / BM;
    const size_t n_nt = (w.n_tiles + BN / 16 - 1) / (BN / 16);
    const size_t total = n_mt * n_nt;
    const size_t grid = (total + kXcds - 1) / kXcds * kXcds;
    hipLaunchKernelGGL((k_gemm_int8<BM, BN, WM, WN, NSA, NSB>), dim3((unsigned)grid),
                       dim3(WM * WN * kWave), lds, s, act_packed, (int)gemm_row_groups(m),
                       sa_ptr, sa_stride, sa_value, w.tiles, w.scales, (int)m, (int)w.n_out,
                       (int)w.n_tiles, (int)(w.kp / kChunkK), (int)n_mt, (int)total, out,
                       acc_out);
    return MRI_OK;
}

}  // namespace

// act_packed: activations in the GEMM fragment layout (gemm_pack_bytes).
mri_status launch_gemm_int8(const int8_t *act_packed, size_t m, const float *sa_ptr,
                            int sa_stride, float sa_value, const QMatrixDev &w,
                            float *out, int32_t *acc_out, hipStream_t s) {
    if (w.n_tiles == 0 || m == 0) return MRI_OK;
    // 256 x 128 tiles when they still give at least half as many workgroups
    // as CUs, else 128 x 128 (measured on MI355X at K = 4096).
    const size_t big = ((m + 255) / 256) * ((w.n_tiles + 7) / 8);
    mri_status st =
        big >= 128 ? launch<256, 128, 4, 2, 4, 8>(act_packed, m, sa_ptr, sa_stride, sa_value, w,
                                                  out, acc_out, s)
                   : launch<128, 128, 2, 2, 4, 8>(act_packed, m, sa_ptr, sa_stride, sa_value, w,
                                                  out, acc_out, s);
    if (st) return st;
    MRI_LAUNCHED("k_gemm_int8");
    return MRI_OK;
}

}  // namespace mri
