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
//
// ROWS instances read the caller's row-major int8 rows directly (no repack
// pass): an activation stage holds two K steps, 128 bytes of each of the
// tile's rows, and each DMA instruction moves 8 rows x 128 bytes (whole
// cache lines).  Piece i (16 bytes) of a row goes to slot i ^ rows_swz(row)
// of its 128-byte LDS row, so the fragment reads (32 rows at one piece
// index) spread over all banks: any 8 consecutive rows use 8 different
// slots, and so do the 8 even and the 8 odd rows of any 16 (rows r and
// r + 8 share the banks of slot s; with i ^ (row % 8) alone, 16-lane groups
// read those pairs from one bank and the counters showed a quarter of the
// LDS cycles in bank conflicts).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <type_traits>
#include <utility>

#include "common.hpp"

namespace mri {
namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));
constexpr int kWave = 64;
constexpr int kXcds = 8;

// LDS slot permutation of the ROWS stages for tile row r (bits 0-2 and 3).
__device__ inline int rows_swz(int r) { return (r & 7) ^ ((r >> 3) & 1); }

template <typename F, int... I>
__device__ inline void static_for_impl(F &&f, std::integer_sequence<int, I...>) {
    (f(std::integral_constant<int, I>{}), ...);
}
template <int N, typename F>
__device__ inline void static_for(F &&f) {
    static_for_impl(f, std::make_integer_sequence<int, N>{});
}

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

// 4 bytes per lane from g into LDS at byte address lds + 4 * lane.
__device__ inline void dma4(const void *g, unsigned lds) {
    asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dword %0, off"
                 :
                 : "v"(g), "s"(lds)
                 : "memory", "m0");
}

// Wait until at most N of this wave's loads are outstanding, then barrier.
template <int N>
__device__ inline void wait_barrier() {
    asm volatile("s_waitcnt vmcnt(%0)\n\ts_barrier" : : "n"(N) : "memory");
}

constexpr int kScDevice = 16;          // cache policy sc1: device scope
constexpr int kWaitVm0 = 0x0F70;       // s_waitcnt vmcnt(0), others untouched

// Whole output tiles, optionally split along K (ks > 1): the ks
// contributors of a tile each run a contiguous, balanced range of its K
// steps, store their int32 partial tile to a workspace slot (device-scope
// sc1 stores) and count themselves on the tile's counter; the one that
// counts last adds the other partials to its own (exact: int32 addition
// wraps and is associative, as the reference's i32 sums), applies the f32
// epilogue and resets the counter to zero for the next call.  No workgroup
// waits for another.  Splitting K puts more workgroups, and more loads in
// flight, on products whose tiles alone would leave most CUs idle.
// ROWS wait counts: the loads issued after the last one a step needs, at
// the wait of step p (before it issues its own).  Issue order per step q:
// activation stage q/2 + nsa - 1 (la2 loads, even q only), then weight step
// q + nsb - 1 (lb loads).  A step needs activation stages <= sa_req and
// weight steps <= sb_req (shift invariant: p is any large value of the
// step's parity).
constexpr int rows_wait(int p, int sa_req, int sb_req, int nsa, int nsb, int la2, int lb) {
    int idx = 0, last = -1;
    for (int q = p - 200; q < p; ++q) {
        if ((q & 1) == 0) {
            const int st = q / 2 + nsa - 1;
            for (int j = 0; j < la2; ++j, ++idx)
                if (st <= sa_req) last = idx;
        }
        const int bs = q + nsb - 1;
        for (int j = 0; j < lb; ++j, ++idx)
            if (bs <= sb_req) last = idx;
    }
    return idx - 1 - last;
}

template <int BM, int BN, int WM, int WN, int NSA, int NSB, bool ROWS = false>
__global__ __launch_bounds__(WM * WN * kWave) void k_gemm_int8(
    const int8_t *__restrict__ act, int mg, const float *__restrict__ sa_ptr, int sa_stride,
    float sa_value, const int8_t *__restrict__ tiles, const float *__restrict__ wscales,
    int M, int N, int n_tiles, int P, int n_mt, int n_tiles_total, float *__restrict__ out,
    int32_t *__restrict__ acc_out, int ks, int32_t *__restrict__ ws, int *__restrict__ cnt) {
    constexpr int NW = WM * WN;                // waves
    constexpr int FA = BM / 32 * 2, FB = BN / 32 * 2;  // fragments per K step (2 k halves)
    constexpr int TM = BM / WM / 32, TN = BN / WN / 32;  // MFMA tiles per wave
    constexpr int LA = FA / NW, LB = FB / NW;  // fragment loads per wave per step
    static_assert(FA % NW == 0 && FB % NW == 0, "load split");
    constexpr int SA = FA * 1024, SB = FB * 1024;  // bytes of one A / B stage
    static_assert(NSA >= 3 && NSB >= 3, "ring depths");
    // ROWS: NSA activation stages of two K steps (SA2 bytes, LA2 loads a wave)
    constexpr int SA2 = 2 * SA, LA2 = 2 * LA;
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
    __shared__ int s_last;

    // XCD-aware work index: this workgroup runs on XCD blockIdx % 8, and the
    // contributors of one tile (adjacent items) on the same XCD.
    const int per_xcd = (int)(gridDim.x / kXcds);
    const int item = (int)(blockIdx.x % kXcds) * per_xcd + (int)(blockIdx.x / kXcds);
    const int tile = item / ks, sp = item - tile * ks;
    if (tile >= n_tiles_total) return;
    // K steps p0 .. p0 + PS - 1 of the tile (ks <= P, so PS >= 1)
    // (ROWS: the split is in step pairs, so ranges start on a stage)
    const int PU = ROWS ? P / 2 : P;
    const int kq = PU / ks, kr = PU - kq * ks;
    const int p0 = (ROWS ? 2 : 1) * (sp * kq + min(sp, kr));
    const int PS = (ROWS ? 2 : 1) * (kq + (sp < kr ? 1 : 0));
    const int mt = tile % n_mt, nt = tile / n_mt;
    const int m0 = mt * BM, T0 = nt * (BN / 16);  // first row, first 16-row weight tile

    const int t = threadIdx.x;
    const int wv = __builtin_amdgcn_readfirstlane(t >> 6), l = t & 63;
    const int wm = wv / WN, wn = wv % WN;
    const unsigned ldsA = __builtin_amdgcn_readfirstlane((unsigned)(size_t)s_buf);
    const unsigned ldsB = ldsA + NSA * (ROWS ? SA2 : SA);

    // This wave's loads.  Fragment f = wv + NW*j holds row group f/2, k half
    // f%2.  Activations are packed (see pack layout): fragment (p, g, h) is
    // 1 KiB at ((p * mg + g) * 2 + h) KiB, so the workgroup's BM/32 row
    // groups of one K step are contiguous.  Weight lane: row 32*(f/2) + l%32
    // of the block, i.e. stored chunk T0 + 2*(f/2) + (l%32)/16 (clamped: rows
    // past N feed only discarded outputs), piece (2*(f%2) + l/32)*16 + l%16.
    const int8_t *a_src[ROWS ? LA2 : LA];
    const int8_t *b_src[LB];
#pragma unroll
    for (int j = 0; j < (ROWS ? LA2 : LA); ++j) {
        const int f = wv + NW * j;
        if constexpr (ROWS) {
            // rows of P * 64 bytes: load f covers tile rows 8f .. 8f + 7,
            // eight lanes a row, lane l%8 (slot l%8) bringing piece
            // (l%8) ^ rows_swz(row)
            const int rl = 8 * f + (l >> 3);
            const int row = min(m0 + rl, M - 1);  // clamped: rows past M
            a_src[j] = act + (size_t)row * (size_t)P * 64 + 16 * ((l & 7) ^ rows_swz(rl));
        } else {
            const int g = min(m0 / 32 + (f >> 1), mg - 1);  // clamped: rows past M
            a_src[j] = act + ((size_t)(2 * g + (f & 1)) * kWave + l) * 16;
        }
    }
#pragma unroll
    for (int j = 0; j < LB; ++j) {
        const int f = wv + NW * j;
        const int T = min(T0 + 2 * (f >> 1) + ((l & 31) >> 4), n_tiles - 1);
        const int piece = (2 * (f & 1) + (l >> 5)) * 16 + (l & 15);
        b_src[j] = tiles + ((size_t)T * kWave + piece) * 16;
    }
    // The epilogue's row and channel scales.  In the large tiles they are
    // loaded before any operand load: at the end they are a dependent memory
    // round trip between the last MFMA and the stores (and the ring's waits
    // count only the loads issued after the one they wait for, so these older
    // ones change none).  Measured (us, one box): 512 x 11008 32.2 -> 32.0,
    // 2048 x 11008 117.4 -> 116.5; in the 128 x 64 tiles, whose short K loop
    // then starts 18 loads later, 2-3 % slower, so those load them at the end.
    constexpr bool kEarlyScales = BM * BN >= 128 * 192;
    float sw[TN], sa[TM][16];
    auto load_scales = [&]() __attribute__((always_inline)) {
#pragma unroll
        for (int j = 0; j < TN; ++j)
            sw[j] = wscales[min(16 * T0 + 32 * (wn * TN + j) + (l & 31), N - 1)];
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int m =
                    min(m0 + 32 * (wm * TM + i) + 8 * (r >> 2) + 4 * (l >> 5) + (r & 3), M - 1);
                sa[i][r] = sa_ptr ? sa_ptr[(size_t)m * sa_stride] : sa_value;
            }
    };
    if constexpr (kEarlyScales) load_scales();

    const size_t a_pitch = (size_t)mg * 2 * 1024;   // bytes per K step
    const size_t b_pitch = (size_t)n_tiles * 1024;  // bytes per K slab

    // Steps p count from the range's first; their indices are clamped to
    // PS - 1: the loads past the end re-read the last step (cached) into
    // buffers no later step reads, which keeps the number of loads per step,
    // and so every wait count, constant.
    auto kstep = [&](int p) __attribute__((always_inline)) { return p0 + min(p, PS - 1); };
    auto issue_a = [&](int p) __attribute__((always_inline)) {
        const unsigned st = ldsA + (unsigned)((p % NSA) * SA);
        const size_t off = (size_t)kstep(p) * a_pitch;
#pragma unroll
        for (int j = 0; j < LA; ++j) dma16(a_src[j] + off, st + (wv + NW * j) * 1024);
    };
    // ROWS: activation stage t (steps 2t, 2t + 1) of the range into buffer t % NSA
    auto issue_a2 = [&](int t) __attribute__((always_inline)) {
        const unsigned st = ldsA + (unsigned)((t % NSA) * SA2);
        const size_t off = (size_t)(p0 / 2 + min(t, PS / 2 - 1)) * 128;
#pragma unroll
        for (int j = 0; j < LA2; ++j) dma16(a_src[j] + off, st + (wv + NW * j) * 1024);
    };
    auto issue_b = [&](int p) __attribute__((always_inline)) {
        const unsigned st = ldsB + (unsigned)((p % NSB) * SB);
        const size_t off = (size_t)kstep(p) * b_pitch;
#pragma unroll
        for (int j = 0; j < LB; ++j) dma16_nt(b_src[j] + off, st + (wv + NW * j) * 1024);
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
        const v4i *sa_ =
            s_buf + (size_t)(ROWS ? ((p >> 1) % NSA) * (SA2 / 16) : (p % NSA) * (SA / 16)) + l;
        const v4i *sb_ = s_buf + (size_t)(NSA * (ROWS ? SA2 : SA) + (p % NSB) * SB) / 16 + l;
#pragma unroll
        for (int h = 0; h < 2; ++h) {
#pragma unroll
            for (int i = 0; i < TM; ++i) {
                if constexpr (ROWS) {  // row r, piece 4 (p % 2) + 2h + l/32 of its 128 bytes
                    const int row = 32 * (wm * TM + i) + (l & 31);
                    const int pc = 4 * (p & 1) + 2 * h + (l >> 5);
                    fa[S][h][i] = sa_[row * 8 + (pc ^ rows_swz(row)) - l];
                } else {
                    fa[S][h][i] = sa_[(2 * (wm * TM + i) + h) * kWave];
                }
            }
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
    // ROWS: an even step p needs stages <= p/2 and weight step p + 1, an odd
    // one stage (p + 1)/2 as well; before the loop, stage 0 and step 0.
    constexpr int WR_E = rows_wait(1000, 500, 1001, NSA, NSB, LA2, LB);
    constexpr int WR_O = rows_wait(1001, 501, 1002, NSA, NSB, LA2, LB);
    constexpr int WR_0 = rows_wait(1000, 500, 1000, NSA, NSB, LA2, LB);
    if constexpr (ROWS) {
        constexpr int QM = 2 * (NSA - 1) > NSB - 1 ? 2 * (NSA - 1) : NSB - 1;
        for (int q = -QM; q < 0; ++q) {
            if ((q & 1) == 0 && q / 2 + NSA - 1 >= 0) issue_a2(q / 2 + NSA - 1);
            if (q + NSB - 1 >= 0) issue_b(q + NSB - 1);
        }
        wait_barrier<WR_0>();
    } else {
        for (int q = -(NMX - 1); q < 0; ++q) {
            if (q + NSA - 1 >= 0) issue_a(q + NSA - 1);
            if (q + NSB - 1 >= 0) issue_b(q + NSB - 1);
        }
        wait_barrier<WAIT0>();
    }
    lds_read(std::integral_constant<int, 0>{}, 0);
    // Step p: wait for step p + 1's loads and barrier (all waves are past
    // step p - 1, whose buffers are refilled next), issue step p + NS - 1,
    // read step p + 1's fragments into the other register set, then the
    // MFMAs of step p (which run on while the next step waits).  The reads
    // past the last step touch a buffer no step reads; they are unused.
    // (ROWS: the even steps, register set 0, issue the activation stage
    // NSA - 1 ahead; stage t's buffer last held stage t - NSA, whose reads
    // ended two steps earlier.)
    auto step = [&](int p, auto cur, auto nxt) __attribute__((always_inline)) {
        if constexpr (ROWS) {
            if constexpr (decltype(cur)::value == 0) {
                wait_barrier<WR_E>();
                issue_a2(p / 2 + NSA - 1);
            } else {
                wait_barrier<WR_O>();
            }
        } else {
            wait_barrier<WAIT>();
            issue_a(p + NSA - 1);
        }
        issue_b(p + NSB - 1);
        lds_read(nxt, p + 1);
        mfmas(cur);
    };
    using S0 = std::integral_constant<int, 0>;
    using S1 = std::integral_constant<int, 1>;
    int p = 0;
    for (; p + 1 < PS; p += 2) {
        step(p, S0{}, S1{});
        step(p + 1, S1{}, S0{});
    }
    if (p < PS) step(p, S0{}, S1{});
    // no load may still be writing LDS when the workgroup ends
    asm volatile("s_waitcnt vmcnt(0)" : : : "memory");

    if (ks > 1) {
        // Partial slot `item`: [wave][accumulator a][register group q][lane]
        // x 16 bytes, so each store and load is 1 KiB contiguous per wave.
        const __amdgpu_buffer_rsrc_t ws_rsrc = __builtin_amdgcn_make_buffer_rsrc(
            ws, 0, (int)min((long long)n_tiles_total * ks * BM * BN * 4, 0x7fffffffLL), kBufWord3);
        auto slot_off = [&](int c) {
            return (int)((((size_t)c * NW + wv) * (TM * TN * 4) * kWave + l) * 16);
        };
        const int mine = slot_off(item);
#pragma unroll
        for (int a = 0; a < TM * TN; ++a)
#pragma unroll
            for (int q = 0; q < 4; ++q)
                __builtin_amdgcn_raw_buffer_store_b128(
                    v4i{acc[a / TN][a % TN][4 * q], acc[a / TN][a % TN][4 * q + 1],
                        acc[a / TN][a % TN][4 * q + 2], acc[a / TN][a % TN][4 * q + 3]},
                    ws_rsrc, mine + (a * 4 + q) * kWave * 16, 0, kScDevice);
        // The partial is at the device's point of coherence (sc1 stores,
        // complete at vmcnt(0)) before any wave passes the barrier and the
        // count; the last contributor reads the partials with sc1 loads,
        // which do not hit lines its XCD's L2 cached before.
        __builtin_amdgcn_s_waitcnt(kWaitVm0);
        __syncthreads();
        if (t == 0)
            s_last = __hip_atomic_fetch_add(&cnt[tile], 1, __ATOMIC_RELAXED,
                                            __HIP_MEMORY_SCOPE_AGENT) == ks - 1;
        __syncthreads();
        if (!s_last) return;
        for (int c = tile * ks; c < tile * ks + ks; ++c) {
            if (c == item) continue;
            const int off = slot_off(c);
            v4i u[TM * TN][4];
#pragma unroll
            for (int a = 0; a < TM * TN; ++a)
#pragma unroll
                for (int q = 0; q < 4; ++q)
                    u[a][q] = __builtin_amdgcn_raw_buffer_load_b128(
                        ws_rsrc, off + (a * 4 + q) * kWave * 16, 0, kScDevice);
#pragma unroll
            for (int a = 0; a < TM * TN; ++a)
#pragma unroll
                for (int q = 0; q < 4; ++q)
#pragma unroll
                    for (int e = 0; e < 4; ++e) acc[a / TN][a % TN][4 * q + e] += u[a][q][e];
        }
        if (t == 0)  // ready for the next call on this stream
            __hip_atomic_store(&cnt[tile], 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }

    // epilogue: lane l, register r of tile (i, j) holds row
    // m0 + 32*(wm*TM + i) + 8*(r/4) + 4*(l/32) + r%4 and column
    // n = 16*T0 + 32*(wn*TN + j) + l%32.  The scales are loaded before any
    // store: a global load issued after output stores would wait for those
    // stores (one in-order counter covers both).
    if constexpr (!kEarlyScales) load_scales();
    if (acc_out) {  // with the int32 accumulators: element stores
#pragma unroll
        for (int j = 0; j < TN; ++j) {
            const int n = 16 * T0 + 32 * (wn * TN + j) + (l & 31);
            if (n >= N) continue;
#pragma unroll
            for (int i = 0; i < TM; ++i) {
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const int m = m0 + 32 * (wm * TM + i) + 8 * (r >> 2) + 4 * (l >> 5) + (r & 3);
                    if (m < M) {
                        float v = (float)acc[i][j][r] * sa[i][r];
                        v = v * sw[j];
                        out[(size_t)m * N + n] = v;
                        acc_out[(size_t)m * N + n] = acc[i][j][r];
                    }
                }
            }
        }
        return;
    }
    // f32 outputs only: the tile is staged in LDS (the ring is free: every
    // wave's loads have landed and the barrier ends all reads of it) and
    // written row by row, 16 contiguous bytes per lane, which measured
    // ~6 us faster than element stores at M = 512, N = 11008.
    constexpr int PITCH = BN + 4;  // floats per staged row (pads the banks)
    float *st = reinterpret_cast<float *>(s_buf);
    __syncthreads();
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int rt = 32 * (wm * TM + i) + 8 * (r >> 2) + 4 * (l >> 5) + (r & 3);
                float v = (float)acc[i][j][r] * sa[i][r];
                st[rt * PITCH + 32 * (wn * TN + j) + (l & 31)] = v * sw[j];
            }
    __syncthreads();
    constexpr int V = BN / 4;  // 16-byte vectors per row
    const int n0 = 16 * T0;
    const bool vec = (N & 3) == 0 && ((size_t)out & 15) == 0;
    for (int e = t; e < BM * V; e += NW * kWave) {
        const int rt = e / V, c4 = e - rt * V;
        const int m = m0 + rt, n = n0 + 4 * c4;
        if (m >= M || n >= N) continue;
        typedef float v4f __attribute__((ext_vector_type(4)));
        const v4f v = *reinterpret_cast<const v4f *>(st + rt * PITCH + 4 * c4);
        float *dst = out + (size_t)m * N + n;
        if (vec && n + 4 <= N) {
            *reinterpret_cast<v4f *>(dst) = v;
        } else {
            const float vv[4] = {v.x, v.y, v.z, v.w};
            for (int q = 0; q < 4 && n + q < N; ++q) dst[q] = vv[q];
        }
    }
}

// Dynamic LDS of k_gemm_int8: the ring, or the staged output tile.
template <int BM, int BN, int NSA, int NSB>
constexpr size_t gemm_lds_bytes() {
    constexpr size_t ring = ((size_t)NSA * (BM / 32) + (size_t)NSB * (BN / 32)) * 2 * 1024;
    constexpr size_t stage = (size_t)BM * (BN + 4) * 4;
    return ring > stage ? ring : stage;
}

// ---------------------------------------------------------------------------
// Stream-K form for the larger products: 256 x 256 output tiles, eight waves
// (4 x 2) of 64 x 128 each (8 accumulators of 32 x 32), a 4-stage LDS ring
// of 32 KiB K steps, and the loads and LDS reads of the next steps placed
// between the MFMAs of the current one.
//
// The K steps of all tiles form one sequence of iterations (tile-major, the
// M tiles of a weight column block adjacent); every workgroup of a
// persistent grid (one per CU) takes an equal contiguous range of it, so
// the work is balanced whatever the tile count.  The ring runs on across
// tile boundaries.  A tile whose K range is split between workgroups is
// finished by whichever contributor arrives last: the others store their
// int32 partial tile to a workspace slot and increment the tile's counter;
// the last one adds the partials to its own (exact: int32 addition wraps
// and is associative, as the reference's i32 sums), applies the f32
// epilogue and resets the counter to zero for the next call.  No workgroup
// waits for another.
// ---------------------------------------------------------------------------
constexpr int kSkNs = 4;                        // ring stages
constexpr int kSkTileInts = 256 * 256;          // int32 of one partial tile
constexpr int kSkMaxTiles = kGemmWsCounters;    // tile counters at the workspace start

// Split of `iters` iterations into nwg ranges: q = iters / nwg each, the
// first rem = iters % nwg ranges one more.  Neither query divides by more
// than a 32-bit uniform value.
struct SkSplit {
    int q, rem;
    __device__ SkSplit(int iters, int nwg) : q(iters / nwg), rem(iters - iters / nwg * nwg) {}
    // first iteration of range r
    __device__ int start(int r) const { return r * q + min(r, rem); }
    // range that holds iteration i (q >= 1)
    __device__ int owner(int i) const {
        const int b = (q + 1) * rem;
        return i < b ? i / (q + 1) : rem + (i - b) / q;
    }
};

template <int NS, int TN, bool ACC>
__global__ __launch_bounds__(512) void k_gemm_sk(
    const int8_t *__restrict__ act, int mg, const float *__restrict__ sa_ptr, int sa_stride,
    float sa_value, const int8_t *__restrict__ tiles, const float *__restrict__ wscales,
    int M, int N, int n_tiles, int P, int n_mt, int iters, float *__restrict__ out,
    int32_t *__restrict__ acc_out, int32_t *__restrict__ ws, int *__restrict__ cnt) {
    // 8 waves, 4 along M x 2 along N; wave (wm, wn) = (wv / 2, wv % 2) owns
    // rows 64*wm.. (TM 32-row blocks) and columns 32*TN*wn.. (TN blocks) of
    // a 256 x BN tile.  With TN = 4, 128 accumulator registers per wave stay
    // in VGPRs beside the fragments, two waves per SIMD.
    constexpr int NW = 8, TM = 2, BN = 64 * TN;
    constexpr int LA = 16 / NW, LB = 2 * BN / 32 / NW;  // fragment loads per wave per step
    constexpr int SA = 16 * 1024, SB = BN / 32 * 2048;  // bytes of one A / B stage
    static_assert(TN == 2 || TN == 4, "tile width");
    constexpr int WAIT = (NS - 3) * (LA + LB);
    constexpr int WAIT0 = WAIT + LA + LB;
    extern __shared__ v4i s_buf[];
    __shared__ int s_last;
    // activation row and weight column scales of a segment's tile, double
    // buffered by segment parity: a wave may fill the next segment's while
    // another still reads this one's
    __shared__ __attribute__((aligned(16))) float s_scale[2][2][256];

    const int nwg = (int)gridDim.x;  // a multiple of 8
    // range index, XCD-major: the ranges of one XCD are adjacent, so the
    // contributors of a tile (and the M tiles sharing weights) share its L2
    const int r = (int)(blockIdx.x % kXcds) * (nwg / kXcds) + (int)(blockIdx.x / kXcds);
    const SkSplit split(iters, nwg);  // nwg <= iters (the launcher's choice)
    const int it0 = split.start(r), it1 = split.start(r + 1);

    const int t = threadIdx.x;
    const int wv = __builtin_amdgcn_readfirstlane(t >> 6), l = t & 63;
    const int wm = wv >> 1, wn = wv & 1;
    const unsigned ldsA = __builtin_amdgcn_readfirstlane((unsigned)(size_t)s_buf);
    const unsigned ldsB = ldsA + NS * SA;
    const size_t a_pitch = (size_t)mg * 2 * 1024;   // bytes per K step
    const size_t b_pitch = (size_t)n_tiles * 1024;  // bytes per K slab

    // Loads of iteration i (clamped to the range's last: loads past the end
    // re-read it into a stage no later step reads, so every wait count is
    // constant).  Fragment f = wv + NW*j: row / weight-column group f/2, k
    // half f%2 (layouts as in k_gemm_int8).  The per-lane parts of the
    // addresses are fixed; next_desc() adds the iteration's.
    // Fragment f = wv + NW*j has the same k half (wv & 1) for every j, so the
    // per-lane part of every A / B address is one offset: A lane l of the
    // 1 KiB fragment, B piece (2*(f%2) + l/32)*16 + l%16 of stored chunk
    // 2*(f/2) + (l%32)/16 of the block.
    const unsigned a_loff = (unsigned)(((wv & 1) * kWave + l) * 16);
    const unsigned b_loff = (unsigned)(((2 * (wv & 1) + (l >> 5)) * 16 + (l & 15)) * 16);
    const int b_lsub = (l & 31) >> 4;
    struct Desc {
        size_t a_off, b_off;  // bytes of the K step
        int g0, T0;           // first row group, first 16-row weight tile
        unsigned sa, sb;      // LDS stages
    };
    // Load cursor: the loads are issued for iterations it0, it0 + 1, ... in
    // order, one iteration per call of next_desc(), so the tile coordinates
    // are carried forward instead of divided out each step.
    int lc_i = it0, lc_n = 0, lc_p, lc_mt, lc_nt;
    {
        const int tl = it0 / P;
        lc_p = it0 - tl * P;
        lc_nt = tl / n_mt;
        lc_mt = tl - lc_nt * n_mt;
    }
    auto next_desc = [&]() __attribute__((always_inline)) {
        Desc d;
        d.a_off = (size_t)lc_p * a_pitch;
        d.b_off = (size_t)lc_p * b_pitch;
        d.g0 = lc_mt * 8;
        d.T0 = lc_nt * (BN / 16);
        const int stg = lc_n % NS;
        d.sa = ldsA + (unsigned)(stg * SA);
        d.sb = ldsB + (unsigned)(stg * SB);
        ++lc_n;
        if (lc_i + 1 < it1) {  // else stay clamped to the range's last
            ++lc_i;
            if (++lc_p == P) {
                lc_p = 0;
                if (++lc_mt == n_mt) {
                    lc_mt = 0;
                    ++lc_nt;
                }
            }
        }
        return d;
    };
    auto dma = [&](const Desc &d, int j, bool b) __attribute__((always_inline)) {
        const unsigned f = (unsigned)(wv + NW * j);
        if (!b) {
            const int g = min(d.g0 + (wv >> 1) + (NW / 2) * j, mg - 1);
            dma16(act + d.a_off + (size_t)g * 2048 + a_loff, d.sa + f * 1024);
        } else {
            const int T = min(d.T0 + 2 * (wv >> 1) + NW * j + b_lsub, n_tiles - 1);
            dma16(tiles + d.b_off + (size_t)T * 1024 + b_loff, d.sb + f * 1024);
        }
    };

    v16i acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) acc[i][j] = v16i{};
    // Fragments of one k half: the MFMAs of half h of a step read fa[h] /
    // fb[h] while the other half's registers are refilled (half 1 of the
    // same iteration, or half 0 of the next).
    v4i fa[2][TM], fb[2][TN];  // [k half][tile]
    auto rd_a = [&](int i, int h, int q) __attribute__((always_inline)) {
        fa[h][q] = s_buf[(size_t)((unsigned)(i - it0) % NS) * (SA / 16) + (2 * (wm * TM + q) + h) * kWave + l];
    };
    auto rd_b = [&](int i, int h, int q) __attribute__((always_inline)) {
        fb[h][q] = s_buf[(size_t)(NS * SA + ((unsigned)(i - it0) % NS) * SB) / 16 + (2 * (wn * TN + q) + h) * kWave + l];
    };

    // f32 epilogue (int8.rs:93).  Register group q of accumulator (i, j)
    // holds 4 values: element e4 is tile row 32*(wm*TM + i) + 8*q +
    // 4*(l/32) + e4 and column 32*(wn*TN + j) + l%32.  The scales come from
    // LDS (s_scale), filled by load_scales when the segment starts: LDS
    // reads do not wait for the output stores, where global loads issued
    // after them would (one in-order counter covers loads and stores).
    const unsigned lds_scale = __builtin_amdgcn_readfirstlane((unsigned)(size_t)&s_scale[0][0][0]);
    auto load_scales = [&](int tl, int buf) __attribute__((always_inline)) {
        const int m0 = (tl % n_mt) * 256, n0 = (tl / n_mt) * BN;
        // waves 0-3: the 256 row scales, waves 4..: the BN column scales
        const unsigned base = lds_scale + (unsigned)(buf * 2048 + wv * 256);
        if (wv < 4) {
            if (sa_ptr) dma4(sa_ptr + (size_t)min(m0 + 64 * wv + l, M - 1) * sa_stride, base);
        } else if (wv < 4 + BN / 64) {
            dma4(wscales + min(n0 + 64 * (wv - 4) + l, N - 1), base);
        }
    };
    // Output stores go through buffer resources: the row step of an
    // element (e4 * N * 4 bytes) is a uniform offset and the column block an
    // immediate one, so a store needs no per-element address arithmetic, and
    // rows past M fall outside the resource, where stores are dropped.
    const int row_bytes = N * 4;
    const __amdgpu_buffer_rsrc_t out_rsrc = __builtin_amdgcn_make_buffer_rsrc(
        out, 0, (int)min((long long)M * N * 4, 0x7fffffffLL), kBufWord3);
    const __amdgpu_buffer_rsrc_t acc_rsrc = __builtin_amdgcn_make_buffer_rsrc(
        acc_out, 0, ACC ? (int)min((long long)M * N * 4, 0x7fffffffLL) : 0, kBufWord3);
    auto col_scales = [&](int buf, float (&sw)[TN]) __attribute__((always_inline)) {
#pragma unroll
        for (int j = 0; j < TN; ++j) sw[j] = s_scale[buf][1][32 * (wn * TN + j) + (l & 31)];
    };
    auto put4 = [&](int tl, int buf, const float (&sw)[TN], int i, int j, int q, const v4i &v)
                    __attribute__((always_inline)) {
        const int m0 = (tl % n_mt) * 256, n0 = (tl / n_mt) * BN;
        const int n = n0 + 32 * (wn * TN + j) + (l & 31);
        const int rt = 32 * (wm * TM + i) + 8 * q + 4 * (l >> 5);  // tile row of e4 = 0
        typedef float v4f __attribute__((ext_vector_type(4)));
        const v4f sa = sa_ptr ? *reinterpret_cast<const v4f *>(&s_scale[buf][0][rt])
                              : v4f{sa_value, sa_value, sa_value, sa_value};
        if (n >= N) return;
        const int voff = (m0 + rt) * row_bytes + n * 4;
#pragma unroll
        for (int e4 = 0; e4 < 4; ++e4) {
            float o = (float)v[e4] * sa[e4];
            o = o * sw[j];
            __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(int, o), out_rsrc, voff,
                                                  e4 * row_bytes, 0);
            if constexpr (ACC)
                __builtin_amdgcn_raw_buffer_store_b32(v[e4], acc_rsrc, voff, e4 * row_bytes, 0);
        }
    };
    auto epilogue = [&](int tl, int buf) __attribute__((always_inline)) {
        float sw[TN];
        col_scales(buf, sw);
        static_for<TM * TN * 4>([&](auto gg) {
            constexpr int a = decltype(gg)::value / 4, q = decltype(gg)::value % 4;
            put4(tl, buf, sw, a / TN, a % TN, q,
                 v4i{acc[a / TN][a % TN][4 * q], acc[a / TN][a % TN][4 * q + 1],
                     acc[a / TN][a % TN][4 * q + 2], acc[a / TN][a % TN][4 * q + 3]});
        });
    };
    // Partial tile slot of range c in tile tl: 0 when the range starts in
    // the tile (its first segment), else 1 (its last segment).  Slot layout:
    // [wave][accumulator a][register group q][lane] x 16 bytes.  Partials
    // are written and read with device-scope (sc1) buffer accesses, which
    // reach the point of coherence of all XCDs, so neither side needs a
    // cache-wide fence (see the arrival count below).
    const __amdgpu_buffer_rsrc_t ws_rsrc = __builtin_amdgcn_make_buffer_rsrc(
        ws, 0, (int)min((long long)nwg * 2 * kSkTileInts * 4, 0x7fffffffLL), kBufWord3);
    auto slot_of = [&](int c, int tl) {
        return split.start(c) >= tl * P ? 0 : 1;
    };
    auto slot_off = [&](int c, int slot) {  // byte offset of this lane's first vector
        return (int)(((size_t)(2 * c + slot) * kSkTileInts +
                      ((size_t)wv * (TM * TN * 4 * kWave) + l) * 4) * 4);
    };
    // End of a segment [k0, k1) of tile tl.  A split tile: every contributor
    // stores its partial and counts itself; the one that counts last sums
    // all slots (int32) and applies the epilogue.
    auto finish = [&](int tl, int k0, int k1, int buf) __attribute__((always_inline)) {
        // The scale loads, issued before the segment's first step, are
        // complete and visible after the second step's wait and barrier; a
        // one-step segment waits here.
        if (k1 - k0 < 2) wait_barrier<0>();
        if (k0 == 0 && k1 == P) {
            epilogue(tl, buf);
            return;
        }
        const int c0 = split.owner(tl * P), c1 = split.owner(tl * P + P - 1);
        const int mine = slot_off(r, slot_of(r, tl));
        static_for<TM * TN>([&](auto aa) {
            constexpr int a = decltype(aa)::value;
#pragma unroll
            for (int q = 0; q < 4; ++q)
                __builtin_amdgcn_raw_buffer_store_b128(
                    v4i{acc[a / TN][a % TN][4 * q], acc[a / TN][a % TN][4 * q + 1],
                        acc[a / TN][a % TN][4 * q + 2], acc[a / TN][a % TN][4 * q + 3]},
                    ws_rsrc, mine + (a * 4 + q) * kWave * 16, 0, kScDevice);
        });
        __builtin_amdgcn_s_waitcnt(kWaitVm0);  // the partial has reached the device
        __syncthreads();
        // Ordering is by the hardware, not by a C++ release/acquire pair:
        // the partials are device-scope (sc1) stores, write-through to the
        // point of coherence of all XCDs, complete at vmcnt(0) above before
        // any wave passes the barrier; the last contributor reads them with
        // sc1 loads, which do not hit lines its XCD's L2 cached before.  An
        // agent-scope release here compiles to buffer_wbl2 (a write-back of
        // the XCD's whole L2) and measured 14 % slower at 2048 x 11008.
        if (t == 0)
            s_last = __hip_atomic_fetch_add(&cnt[tl], 1, __ATOMIC_RELAXED,
                                            __HIP_MEMORY_SCOPE_AGENT) == c1 - c0;
        __syncthreads();
        if (!s_last) return;
        // Sum of all slots, one accumulator (4 vectors) per pass; the next
        // pass's loads are issued before this pass's stores (they would
        // otherwise wait for the stores), up to four contributors at a time.
        float sw[TN];
        col_scales(buf, sw);
        auto load_pass = [&](int a, int cb, v4i (&u)[4][4]) __attribute__((always_inline)) {
#pragma unroll
            for (int cc = 0; cc < 4; ++cc) {
                const int c = min(cb + cc, c1);
                const int off = slot_off(c, slot_of(c, tl)) + a * 4 * kWave * 16;
#pragma unroll
                for (int v = 0; v < 4; ++v)
                    u[cc][v] = __builtin_amdgcn_raw_buffer_load_b128(ws_rsrc, off + v * kWave * 16, 0,
                                                                   kScDevice);
            }
        };
        v4i u[4][4];
        load_pass(0, c0, u);
        static_for<TM * TN>([&](auto aa) {
            constexpr int a = decltype(aa)::value;
            v4i sum[4];
#pragma unroll
            for (int v = 0; v < 4; ++v) sum[v] = v4i{0, 0, 0, 0};
            for (int cb = c0;;) {
#pragma unroll
                for (int cc = 0; cc < 4; ++cc)
                    if (cb + cc <= c1) {
#pragma unroll
                        for (int v = 0; v < 4; ++v) sum[v] += u[cc][v];
                    }
                cb += 4;
                if (cb > c1) break;
                load_pass(a, cb, u);  // more than four contributors
            }
            if constexpr (a + 1 < TM * TN) load_pass(a + 1, c0, u);
#pragma unroll
            for (int v = 0; v < 4; ++v) put4(tl, buf, sw, a / TN, a % TN, v, sum[v]);
        });
        if (t == 0)  // ready for the next call on this stream
            __hip_atomic_store(&cnt[tl], 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    };

    // prologue: the first segment's scales, iterations it0 .. it0 + NS - 2
    load_scales(it0 / P, 0);
#pragma unroll
    for (int q = 0; q < NS - 1; ++q) {
        const Desc d = next_desc();  // iteration it0 + q
#pragma unroll
        for (int j = 0; j < LA; ++j) dma(d, j, false);
#pragma unroll
        for (int j = 0; j < LB; ++j) dma(d, j, true);
    }
    wait_barrier<WAIT0>();
    using RD = std::true_type;
    using NORD = std::false_type;
    // half 0 of iteration i (in LDS and visible)
    auto read_h0 = [&](int i) __attribute__((always_inline)) {
#pragma unroll
        for (int q = 0; q < TM; ++q) rd_a(i, 0, q);
#pragma unroll
        for (int q = 0; q < TN; ++q) rd_b(i, 0, q);
    };
    read_h0(it0);
    // Step i: wait for iteration i+1's loads and barrier (all waves are
    // past step i-1, whose stage is refilled next), then the 16 MFMAs of
    // step i with the 4 loads of iteration i+NS-1 placed between them, and
    // the fragment reads: half 1 of iteration i during half 0's MFMAs, and,
    // unless it is the segment's last step, half 0 of iteration i+1 during
    // half 1's.  Reads go in order of first use (A0, B0..B3, A1).
    auto step = [&](int i, auto rd) __attribute__((always_inline)) {
        const Desc d = next_desc();  // iteration i + NS - 1
        wait_barrier<WAIT>();
        static_for<2 * TM * TN>([&](auto kk) {
            constexpr int k = decltype(kk)::value;
            constexpr int h = k / (TM * TN), ii = (k / TN) % TM, jj = k % TN;
            acc[ii][jj] =
                __builtin_amdgcn_mfma_i32_32x32x32_i8(fa[h][ii], fb[h][jj], acc[ii][jj], 0, 0, 0);
            // load n goes with MFMA n * MF / (LA + LB)
            constexpr int MF = 2 * TM * TN, ND = LA + LB;
            constexpr int n = (k * ND + MF - 1) / MF;  // first load at or after MFMA k
            if constexpr (n < ND && n * MF / ND == k) {
                if constexpr (n < LA) dma(d, n, false);
                else dma(d, n - LA, true);
            }
            // fragment read slot of the half: from its second MFMA when the
            // half has more MFMAs than reads
            constexpr int rr = k % (TM * TN) - (TM * TN > TM + TN ? 1 : 0);
            if constexpr (rr >= 0 && rr < TM + TN && (h == 0 || decltype(rd)::value)) {
                const int ir = h == 0 ? i : i + 1;
                if constexpr (rr == 0) rd_a(ir, 1 - h, 0);
                else if constexpr (rr <= TN) rd_b(ir, 1 - h, rr - 1);
                else rd_a(ir, 1 - h, rr - TN);
            }
            __builtin_amdgcn_sched_barrier(0);
        });
    };
    // Segments: the steps of one tile within the range, then the segment's
    // end.  The last step reads no fragments ahead, so no fragment is held
    // in registers across the end; the next segment's first ones are read
    // after it (its stage is complete since the last step's wait, and
    // refilled two steps later).
    for (int i = it0, buf = 0; i < it1; buf ^= 1) {
        const int tl = i / P;
        const int s1 = min(it1, (tl + 1) * P);
        int j = i;
        for (; j + 1 < s1; ++j) step(j, RD{});
        step(j, NORD{});
        finish(tl, i - tl * P, s1 - tl * P, buf);
        // nothing the compiler tracks may be outstanding where the next
        // segment's loop starts, or it waits for it inside the loop
        __builtin_amdgcn_s_waitcnt(kWaitVm0);
#pragma unroll
        for (int a = 0; a < TM; ++a)
#pragma unroll
            for (int b = 0; b < TN; ++b) acc[a][b] = v16i{};
        i = s1;
        if (i < it1) {
            load_scales(i / P, buf ^ 1);
            read_h0(i);
        }
    }
    // no load may still be writing LDS when the workgroup ends
    asm volatile("s_waitcnt vmcnt(0)" : : : "memory");
}

// ks > 1: K split in ks ranges per tile, with ws the stream-K workspace
// (tile counters first, then the partial slots).
template <int BM, int BN, int WM, int WN, int NSA, int NSB, bool ROWS = false>
mri_status launch(const int8_t *act_packed, size_t m, const float *sa_ptr, int sa_stride,
                  float sa_value, const QMatrixDev &w, float *out, int32_t *acc_out,
                  hipStream_t s, int ks = 1, void *ws = nullptr) {
    constexpr size_t lds = gemm_lds_bytes<BM, BN, ROWS ? 2 * NSA : NSA, NSB>();
    static DeviceOnce attr;  // the attribute belongs to the function
    MRI_HIP(attr.run([&](int) {
        return hipFuncSetAttribute(
            reinterpret_cast<const void *>(&k_gemm_int8<BM, BN, WM, WN, NSA, NSB, ROWS>),
            hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    }));
    const size_t n_mt = (m + BM - 1) / BM;
    const size_t n_nt = (w.n_tiles + BN / 16 - 1) / (BN / 16);
    const size_t total = n_mt * n_nt;
    if (ks < 1 || (size_t)ks > w.kp / kChunkK || (ks > 1 && !ws))
        return set_error(MRI_ERR_INVALID_ARGUMENT, "gemm: bad K split");
    const size_t grid = (total * ks + kXcds - 1) / kXcds * kXcds;
    int *cnt = static_cast<int *>(ws);
    int32_t *part = ws ? reinterpret_cast<int32_t *>(cnt + kSkMaxTiles) : nullptr;
    hipLaunchKernelGGL((k_gemm_int8<BM, BN, WM, WN, NSA, NSB, ROWS>), dim3((unsigned)grid),
                       dim3(WM * WN * kWave), lds, s, act_packed, (int)gemm_row_groups(m),
                       sa_ptr, sa_stride, sa_value, w.tiles, w.scales, (int)m, (int)w.n_out,
                       (int)w.n_tiles, (int)(w.kp / kChunkK), (int)n_mt, (int)total, out,
                       acc_out, ks, part, cnt);
    return MRI_OK;
}

// Stream-K geometry of an m-row product: workgroups (one per CU, at most
// one per iteration, a multiple of 8) and iterations (tiles x K steps).
struct SkShape {
    int nwg = 0, iters = 0, n_mt = 0, n_tt = 0;
};
SkShape sk_shape(size_t m, const QMatrixDev &w, int bn) {
    const int cus = device_cus();
    SkShape sh;
    if (cus <= 0) return sh;
    sh.n_mt = (int)((m + 255) / 256);
    sh.n_tt = sh.n_mt * (int)((w.n_tiles + bn / 16 - 1) / (bn / 16));
    const long long iters = (long long)sh.n_tt * (long long)(w.kp / kChunkK);
    // buffer offsets of the epilogue are 32-bit: the output must stay below 2 GiB
    if (iters > (1LL << 30) || sh.n_tt > kSkMaxTiles ||
        (long long)m * (long long)w.n_out * 4 > 0x7fffffffLL)
        return SkShape{};
    sh.iters = (int)iters;
    sh.nwg = (int)(std::min<long long>(cus, iters) / kXcds * kXcds);
    return sh;
}

template <int TN>
mri_status launch_sk(const int8_t *act_packed, size_t m, const float *sa_ptr, int sa_stride,
                     float sa_value, const QMatrixDev &w, float *out, int32_t *acc_out,
                     void *ws, const SkShape &sh, hipStream_t s) {
    constexpr size_t lds = (size_t)kSkNs * (16 * 1024 + 2 * TN * 2048);
    static DeviceOnce attr;
    MRI_HIP(attr.run([&](int) {
        hipError_t e = hipFuncSetAttribute(
            reinterpret_cast<const void *>(&k_gemm_sk<kSkNs, TN, false>),
            hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
        if (e != hipSuccess) return e;
        return hipFuncSetAttribute(reinterpret_cast<const void *>(&k_gemm_sk<kSkNs, TN, true>),
                                   hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    }));
    auto *cnt = static_cast<int *>(ws);
    auto *part = reinterpret_cast<int32_t *>(cnt + kSkMaxTiles);
    auto *kern = acc_out ? &k_gemm_sk<kSkNs, TN, true> : &k_gemm_sk<kSkNs, TN, false>;
    hipLaunchKernelGGL(kern, dim3((unsigned)sh.nwg), dim3(512), lds, s, act_packed,
                       (int)gemm_row_groups(m), sa_ptr, sa_stride, sa_value, w.tiles, w.scales,
                       (int)m, (int)w.n_out, (int)w.n_tiles, (int)(w.kp / kChunkK), sh.n_mt,
                       sh.iters, out, acc_out, part, cnt);
    MRI_LAUNCHED("k_gemm_sk");
    return MRI_OK;
}

// Kernel plan of an m-row product.  Measured on MI355X (random int8
// operands, K = 4096 and 11008, M = 64 .. 1024, N = 4096 and 11008): the K
// loop of every tile shape is bound by the CU's LDS port (DMA writes plus
// each wave's fragment reads) more than by HBM or MFMA, so the shape that
// keeps the most CUs busy in one pass wins, and a K split pays for its
// partial tiles only while it adds CUs.
//  - 128 x 64 tiles when at most one per CU and either one M tile (M <= 128)
//    or at least half the CUs: 128 x 4096 x 4096 in 11.8 us with a 4-way K
//    split (24.8 us as 128 x 128 tiles), 512 x 4096 x 4096 in 18.1 us;
//  - 128 x 128 tiles when they fit one pass: 1024 x 4096 x 4096 in 26.2 us
//    (36.3 us as stream-K), 256 x 11008 x 4096 in 24.4 us;
//  - else 256 x 256 stream-K when its tiles come in whole passes (no split
//    tile: 4096 x 4096 x 4096 in 82.7 us, 92.2 as 256 x 128 whole tiles),
//  - else the cheapest of 256 x 128 whole tiles, 128 x 192 whole tiles and
//    256 x 128 stream-K.  A whole-tile launch takes about one tile's time per
//    pass of the CUs, however full the last pass (~37.5 us at K = 4096 for
//    256 x 128, ~35 for 128 x 192), and stream-K about 1.6 tile times per
//    pass of work (its partial tiles and fix-ups): at K = 4096, N = 11008,
//    M = 512 / 768 / 1024 / 1280 / 1536 / 2048 take 35.8 / 70.7 / 75.3 / 81.0
//    / 115 / 127 us as 256 x 128 whole tiles, 34.2 / 66.0 / 69-76 / 105 /
//    112 / 149 as 128 x 192 and - / 62.9 / 86 / 102 / 118 / 153 as stream-K.
// A K split is at most 4-way, keeps at least 16 K steps per contributor
// and at most one workgroup per CU.
enum class GemmKind { T128x64, T128x128, T128x192, T256x128, SK128, SK256 };
struct GemmPlan {
    GemmKind kind = GemmKind::T256x128;
    int ks = 1;
    SkShape sk;
    size_t tiles = 0;  // whole tiles of the T kinds
};

GemmPlan plan_gemm(size_t m, const QMatrixDev &w) {
    GemmPlan pl;
    const size_t cus = (size_t)std::max(device_cus(), 0);
    const size_t P = w.kp / kChunkK;
    const size_t mt128 = (m + 127) / 128;
    const size_t t64 = mt128 * ((w.n_tiles + 3) / 4), t128 = mt128 * ((w.n_tiles + 7) / 8);
    auto split = [&](size_t tiles) {
        const size_t ks = std::min<size_t>({cus / tiles, 4, P / 16});
        return (int)std::max<size_t>(ks, 1);
    };
    if (cus > 0 && t64 <= cus && (mt128 == 1 || 2 * t64 >= cus)) {
        pl.kind = GemmKind::T128x64;
        pl.tiles = t64;
        pl.ks = split(t64);
        return pl;
    }
    if (cus > 0 && t128 <= cus) {
        pl.kind = GemmKind::T128x128;
        pl.tiles = t128;
        pl.ks = split(t128);
        return pl;
    }
    const size_t big = ((m + 255) / 256) * ((w.n_tiles + 7) / 8);
    const size_t mid = mt128 * ((w.n_tiles + 11) / 12);  // 128 x 192 tiles
    pl.kind = GemmKind::T256x128;
    pl.tiles = big;
    if (cus == 0) return pl;
    const SkShape sh4 = sk_shape(m, w, 256), sh2 = sk_shape(m, w, 128);
    if (sh4.nwg > 0 && sh4.n_tt >= sh4.nwg && sh4.n_tt % sh4.nwg == 0) {
        pl.kind = GemmKind::SK256;
        pl.sk = sh4;
        return pl;
    }
    auto passes = [&](size_t tiles) { return (double)((tiles + cus - 1) / cus); };
    const double t_big = passes(big), t_mid = 0.94 * passes(mid);
    const double t_sk = sh2.nwg > 0 ? 1.6 * (double)big / (double)cus : 1e30;
    if (t_mid < t_big && t_mid <= t_sk) {
        pl.kind = GemmKind::T128x192;
        pl.tiles = mid;
    } else if (t_sk < t_big) {
        pl.kind = GemmKind::SK128;
        pl.sk = sh2;
    }
    return pl;
}

size_t plan_ws_bytes(const GemmPlan &pl) {
    switch (pl.kind) {
        case GemmKind::SK128:
        case GemmKind::SK256:
            // [tile counters, fixed place and size][partial tiles: 2 slots per workgroup]
            return (size_t)kSkMaxTiles * sizeof(int) +
                   (size_t)pl.sk.nwg * 2 * kSkTileInts * sizeof(int32_t);
        case GemmKind::T128x64:
        case GemmKind::T128x128:
            if (pl.ks > 1) {
                const size_t tile = pl.kind == GemmKind::T128x64 ? 128 * 64 : 128 * 128;
                return (size_t)kSkMaxTiles * sizeof(int) +
                       pl.tiles * (size_t)pl.ks * tile * sizeof(int32_t);
            }
            return 0;
        default:
            return 0;
    }
}

}  // namespace

size_t gemm_ws_bytes(size_t m, const QMatrixDev &w) { return plan_ws_bytes(plan_gemm(m, w)); }

// The caller's int8 rows ([m][k], 16-byte aligned) can feed the GEMM as they
// are when the plan takes 128-row whole tiles and K is a whole number of
// 128-byte stages with no padding; the other plans (256-row tiles, stream-K)
// read the packed layout.  Measured against the repack pass plus the packed
// kernel: the ROWS kernel takes 0.2-0.8 us more at these plans (512 x 11008:
// 35.0 against 34.2-34.8; 128 x 11008: 16.8 against 16.6) and saves the
// 4-5 us repack; at 256-row tiles it was 7 us slower (2048 x 11008).
bool gemm_rows_ok(size_t m, const QMatrixDev &w, const void *act) {
    if ((reinterpret_cast<uintptr_t>(act) & 15) || w.k_in != w.kp || w.kp % 128) return false;
    const GemmKind k = plan_gemm(m, w).kind;
    return k == GemmKind::T128x64 || k == GemmKind::T128x128 || k == GemmKind::T128x192;
}

// act_packed: activations in the GEMM fragment layout (gemm_pack_bytes).
// ws: gemm_ws_bytes(m, w) bytes (may be null when that is 0); its first
// kSkMaxTiles ints (the tile counters, at the same place for every shape)
// were zeroed when it was allocated, and every call leaves them zero again.
// Without a workspace the plan falls back to whole tiles and no K split.
mri_status launch_gemm_int8(const int8_t *act_packed, size_t m, const float *sa_ptr,
                            int sa_stride, float sa_value, const QMatrixDev &w,
                            float *out, int32_t *acc_out, void *ws, hipStream_t s, bool rows) {
    if (w.n_tiles == 0 || m == 0) return MRI_OK;
    GemmPlan pl = plan_gemm(m, w);
    if (!ws) {
        pl.ks = 1;
        if (pl.kind == GemmKind::SK128 || pl.kind == GemmKind::SK256) pl.kind = GemmKind::T256x128;
    }
    mri_status st = MRI_OK;
    if (rows) {  // act_packed holds the caller's rows (gemm_rows_ok)
        if (!gemm_rows_ok(m, w, act_packed))
            return set_error(MRI_ERR_INVALID_ARGUMENT, "gemm: rows not usable for this plan");
        if (pl.kind == GemmKind::T128x64)
            st = launch<128, 64, 4, 1, 4, 8, true>(act_packed, m, sa_ptr, sa_stride, sa_value, w,
                                                   out, acc_out, s, pl.ks, ws);
        else if (pl.kind == GemmKind::T128x128)
            st = launch<128, 128, 2, 2, 4, 8, true>(act_packed, m, sa_ptr, sa_stride, sa_value, w,
                                                    out, acc_out, s, pl.ks, ws);
        else
            st = launch<128, 192, 2, 2, 3, 8, true>(act_packed, m, sa_ptr, sa_stride, sa_value, w,
                                                    out, acc_out, s);
        if (st) return st;
        MRI_LAUNCHED("k_gemm_int8");
        return MRI_OK;
    }
    switch (pl.kind) {
        case GemmKind::SK256:
            return launch_sk<4>(act_packed, m, sa_ptr, sa_stride, sa_value, w, out, acc_out, ws,
                                pl.sk, s);
        case GemmKind::SK128:
            return launch_sk<2>(act_packed, m, sa_ptr, sa_stride, sa_value, w, out, acc_out, ws,
                                pl.sk, s);
        case GemmKind::T128x64:
            st = launch<128, 64, 4, 1, 8, 8>(act_packed, m, sa_ptr, sa_stride, sa_value, w, out,
                                             acc_out, s, pl.ks, ws);
            break;
        case GemmKind::T128x128:
            st = launch<128, 128, 2, 2, 8, 8>(act_packed, m, sa_ptr, sa_stride, sa_value, w, out,
                                              acc_out, s, pl.ks, ws);
            break;
        case GemmKind::T128x192:
            st = launch<128, 192, 2, 2, 4, 8>(act_packed, m, sa_ptr, sa_stride, sa_value, w, out,
                                              acc_out, s);
            break;
        default:
            st = launch<256, 128, 4, 2, 4, 8>(act_packed, m, sa_ptr, sa_stride, sa_value, w, out,
                                              acc_out, s);
            break;
    }
    if (st) return st;
    MRI_LAUNCHED("k_gemm_int8");
    return MRI_OK;
}

}  // namespace mri
