// gemv.hip — decode GEMV (M <= 4) on CDNA4 MFMA, streaming the weights
// through a per-wave ring of loads that is kept continuously in flight.
//
// Work decomposition: one workgroup of S waves owns one tile of 16 output
// channels; wave w streams a contiguous segment of the tile's 1 KiB weight
// chunks (whole multiples of 4 chunks).  S is chosen on the host so that
// n_tiles * S waves (about 2-3 per SIMD) are all resident at once.
//
// Ring: each wave keeps D chunk loads outstanding.  Slot s of the ring holds
// the segment's chunks i = s (mod D); the loop body is unrolled by D so every
// slot is a fixed register range, and after chunk i is consumed the load of
// chunk i + D is issued into the same slot.  The scale loads of Q8_0 ride
// the same ring (one 16-byte load per 4 chunks).  The int8 activations are
// staged in LDS once per workgroup and read just in time (a 4-deep ring).
//
//  * Per-channel INT8: v_mfma_i32_16x16x64_i8 accumulates exact int32 sums;
//    the S partial accumulators are added through LDS in wave order and
//    wave 0 applies ((f32)acc * s_a) * s_w (int8.rs:93).
//  * Q8_0: one v_mfma_i32_16x16x32_i8 per 32-element block gives the exact
//    block dot; t_b = ((f32)dot_b * s_a) * d_b (q8_direct.rs:281).  The
//    reference adds the t_b in block order.  Wave 0 folds the terms of its
//    own (first) segment in registers as it goes; waves 1..S-1 store theirs
//    to LDS; after one barrier wave 0 continues the fold over the later
//    segments in block order.  The f32 result is bit-identical to the
//    sequential reference.
//  * Fused prologue (one f32 row, the decode case): the S waves split the
//    activation read, reduce max|x| through LDS, quantize (symmetric.rs:42-57;
//    per row and per tensor coincide for one row) and write the int8 row to
//    LDS in the weight chunk order.  The activation loads are issued before
//    the ring's first D weight loads, so the prologue overlaps the weight
//    stream.  Other calls copy pre-quantized rows to LDS instead.
#include <type_traits>

#include "common.hpp"

namespace mri {
namespace {

typedef int v4i __attribute__((ext_vector_type(4)));

constexpr int kWave = 64;
constexpr int kD = 16;        // ring depth (chunks in flight per wave)
constexpr int kDA = 4;        // activation (LDS) ring depth
constexpr int kMaxM = 4;
constexpr size_t kMaxLds = 64 * 1024;

__device__ inline long lo8(const v4i &v) {
    return (long)(((unsigned long)(unsigned)v.y << 32) | (unsigned)v.x);
}
__device__ inline long hi8(const v4i &v) {
    return (long)(((unsigned long)(unsigned)v.w << 32) | (unsigned)v.z);
}

__device__ inline float wave_max(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o));
    return v;
}

__device__ inline int round_clamp_i8(float y) {
    float r = roundf(y);              // ties away from zero, like f32::round
    if (r != r) return 0;             // `NaN as i8` == 0
    r = fminf(fmaxf(r, -127.0f), 127.0f);
    return (int)r;
}

// Activation source of a launch: f32 rows quantized in the kernel (x != 0)
// or int8 rows of pitch kp already quantized (act != 0).
struct ActIn {
    const float *x;      // [M][K] f32, 16-byte aligned, K % 4 == 0
    const int8_t *act;   // [M][kp] int8 (Q8_0: chunk-permuted), 16-byte aligned
    int K;
    int8_t *act_q_out;   // optional plain [M*K] int8 (INT8 fused path)
    float *scale_out;    // optional: INT8 [1], Q8_0 [M] (fused path)
};

// Activation staging is split in two so that its global loads can be issued
// before the weight ring: loads return in issue order, and activation loads
// queued behind a full ring would stall the prologue for a whole HBM round
// trip.  Each thread holds up to kXR 16-byte pieces of the activations.
constexpr int kXR = 8;

// f32 activation row (M = 1): piece e of thread t is float4 j = t + S*64*e.
template <int S>
__device__ inline void load_x(const ActIn &in, v4i (&xr)[kXR]) {
    const int K4 = in.K / 4;
    const v4i *x4 = reinterpret_cast<const v4i *>(in.x);
    // unconditional loads (index clamped, uses are guarded): a conditional
    // load would make the compiler serialize on the register's previous value
#pragma unroll
    for (int e = 0; e < kXR; ++e) xr[e] = x4[min((int)threadIdx.x + S * kWave * e, K4 - 1)];
}

// quantize_symmetric (symmetric.rs:42-57) of the single row held in xr, into
// LDS (chunk-permuted when perm).  red: S floats of LDS.  Per-row and
// per-tensor scaling coincide for one row.
template <int S>
__device__ void quantize_x(const ActIn &in, bool perm, const v4i (&xr)[kXR], int8_t *s_act,
                           float *red, float &scale, bool writer) {
    const int t = threadIdx.x, w = t >> 6;
    const int K4 = in.K / 4;
    float mx = 0.0f;
#pragma unroll
    for (int e = 0; e < kXR; ++e) {
        if (t + S * kWave * e < K4) {
            const float4 v = __builtin_bit_cast(float4, xr[e]);
            mx = fmaxf(mx, fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w))));
        }
    }
    mx = wave_max(mx);
    if ((t & 63) == 0) red[w] = mx;
    __syncthreads();
    mx = 0.0f;
#pragma unroll
    for (int s = 0; s < S; ++s) mx = fmaxf(mx, red[s]);
    scale = mx == 0.0f ? 1.0f : __fdiv_rn(mx, 127.0f);
    const float inv = __fdiv_rn(1.0f, scale);
#pragma unroll
    for (int e = 0; e < kXR; ++e) {
        const int j = t + S * kWave * e;
        if (j < K4) {
            const float4 v = __builtin_bit_cast(float4, xr[e]);
            const int q0 = round_clamp_i8(v.x * inv);
            const int q1 = round_clamp_i8(v.y * inv);
            const int q2 = round_clamp_i8(v.z * inv);
            const int q3 = round_clamp_i8(v.w * inv);
            const int kk = 4 * j;
            const int pos = perm ? (kk & ~63) + q8_perm(kk & 63) : kk;
            const int packed =
                (q0 & 255) | ((q1 & 255) << 8) | ((q2 & 255) << 16) | (q3 << 24);
            *reinterpret_cast<int *>(s_act + pos) = packed;
            if (writer && in.act_q_out) {
                int8_t *o = in.act_q_out + kk;
                o[0] = (int8_t)q0;
                o[1] = (int8_t)q1;
                o[2] = (int8_t)q2;
                o[3] = (int8_t)q3;
            }
        }
    }
    if (writer && t == 0 && in.scale_out) in.scale_out[0] = scale;
    __syncthreads();
}

// Pre-quantized rows [M][kp]: piece e of thread t is v4i index t + S*64*e.
template <int S>
__device__ inline void load_act(const int8_t *act, int M, int kp, v4i (&xr)[kXR]) {
    const int n16 = M * kp / 16;
    const v4i *src = reinterpret_cast<const v4i *>(act);
#pragma unroll
    for (int e = 0; e < kXR; ++e) xr[e] = src[min((int)threadIdx.x + S * kWave * e, n16 - 1)];
}

template <int S>
__device__ inline void store_act(int M, int kp, const v4i (&xr)[kXR], int8_t *s_act) {
    const int n16 = M * kp / 16;
    v4i *dst = reinterpret_cast<v4i *>(s_act);
#pragma unroll
    for (int e = 0; e < kXR; ++e) {
        const int i = threadIdx.x + S * kWave * e;
        if (i < n16) dst[i] = xr[e];
    }
    __syncthreads();
}

// Whether the activations of a launch fit the per-thread register staging.
__host__ __device__ inline bool act_fits(bool fused, int m, int k, int kp, int s) {
    const int threads = s * kWave;
    if (fused) return m == 1 && (k / 4 + threads - 1) / threads <= kXR;
    return (m * kp / 16 + threads - 1) / threads <= kXR;
}

// Chunks per wave segment: a whole number of 4-chunk scale groups.
__host__ __device__ inline int seg_chunks(int P, int S) {
    return ((P + S - 1) / S + 3) & ~3;
}

// ---------------------------------------------------------------------------
// Per-channel INT8.
// ---------------------------------------------------------------------------
template <int NI, int S, bool FUSED>
__global__ __launch_bounds__(S * kWave, 3) void k_gemv_int8(
    ActIn in, int M, int kp, const float *__restrict__ sa_ptr, int sa_stride,
    float sa_value, const v4i *__restrict__ tiles, const float *__restrict__ wscales,
    int N, int P, float *__restrict__ out, int32_t *__restrict__ acc_out) {
    extern __shared__ v4i s_lds[];
    const int T = blockIdx.x;
    // wave index as a scalar: segment bounds and loop guards stay uniform, so
    // no MFMA ever sits under a partial EXEC mask.
    const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int l = threadIdx.x & 63;
    const int r = l & 15, g = l >> 4;
    const int per = seg_chunks(P, S);
    const int c0 = min(w * per, P), c1 = min(c0 + per, P);
    const int nc = c1 - c0;
    const int last = max(c1 - 1, 0);
    const v4i *wp = tiles + (size_t)T * P * kWave + l;

    // LDS: [act M*kp][red S*4 floats][partials (S-1)*64 v4i]
    int8_t *s_act = reinterpret_cast<int8_t *>(s_lds);
    float *red = reinterpret_cast<float *>(s_act + (size_t)M * kp);
    v4i *part = reinterpret_cast<v4i *>(red + S * kMaxM);

    const bool aval = r < M;
    const v4i *ap = reinterpret_cast<const v4i *>(s_act + (size_t)(aval ? r : 0) * kp) + g;
    const v4i zero = {0, 0, 0, 0};
    v4i acc = zero;
    v4i wr[kD];
    v4i ar[kDA];

    // Every global load below is unconditional (indices clamped to the
    // segment): a load inside a branch makes the compiler's wait counts
    // conservative, which would drain the whole ring at the first use.
    v4i xr[kXR];
    if constexpr (FUSED) load_x<S>(in, xr);
    else load_act<S>(in.act, M, kp, xr);
#pragma unroll
    for (int s = 0; s < kD; ++s)
        wr[s] = __builtin_nontemporal_load(wp + (size_t)min(c0 + s, last) * kWave);
    if constexpr (FUSED) {
        quantize_x<S>(in, false, xr, s_act, red, sa_value, T == 0);
        sa_ptr = nullptr;
    } else {
        store_act<S>(M, kp, xr, s_act);
    }
#pragma unroll
    for (int s = 0; s < kDA; ++s) ar[s] = ap[(size_t)min(c0 + s, last) * 4];

    auto step = [&](int s, int i) __attribute__((always_inline)) {
        __builtin_amdgcn_sched_barrier(0);
        const v4i a = aval ? ar[s % kDA] : zero;
        acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(a, wr[s], acc, 0, 0, 0);
        __builtin_amdgcn_sched_barrier(0);
        ar[s % kDA] = ap[(size_t)min(c0 + i + kDA, last) * 4];
    };
    // full laps: consume chunk i from slot s, then load chunk i + D into it
    const int laps = (nc + kD - 1) / kD;
    for (int lap = 0; lap + 1 < laps; ++lap) {
#pragma unroll
        for (int s = 0; s < kD; ++s) {
            const int i = lap * kD + s;
            step(s, i);
            wr[s] = __builtin_nontemporal_load(wp + (size_t)min(c0 + i + kD, last) * kWave);
        }
    }
    // final lap: no more loads
    if (laps > 0) {
#pragma unroll
        for (int s = 0; s < kD; ++s) {
            const int i = (laps - 1) * kD + s;
            if (i < nc) step(s, i);
        }
    }

    // exact int32 reduction over the S segments, in wave order
    if (w > 0) part[(w - 1) * kWave + l] = acc;
    __syncthreads();
    if (w > 0) return;
#pragma unroll
    for (int s = 1; s < S; ++s) acc += part[(s - 1) * kWave + l];

    const int n = T * 16 + r;
    if (n >= N || g != 0) return;
    const float sw = wscales[n];
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

// ---------------------------------------------------------------------------
// Q8_0.  MFMA output rows m = 4*(l/16) + i: with M <= 4 the valid rows are
// the NI registers of lane group 0 (lanes 0..15, one output channel each).
// ---------------------------------------------------------------------------
template <int NI, int S, bool FUSED>
__global__ __launch_bounds__(S * kWave, 3) void k_gemv_q8_0(
    ActIn in, int M, int kp, const float *__restrict__ sa_rows,
    const v4i *__restrict__ tiles, const v4i *__restrict__ qscales, int N, int P,
    int Q, int nb, float *__restrict__ out, int32_t *__restrict__ block_dots) {
    static_assert(kD % 4 == 0, "the scale ring holds whole groups");
    extern __shared__ v4i s_lds[];
    const int T = blockIdx.x;
    const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int l = threadIdx.x & 63;
    const int r = l & 15, g = l >> 4;
    const int Pe = (nb + 1) / 2;          // chunks holding real blocks
    const int per = seg_chunks(P, S);
    const int c1 = min(min(w * per, P) + per, Pe);
    const int c0 = min(min(w * per, P), c1);
    const int nc = c1 - c0;
    const int last = max(c1 - 1, 0);
    const int seg_blocks = 2 * per;
    const v4i *wp = tiles + (size_t)T * P * kWave + l;
    const v4i *sp = qscales + (size_t)T * Q * 16 + r;

    // LDS: [act M*kp][red S*4 floats][terms (S-1) x seg_blocks x NI x 16 floats]
    int8_t *s_act = reinterpret_cast<int8_t *>(s_lds);
    float *red = reinterpret_cast<float *>(s_act + (size_t)M * kp);
    float *terms = red + S * kMaxM;
    float *tw = terms + (size_t)(w > 0 ? w - 1 : 0) * seg_blocks * NI * 16;

    const bool aval = r < M;
    const v4i *ap = reinterpret_cast<const v4i *>(s_act + (size_t)(aval ? r : 0) * kp) + g;
    const v4i zero = {0, 0, 0, 0};
    const int n = T * 16 + r;
    v4i wr[kD];
    v4i sr[kD / 4];
    v4i ar[kDA];

    // ring slot s holds chunk c0 + i with i = s (mod D); the scale slot s/4
    // holds the group of chunks c0 + (i & ~3) .. +3 (c0 is a multiple of 4)
    // Every global load below is unconditional (indices clamped to the
    // segment); see the INT8 kernel.
    v4i xr[kXR];
    if constexpr (FUSED) load_x<S>(in, xr);
    else load_act<S>(in.act, M, kp, xr);
#pragma unroll
    for (int s = 0; s < kD; ++s) {
        const int p = min(c0 + s, last);
        wr[s] = __builtin_nontemporal_load(wp + (size_t)p * kWave);
        if (s % 4 == 0) sr[s / 4] = sp[(size_t)(p / 4) * 16];
    }
    float sa[NI];
    if constexpr (FUSED) {
        static_assert(!FUSED || NI == 1, "the fused prologue quantizes one row");
        quantize_x<S>(in, true, xr, s_act, red, sa[0], T == 0);
    } else {
#pragma unroll
        for (int i = 0; i < NI; ++i) sa[i] = sa_rows[i];
        store_act<S>(M, kp, xr, s_act);
    }
#pragma unroll
    for (int s = 0; s < kDA; ++s) ar[s] = ap[(size_t)min(c0 + s, last) * 4];

    float fs[NI];
#pragma unroll
    for (int i = 0; i < NI; ++i) fs[i] = 0.0f;

    // Epilogue of chunk i (ring slot s): the two block terms, folded in order
    // (wave 0) or stored for the later fold (waves 1..S-1).
    auto epilogue = [&](const v4i (&dots)[2], int s, int i) __attribute__((always_inline)) {
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const int bl = 2 * i + h;            // block within the segment
            const int b = 2 * c0 + bl;
            if (b < nb) {
                const int j = (2 * (s % 4) + h) & 7;
                const unsigned word = (unsigned)sr[s / 4][j >> 1];
                const float d = f16_bits_to_f32((j & 1) ? (word >> 16) : (word & 0xFFFFu));
                if (g == 0) {
#pragma unroll
                    for (int k = 0; k < NI; ++k) {
                        float t = (float)dots[h][k] * sa[k];
                        t = t * d;
                        if (w == 0) fs[k] = fs[k] + t;
                        else tw[(bl * NI + k) * 16 + r] = t;
                    }
                    if (block_dots && n < N) {
#pragma unroll
                        for (int k = 0; k < NI; ++k)
                            block_dots[((size_t)k * N + n) * nb + b] = dots[h][k];
                    }
                }
            }
        }
    };

    v4i dots[2][2];
    // One chunk: its two block MFMAs, then the previous chunk's epilogue
    // (which overlaps them).  LOADS: refill the weight slot with chunk i + D
    // and, after a group's fourth chunk, its scale slot with the group one
    // lap later.
    auto step = [&](int s, int i, auto loads) __attribute__((always_inline)) {
        __builtin_amdgcn_sched_barrier(0);
        const v4i a = aval ? ar[s % kDA] : zero;
        dots[s & 1][0] = __builtin_amdgcn_mfma_i32_16x16x32_i8(lo8(a), lo8(wr[s]), zero, 0, 0, 0);
        dots[s & 1][1] = __builtin_amdgcn_mfma_i32_16x16x32_i8(hi8(a), hi8(wr[s]), zero, 0, 0, 0);
        __builtin_amdgcn_sched_barrier(0);
        ar[s % kDA] = ap[(size_t)min(c0 + i + kDA, last) * 4];
        if constexpr (decltype(loads)::value)
            wr[s] = __builtin_nontemporal_load(wp + (size_t)min(c0 + i + kD, last) * kWave);
        if (i > 0) {
            const int sp_ = (s + kD - 1) % kD;
            epilogue(dots[(s + 1) & 1], sp_, i - 1);
            if constexpr (decltype(loads)::value) {
                if (s % 4 == 0)
                    sr[sp_ / 4] = sp[(size_t)(min(c0 + i - 4 + kD, last) / 4) * 16];
            }
        }
        __builtin_amdgcn_sched_barrier(0);
    };
    const int laps = (nc + kD - 1) / kD;
    for (int lap = 0; lap + 1 < laps; ++lap) {
#pragma unroll
        for (int s = 0; s < kD; ++s) step(s, lap * kD + s, std::true_type{});
    }
    if (laps > 0) {
#pragma unroll
        for (int s = 0; s < kD; ++s) {
            const int i = (laps - 1) * kD + s;
            if (i < nc) {
                step(s, i, std::false_type{});
                // the segment's last chunk has no next step to lag into
                if (i == nc - 1) epilogue(dots[s & 1], s, i);
            }
        }
    }

    __syncthreads();
    if (w != 0 || g != 0) return;
    // continue the block-ordered fold over the later segments
    for (int s = 1; s < S; ++s) {
        const int e1 = min(min(s * per, P) + per, Pe);
        const int e0 = min(min(s * per, P), e1);
        const int cnt = min(2 * (e1 - e0), nb - 2 * e0);
        const float *ts = terms + (size_t)(s - 1) * seg_blocks * NI * 16 + r;
        for (int bl = 0; bl < cnt; ++bl) {
#pragma unroll
            for (int k = 0; k < NI; ++k) fs[k] = fs[k] + ts[(bl * NI + k) * 16];
        }
    }
    if (n >= N) return;
#pragma unroll
    for (int k = 0; k < NI; ++k)
        if (k < M) out[(size_t)k * N + n] = fs[k];
}

// Waves per tile: about two waves per SIMD over the launch, at least two
// scale groups (8 chunks) per wave.
int pick_s(size_t n_tiles, size_t P) {
    int s = 1;
    while (s < 8 && n_tiles * (size_t)(2 * s) <= 3072 && P >= (size_t)(16 * s)) s *= 2;
    return s;
}

size_t lds_i8(int s, size_t m, size_t kp) {
    return m * kp + (size_t)s * kMaxM * 4 + (size_t)(s - 1) * kWave * 16;
}

size_t lds_q8(int s, size_t m, size_t kp) {
    const size_t seg_blocks = 2 * (size_t)seg_chunks((int)(kp / kChunkK), s);
    return m * kp + (size_t)s * kMaxM * 4 + (size_t)(s - 1) * seg_blocks * m * 16 * 4;
}

// Largest S <= pick_s that fits LDS; then more waves if the activations
// need more threads to fit the register staging.  0 = unsupported.
int fit_s(bool q8, bool fused, size_t n_tiles, size_t m, size_t k, size_t kp) {
    auto lds = [&](int s) { return q8 ? lds_q8(s, m, kp) : lds_i8(s, m, kp); };
    int s = pick_s(n_tiles, kp / kChunkK);
    while (s < 8 && !act_fits(fused, (int)m, (int)k, (int)kp, s)) s *= 2;
    while (s > 1 && lds(s) > kMaxLds) s /= 2;
    if (lds(s) > kMaxLds || !act_fits(fused, (int)m, (int)k, (int)kp, s)) return 0;
    return s;
}

template <int NI, int S, bool FUSED>
void launch_i8(ActIn in, size_t m, const float *sa_ptr, int sa_stride, float sa_value,
               const QMatrixDev &w, float *out, int32_t *acc_out, hipStream_t st) {
    hipLaunchKernelGGL((k_gemv_int8<NI, S, FUSED>), dim3((unsigned)w.n_tiles),
                       dim3(S * kWave), lds_i8(S, m, w.kp), st, in, (int)m, (int)w.kp,
                       sa_ptr, sa_stride, sa_value, reinterpret_cast<const v4i *>(w.tiles),
                       w.scales, (int)w.n_out, (int)(w.kp / kChunkK), out, acc_out);
}

template <int NI, int S, bool FUSED>
void launch_q8(ActIn in, size_t m, const float *sa_rows, const Q8MatrixDev &w,
               float *out, int32_t *block_dots, hipStream_t st) {
    hipLaunchKernelGGL((k_gemv_q8_0<NI, S, FUSED>), dim3((unsigned)w.n_tiles),
                       dim3(S * kWave), lds_q8(S, m, w.kp), st, in, (int)m, (int)w.kp,
                       sa_rows, reinterpret_cast<const v4i *>(w.tiles),
                       reinterpret_cast<const v4i *>(w.scales), (int)w.n_out,
                       (int)(w.kp / kChunkK), (int)(w.kp / (kQK * kQ8ScaleGroup)),
                       (int)w.n_blocks, out, block_dots);
}

template <int NI, bool FUSED>
void dispatch_i8(int s, ActIn in, size_t m, const float *sa_ptr, int sa_stride,
                 float sa_value, const QMatrixDev &w, float *out, int32_t *acc_out,
                 hipStream_t st) {
    switch (s) {
    case 1: launch_i8<NI, 1, FUSED>(in, m, sa_ptr, sa_stride, sa_value, w, out, acc_out, st); break;
    case 2: launch_i8<NI, 2, FUSED>(in, m, sa_ptr, sa_stride, sa_value, w, out, acc_out, st); break;
    case 4: launch_i8<NI, 4, FUSED>(in, m, sa_ptr, sa_stride, sa_value, w, out, acc_out, st); break;
    default: launch_i8<NI, 8, FUSED>(in, m, sa_ptr, sa_stride, sa_value, w, out, acc_out, st); break;
    }
}

template <int NI, bool FUSED>
void dispatch_q8(int s, ActIn in, size_t m, const float *sa_rows, const Q8MatrixDev &w,
                 float *out, int32_t *block_dots, hipStream_t st) {
    switch (s) {
    case 1: launch_q8<NI, 1, FUSED>(in, m, sa_rows, w, out, block_dots, st); break;
    case 2: launch_q8<NI, 2, FUSED>(in, m, sa_rows, w, out, block_dots, st); break;
    case 4: launch_q8<NI, 4, FUSED>(in, m, sa_rows, w, out, block_dots, st); break;
    default: launch_q8<NI, 8, FUSED>(in, m, sa_rows, w, out, block_dots, st); break;
    }
}

}  // namespace

bool gemv_int8_supported(bool fused, size_t m, size_t n_tiles, size_t k, size_t kp) {
    return m >= 1 && m <= (size_t)kMaxM && fit_s(false, fused, n_tiles, m, k, kp) > 0;
}

bool gemv_q8_supported(bool fused, size_t m, size_t n_tiles, size_t k, size_t kp) {
    return m >= 1 && m <= (size_t)kMaxM && fit_s(true, fused, n_tiles, m, k, kp) > 0;
}

bool gemv_fusable(size_t m, size_t k, const float *x) {
    return m == 1 && k % 4 == 0 && x &&
           (reinterpret_cast<uintptr_t>(x) & 15) == 0;
}

mri_status launch_gemv_int8(const float *x, const int8_t *act, size_t m,
                            const float *sa_ptr, int sa_stride, float sa_value,
                            const QMatrixDev &w, float *out, int8_t *act_q_out,
                            float *scale_out, int32_t *acc_out, hipStream_t st) {
    if (w.n_tiles == 0 || m == 0) return MRI_OK;
    const int s = fit_s(false, x != nullptr, w.n_tiles, m, w.k_in, w.kp);
    if (s == 0) return set_error(MRI_ERR_INVALID_ARGUMENT, "gemv: shape not supported");
    const ActIn in{x, act, (int)w.k_in, act_q_out, scale_out};
    if (x) {
        dispatch_i8<1, true>(s, in, m, nullptr, 0, 0.0f, w, out, acc_out, st);
    } else {
        if (m == 1) dispatch_i8<1, false>(s, in, m, sa_ptr, sa_stride, sa_value, w, out, acc_out, st);
        else if (m == 2) dispatch_i8<2, false>(s, in, m, sa_ptr, sa_stride, sa_value, w, out, acc_out, st);
        else dispatch_i8<4, false>(s, in, m, sa_ptr, sa_stride, sa_value, w, out, acc_out, st);
    }
    MRI_LAUNCHED("k_gemv_int8");
    return MRI_OK;
}

mri_status launch_gemv_q8_0(const float *x, const int8_t *act, size_t m,
                            const float *sa_rows, const Q8MatrixDev &w, float *out,
                            int32_t *block_dots, float *scales_out, hipStream_t st) {
    if (w.n_tiles == 0 || m == 0) return MRI_OK;
    const int s = fit_s(true, x != nullptr, w.n_tiles, m, w.k_in, w.kp);
    if (s == 0) return set_error(MRI_ERR_INVALID_ARGUMENT, "gemv: shape not supported");
    const ActIn in{x, act, (int)w.k_in, nullptr, scales_out};
    if (x) {
        dispatch_q8<1, true>(s, in, m, nullptr, w, out, block_dots, st);
    } else {
        if (m == 1) dispatch_q8<1, false>(s, in, m, sa_rows, w, out, block_dots, st);
        else if (m == 2) dispatch_q8<2, false>(s, in, m, sa_rows, w, out, block_dots, st);
        else if (m == 3) dispatch_q8<3, false>(s, in, m, sa_rows, w, out, block_dots, st);
        else dispatch_q8<4, false>(s, in, m, sa_rows, w, out, block_dots, st);
    }
    MRI_LAUNCHED("k_gemv_q8_0");
    return MRI_OK;
}

}  // namespace mri
