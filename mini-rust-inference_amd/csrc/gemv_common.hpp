// gemv_common.hpp — shared pieces of the decode GEMV kernels (M <= 4) of
// gemv_int8.hip and gemv_q8.hip: a single sweep over the weight stream with
// a ring of loads in flight per wave.
//
// Work decomposition: a workgroup holds TPW tiles of 16 output channels with
// S waves each; a tile's K chunks are split over its S waves (INT8: evenly;
// Q8_0: lap blocks of 4 chunks dealt out round-robin).  INT8 weights are
// slab-major (chunk (p, T) at (p * n_tiles + T) KiB), so the waves of all
// tiles that run together read one contiguous, moving window; Q8_0 lap
// blocks are tile-major with the scales inside, so each wave reads whole
// 4 KiB runs and the scales come from the same DRAM pages as the quants.
//
// Ring: each wave keeps D chunk loads in flight.  Slot s holds the chunks
// i == s (mod D) of its segment; the loop body is unrolled by D, so every
// slot is a fixed register range, and after chunk i is consumed the load of
// chunk i + D is issued into the same slot.  The loop contains no other
// global memory instruction (the Q8_0 scale loads ride the same ring, one
// 16-byte load per 4 chunks), so the wait before each MFMA leaves D - 1
// loads outstanding.  Optional int32 debug outputs are compiled into a
// separate kernel instance so that the timed kernel has no stores in the
// loop.
//
//  * Fused prologue (one f32 row, the decode case): the S waves split the
//    activation read, reduce max|x| through LDS, quantize (symmetric.rs:42-57;
//    per row and per tensor coincide for one row) and write the int8 row to
//    LDS in the weight chunk order.  The activation loads are issued just
//    before the ring's first weight loads, so the prologue overlaps the
//    weight stream.  Other calls copy pre-quantized rows to LDS instead.
#pragma once

#include <cstdlib>
#include <type_traits>
#include <utility>

#include "common.hpp"

namespace mri {
namespace gemv {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v2i __attribute__((ext_vector_type(2)));

constexpr int kWave = 64;
constexpr int kMaxM = 4;
// An int8 MFMA whose accumulator starts from kDotBias, the bits of
// kDotBiasF = 1.5 * 2^23, leaves the bits of the f32 number kDotBiasF + dot
// for any |dot| < 2^22 (the f32 spacing in [2^23, 2^24) is 1): subtracting
// kDotBiasF gives (f32)dot exactly, at full rate, where v_cvt_f32_i32 issues
// at half rate.  A Q8_0 block dot is at most 32 * 128 * 127 < 2^22.
constexpr int kDotBias = 0x4B400000;
constexpr float kDotBiasF = 12582912.0f;
constexpr size_t kMaxLds = 64 * 1024;

inline size_t ceil_div(size_t a, size_t b) { return (a + b - 1) / b; }

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

// The same map in six instructions: round(y), ties away from zero, is
// trunc(y + copysign(0.5 - 2^-25, y)) for every f32 that is not NaN (the
// sum rounds up to the next integer exactly when the fraction is >= 1/2;
// checked over all 2^32 bit patterns); v_cvt_i32_f32 saturates and maps NaN
// to 0, so the clamp to [-127, 127] is an integer med3.
__device__ inline int cvt_i32_sat(float r) {
    int v;
    asm("v_cvt_i32_f32 %0, %1" : "=v"(v) : "v"(r));
    return v;
}
__device__ inline int quant_i8(float y) {
    const float r = __builtin_truncf(y + __builtin_copysignf(0.49999997f, y));
    return min(max(cvt_i32_sat(r), -127), 127);
}
// Four values times inv, quantized as quant_i8 and packed little-endian.
__device__ inline int quant4_packed(float4 v, float inv) {
    const unsigned q0 = (unsigned)quant_i8(v.x * inv), q1 = (unsigned)quant_i8(v.y * inv);
    const unsigned q2 = (unsigned)quant_i8(v.z * inv), q3 = (unsigned)quant_i8(v.w * inv);
    // v_perm_b32: selector bytes 0-3 pick bytes of the second operand, 4-7
    // of the first, 0x0c gives zero
    const unsigned lo = __builtin_amdgcn_perm(q1, q0, 0x0c0c0400u);
    const unsigned hi = __builtin_amdgcn_perm(q3, q2, 0x04000c0cu);
    return (int)(lo | hi);
}

// Masked row layout of a one-row Q8_0 MFMA operand (the kernels' chained
// form): lap q of the row is a 512-byte area of 32 entries of 16 bytes;
// entry (2s + h) + 8g holds the 8 bytes of lane group g of block 2s + h of
// the lap's chunk s (elements 8g .. 8g + 7 of that block) in bytes 8h .. 8h
// + 7 and zeros in the other half, so that lane (r = 2s + h, g) of the
// chunk's MFMA reads row r of the A operand in one 16-byte load.
// Byte offset of the data word of elements kk .. kk + 3 (kk % 4 == 0); the
// zero word that goes with it is at offset ^ 8.
__device__ inline int masked_off(int kk) {
    const int e = kk & 63, s = (kk >> 6) & 3, h = e >> 5, g = (e >> 3) & 3;
    return (kk >> 8) * 512 + 16 * (2 * s + h + 8 * g) + 8 * h + (e & 4);
}

// Calls f(std::integral_constant<int, I>) for I = 0 .. N-1 (compile-time
// ring slot indices).
template <typename F, int... I>
__device__ inline void static_for_impl(F &&f, std::integer_sequence<int, I...>) {
    (f(std::integral_constant<int, I>{}), ...);
}
template <int N, typename F>
__device__ inline void static_for(F &&f) {
    static_for_impl(f, std::make_integer_sequence<int, N>{});
}

// Even split of `units` over `parts`: part w gets [lo, hi).
__host__ __device__ inline int split_lo(int units, int parts, int w) {
    return (int)((long)units * w / parts);
}

// Activation source of a launch: f32 rows quantized in the kernel (x != 0)
// or int8 rows of pitch kp already quantized (act != 0).  Kernel instances
// with OPS take the row operations (RowOps, in common.hpp) as well: with
// norm_w, the fused row is RMS-normalized before it is quantized,
// w * (x * rms_inv) with rms_inv = 1 / sqrt(mean(x^2) + eps)
// (ops/norm/rmsnorm.rs:100-114); x_out receives a copy of the row as read;
// accum: the kernel adds its result to out instead of storing it (the
// residual add, forward_int8.rs:100-121).
struct ActIn {
    const float *x;      // [1][K] f32, 16-byte aligned, K % 4 == 0
    const int8_t *act;   // [M][kp] int8 (Q8_0: chunk-permuted), 16-byte aligned
    int K;
    int8_t *act_q_out;   // optional plain [K] int8 (INT8 fused path)
    float *scale_out;    // optional [1] (fused path)
    const float *norm_w = nullptr;  // optional [K], 16-byte aligned (fused path)
    float eps = 0.0f;
    float *x_out = nullptr;         // optional [K], 16-byte aligned (fused path)
    const float *up = nullptr;      // optional [K]: x is a SwiGLU gate row (fused path)
    unsigned long long *arg_keys = nullptr;  // optional: per-tile argmax keys (RowOps)
    int accum = 0;
    const float *rope_cos = nullptr, *rope_sin = nullptr;
    int rope_n = 0, hd = 2, seg1 = INT_MAX, seg2 = INT_MAX, silu_n = 0;
    float *out1 = nullptr, *out2 = nullptr;
    const unsigned long long *in_keys = nullptr;  // x is a table row picked by keys (RowOps)
    int n_in_keys = 0;
    uint32_t *tok_out = nullptr;

    ActIn(const float *x_, const int8_t *act_, int k, int8_t *aq, float *so, const RowOps &o)
        : x(x_), act(act_), K(k), act_q_out(aq), scale_out(so), norm_w(o.norm_w), eps(o.eps),
          x_out(o.x_out), up(o.up), arg_keys(o.arg_keys), accum(o.accum ? 1 : 0), rope_cos(o.rope_cos), rope_sin(o.rope_sin),
          rope_n(o.rope_n), hd(o.hd), seg1(o.seg1), seg2(o.seg2), silu_n(o.silu_n),
          out1(o.out1), out2(o.out2),
          in_keys(o.in_keys), n_in_keys(o.n_in_keys), tok_out(o.tok_out) {}
};

// The fused row of a decode step whose token is still on the device as the
// previous step's argmax keys (ActIn::in_keys): the workgroup reduces the
// keys (each thread a strided share, then the wave, then the NW waves
// through LDS), takes the index of the largest (0 when every key is 0, as
// launch_argmax_keys does), stores it to tok_out from workgroup 0 and
// returns that row of the table in.x.  Without keys, in.x itself.  Called
// by every thread of the workgroup (it has a barrier).
template <int NW>
__device__ inline const float *row_of_keys(const ActIn &in) {
    if (!in.in_keys) return in.x;
    __shared__ unsigned long long s_key[NW];
    const int t = threadIdx.x;
    unsigned long long k = 0;
#pragma unroll 4
    for (int i = t; i < in.n_in_keys; i += NW * kWave) {
        const unsigned long long v = in.in_keys[i];
        k = v > k ? v : k;
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        const unsigned lo = __shfl_xor((unsigned)k, o), hi = __shfl_xor((unsigned)(k >> 32), o);
        const unsigned long long ok = ((unsigned long long)hi << 32) | lo;
        k = ok > k ? ok : k;
    }
    if ((t & 63) == 0) s_key[t >> 6] = k;
    __syncthreads();
    k = s_key[0];
#pragma unroll
    for (int w = 1; w < NW; ++w) k = s_key[w] > k ? s_key[w] : k;
    const uint32_t tok = k ? (uint32_t)k : 0u;
    if (blockIdx.x == 0 && t == 0 && in.tok_out) *in.tok_out = tok;
    return in.x + (size_t)tok * in.K;
}

// The destination of output channel n of the row operations, its old value
// (for the residual add) and its RoPE factors, loaded when the kernel
// starts, so that the epilogue waits for no load of its own (a dependent
// round trip at the end of every decode-step projection otherwise).  n is
// clamped: a lane past N loads an element it never stores.
struct RowDst {
    float *o;
    float base = 0.0f, c = 1.0f, s = 0.0f;
};
__device__ inline RowDst row_dst(const ActIn &in, float *out, int n, int N) {
    const int nc = min(n, N - 1);
    RowDst d;
    d.o = nc >= in.seg2 ? in.out2 + (nc - in.seg2)
        : nc >= in.seg1 ? in.out1 + (nc - in.seg1)
                        : out + nc;
    if (in.accum) d.base = *d.o;
    if (in.rope_n > 0) {
        const int i = (nc % in.hd) >> 1;
        d.c = in.rope_cos[i];
        d.s = in.rope_sin[i];
    }
    return d;
}

// Epilogue of the row operations for output channel n of the row with value
// v, where pv is the value of channel n ^ 1: RoPE below rope_n, as
// rope_apply computes it (out[2i] = x0*c - x1*s, out[2i+1] = x1*c + x0*s),
// or the SiLU v / (1 + exp(-v)) below silu_n, then the store by output
// segment, or the residual accumulate.
__device__ inline void row_store(const ActIn &in, const RowDst &d, int n, float v, float pv) {
    if (n < in.silu_n) v = v / (1.0f + expf(-v));
    if (n < in.rope_n) {
        const float a = v * d.c, b = pv * d.s;
        v = (n & 1) ? a + b : a - b;
    }
    *d.o = in.accum ? d.base + v : v;
}

// Greedy argmax keys in the epilogue of a one-row projection, called by the
// one wave of tile T that holds its outputs (lanes with mine set hold
// channel n's value v): the tile's largest argmax_key goes to keys[T].
__device__ inline void row_argmax_key(unsigned long long *keys, int T, float v, int n,
                                      bool mine) {
    unsigned long long key = mine ? argmax_key(v, n) : 0ull;
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        const unsigned lo = __shfl_xor((unsigned)key, o), hi = __shfl_xor((unsigned)(key >> 32), o);
        const unsigned long long ok = ((unsigned long long)hi << 32) | lo;
        key = ok > key ? ok : key;
    }
    if ((threadIdx.x & 63) == 0) keys[T] = key;
}

// Each thread stages XR 16-byte pieces of the activations in registers:
// piece e of thread t is element t + S*64*e (index clamped, use guarded).
// The loads are unconditional so that no wait count depends on a branch.
template <int S, int XR>
__device__ inline void stage_load(const v4i *src, int n16, v4i (&xr)[XR]) {
#pragma unroll
    for (int e = 0; e < XR; ++e) xr[e] = src[min((int)threadIdx.x + S * kWave * e, n16 - 1)];
}

// SwiGLU of the staged gate pieces with the up pieces staged in wn
// (ops/activation/swiglu.rs): the gate row already holds g / (1 + exp(-g))
// (stored so by the gate projection's epilogue, RowOps::silu_n), and x =
// that times u, which is how the separate SwiGLU kernels evaluate
// g / (1 + exp(-g)) * u, so the values are theirs.
template <int S, int XR>
__device__ inline void act_swiglu(const ActIn &in, v4i (&xr)[XR], const v4i (&wn)[XR]) {
    const int K4 = in.K / 4;
#pragma unroll
    for (int e = 0; e < XR; ++e) {
        if ((int)threadIdx.x + S * kWave * e < K4) {
            const float4 g = __builtin_bit_cast(float4, xr[e]);
            const float4 u = __builtin_bit_cast(float4, wn[e]);
            xr[e] = __builtin_bit_cast(v4i, float4{g.x * u.x, g.y * u.y, g.z * u.z, g.w * u.w});
        }
    }
}

// The activation prologue runs after the priming of the weight ring: the
// kernels issue the activation loads (stage_load), then the ring's first
// weight loads, then consume the activations.  Loads return in issue order,
// so act_begin waits for the activation loads alone while the weight loads
// stay in flight.  act_begin consumes the staged registers (the per-wave
// max|x| of an f32 row, or the copy of int8 rows into LDS); act_end
// finishes the quantization: block max through LDS, quantize_symmetric
// (symmetric.rs:42-57; per row and per tensor coincide for one row) of the
// row held in xr into LDS (chunk-permuted when perm).  Neither waits for
// global loads at its barriers beyond the activations'.
__device__ inline float wave_sum_f(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = v + __shfl_xor(v, o);
    return v;
}

// MASKED: the int8 rows (one row) are copied into the masked layout instead
// (piece i, lane group i % 4 of chunk i / 4, goes to its two entries).
template <int S, int XR, bool FUSED, bool OPS, bool MASKED = false>
__device__ inline void act_begin(const ActIn &in, int n16, const v4i (&xr)[XR], int8_t *s_act,
                                 float *red) {
    const int t = threadIdx.x;
    if constexpr (FUSED) {
        const int K4 = in.K / 4;
        if (OPS && in.x_out && blockIdx.x == 0) {
#pragma unroll
            for (int e = 0; e < XR; ++e)
                if (t + S * kWave * e < K4)
                    reinterpret_cast<v4i *>(in.x_out)[t + S * kWave * e] = xr[e];
        }
        if (OPS && in.norm_w) {  // sum of squares for the RMS norm
            float ss = 0.0f;
#pragma unroll
            for (int e = 0; e < XR; ++e) {
                if (t + S * kWave * e < K4) {
                    const float4 v = __builtin_bit_cast(float4, xr[e]);
                    ss = ss + v.x * v.x;
                    ss = ss + v.y * v.y;
                    ss = ss + v.z * v.z;
                    ss = ss + v.w * v.w;
                }
            }
            ss = wave_sum_f(ss);
            if ((t & 63) == 0) red[t >> 6] = ss;
        } else {
            float mx = 0.0f;
#pragma unroll
            for (int e = 0; e < XR; ++e) {
                if (t + S * kWave * e < K4) {
                    const float4 v = __builtin_bit_cast(float4, xr[e]);
                    mx = fmaxf(mx, fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)),
                                         fmaxf(fabsf(v.z), fabsf(v.w))));
                }
            }
            mx = wave_max(mx);
            if ((t & 63) == 0) red[t >> 6] = mx;
        }
    } else {
        v4i *dst = reinterpret_cast<v4i *>(s_act);
#pragma unroll
        for (int e = 0; e < XR; ++e) {
            const int i = t + S * kWave * e;
            if (i < n16) {
                if constexpr (MASKED) {
                    const int ent = (i >> 4) * 32 + 2 * ((i >> 2) & 3) + 8 * (i & 3);
                    dst[ent] = v4i{xr[e].x, xr[e].y, 0, 0};
                    dst[ent + 1] = v4i{0, 0, xr[e].z, xr[e].w};
                } else {
                    dst[i] = xr[e];
                }
            }
        }
    }
    // keep the uses above after the weight loads issued before them
    __builtin_amdgcn_sched_barrier(0);
}

// wn: the norm weight pieces staged like xr (used when in.norm_w).
// layout: kLayPlain (element kk at byte kk), kLayPerm (chunk-permuted,
// q8_perm) or kLayMasked (masked_off, with the zero word beside each data
// word).
enum : int { kLayPlain = 0, kLayPerm = 1, kLayMasked = 2 };
template <int S, int XR, bool FUSED, bool OPS>
__device__ inline void act_end(const ActIn &in, int layout, v4i (&xr)[XR], const v4i (&wn)[XR],
                               int8_t *s_act, float *red, float &scale, bool writer) {
    __syncthreads();
    if constexpr (FUSED) {
        const int t = threadIdx.x;
        const int K4 = in.K / 4;
        float mx = 0.0f;
        if (OPS && in.norm_w) {
            float ss = 0.0f;
#pragma unroll
            for (int s = 0; s < S; ++s) ss = ss + red[s];
            const float mean_sq = __fdiv_rn(ss, (float)in.K);
            const float rms_inv = __fdiv_rn(1.0f, __fsqrt_rn(mean_sq + in.eps));
#pragma unroll
            for (int e = 0; e < XR; ++e) {
                if (t + S * kWave * e < K4) {
                    const float4 v = __builtin_bit_cast(float4, xr[e]);
                    const float4 w = __builtin_bit_cast(float4, wn[e]);
                    const float4 y = {w.x * (v.x * rms_inv), w.y * (v.y * rms_inv),
                                      w.z * (v.z * rms_inv), w.w * (v.w * rms_inv)};
                    xr[e] = __builtin_bit_cast(v4i, y);
                    mx = fmaxf(mx, fmaxf(fmaxf(fabsf(y.x), fabsf(y.y)),
                                         fmaxf(fabsf(y.z), fabsf(y.w))));
                }
            }
            mx = wave_max(mx);
            if ((t & 63) == 0) red[S + (t >> 6)] = mx;
            __syncthreads();
            mx = 0.0f;
#pragma unroll
            for (int s = 0; s < S; ++s) mx = fmaxf(mx, red[S + s]);
        } else {
#pragma unroll
            for (int s = 0; s < S; ++s) mx = fmaxf(mx, red[s]);
        }
        scale = mx == 0.0f ? 1.0f : __fdiv_rn(mx, 127.0f);
        const float inv = __fdiv_rn(1.0f, scale);
#pragma unroll
        for (int e = 0; e < XR; ++e) {
            const int j = t + S * kWave * e;
            if (j < K4) {
                const float4 v = __builtin_bit_cast(float4, xr[e]);
                const int q0 = round_clamp_i8(v.x * inv);
                const int q1 = round_clamp_i8(v.y * inv);
                const int q2 = round_clamp_i8(v.z * inv);
                const int q3 = round_clamp_i8(v.w * inv);
                const int kk = 4 * j;
                const int pos = layout == kLayMasked ? masked_off(kk)
                                : layout == kLayPerm ? (kk & ~63) + q8_perm(kk & 63)
                                                     : kk;
                const int packed =
                    (q0 & 255) | ((q1 & 255) << 8) | ((q2 & 255) << 16) | (q3 << 24);
                *reinterpret_cast<int *>(s_act + pos) = packed;
                if (layout == kLayMasked) *reinterpret_cast<int *>(s_act + (pos ^ 8)) = 0;
                if (writer && in.act_q_out)
                    *reinterpret_cast<int *>(in.act_q_out + kk) = packed;
            }
        }
        if (writer && t == 0 && in.scale_out) in.scale_out[0] = scale;
        __syncthreads();
    }
}

// The end of the prologue for the lap-wise quantization (the kernels'
// LAZY instances): the same arithmetic as act_end up to the row scale, but
// the row (RMS-normalized when in.norm_w) goes to LDS as f32 (s_xf, K
// floats) instead of being quantized; returns 1 / scale.  act_begin has run.
// STAGE false: the row stays in xr only (no norm; the caller quantizes from
// its registers).
template <int S, int XR, bool OPS, bool STAGE = true>
__device__ inline float act_end_lazy(const ActIn &in, v4i (&xr)[XR], const v4i (&wn)[XR],
                                     float *s_xf, float *red, float &scale, bool writer) {
    const int t = threadIdx.x;
    const int K4 = in.K / 4;
    v4i *s_x4 = reinterpret_cast<v4i *>(s_xf);
    const bool norm = OPS && in.norm_w;
    if (STAGE && !norm) {
#pragma unroll
        for (int e = 0; e < XR; ++e)
            if (t + S * kWave * e < K4) s_x4[t + S * kWave * e] = xr[e];
    }
    __syncthreads();
    float mx = 0.0f;
    if (norm) {
        float ss = 0.0f;
#pragma unroll
        for (int s = 0; s < S; ++s) ss = ss + red[s];
        const float mean_sq = __fdiv_rn(ss, (float)in.K);
        const float rms_inv = __fdiv_rn(1.0f, __fsqrt_rn(mean_sq + in.eps));
#pragma unroll
        for (int e = 0; e < XR; ++e) {
            if (t + S * kWave * e < K4) {
                const float4 v = __builtin_bit_cast(float4, xr[e]);
                const float4 w = __builtin_bit_cast(float4, wn[e]);
                const float4 y = {w.x * (v.x * rms_inv), w.y * (v.y * rms_inv),
                                  w.z * (v.z * rms_inv), w.w * (v.w * rms_inv)};
                s_x4[t + S * kWave * e] = __builtin_bit_cast(v4i, y);
                mx = fmaxf(mx, fmaxf(fmaxf(fabsf(y.x), fabsf(y.y)),
                                     fmaxf(fabsf(y.z), fabsf(y.w))));
            }
        }
        mx = wave_max(mx);
        if ((t & 63) == 0) red[S + (t >> 6)] = mx;
        __syncthreads();
        mx = 0.0f;
#pragma unroll
        for (int s = 0; s < S; ++s) mx = fmaxf(mx, red[S + s]);
    } else {
#pragma unroll
        for (int s = 0; s < S; ++s) mx = fmaxf(mx, red[s]);
    }
    scale = mx == 0.0f ? 1.0f : __fdiv_rn(mx, 127.0f);
    if (writer && t == 0 && in.scale_out) in.scale_out[0] = scale;
    return __fdiv_rn(1.0f, scale);
}

}  // namespace gemv
}  // namespace mri
