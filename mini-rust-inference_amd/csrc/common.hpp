// common.hpp — shared definitions of the gfx950 quantized-matmul library.
//
// Device weight layouts (chosen at upload time, not visible through the ABI):
//
//  * Per-channel INT8 (QuantizedMatrix, per_channel.rs:31-40) is stored as
//    "MFMA chunks": the output rows are grouped in tiles of 16 and K in
//    slabs of 64.  Chunk (p, T) (slab p, tile T) is 1 KiB; chunks are stored
//    slab-major, at byte offset (p * n_tiles + T) * 1024, so a sweep over K
//    by the waves of all tiles reads one contiguous, moving window.  Inside
//    a chunk, lane l (0..63) owns 16 bytes at l * 16: row 16*T + (l % 16),
//    k = 64*p + 16*(l / 16) + [0, 16).  This is the B operand of
//    v_mfma_i32_16x16x64_i8 for lane l (the A operand uses the same k
//    assignment), so one global_load_dwordx4 per lane per chunk feeds one
//    MFMA and a wave reads 1 KiB contiguous bytes per instruction.
//    Scales: f32 [n_tiles * 16] (zero padded).
//
//  * Q8_0 (Q8_0WeightMatrix, q8_direct.rs:60-69) is stored in "lap blocks"
//    of 8 Q8_0 blocks (256 k) x 16 rows, 4352 bytes each (the raw block
//    size, 34 bytes x 128), tile-major: lap block (T, q) of tile T and lap
//    q = 0 .. G-1 (G = Kp / 256, Kp = K rounded up to 256) sits at byte
//    offset (T * G + q) * 4352, so a tile's whole K is one contiguous run
//    and a sweep reads quants and scales from the same DRAM pages.  A lap
//    block holds:
//     - 4 chunks of 1 KiB (c = 0..3, slab p = 4q + c) in which lane l's 16
//       bytes hold two 8-byte B operands of v_mfma_i32_16x16x32_i8 (one MFMA
//       per 32-element block): bytes [8h, 8h+8) = quants [8g, 8g+8) of block
//       2p+h of row 16T + (l % 16), g = l / 16;
//     - then 16 x 16 bytes of f16 scales (2 bytes per block, as in GGUF):
//       row r at byte 4096 + 16 r holds the scales of blocks 8q .. 8q+7, so
//       one 16-byte load gives a lane the scales of its 4 chunks.
//
//  * Q4_0 for the W4A8 path (an extension) uses the same lap blocks with
//    4-bit quants, 2304 bytes each: 2 KiB of quants, then the 256 bytes of
//    f16 scales at byte 2048.  Quant piece u (0..1) of lane l is 16 bytes at
//    byte (u * 64 + l) * 16: u32 word 2c' + h (c' = 0..1) holds the quants
//    of block 2p + h, p = 4q + 2u + c', that lane l's MFMA B operand needs
//    (elements 8g .. 8g+7, g = l / 16, row 16T + l % 16): byte i has element
//    8g + i in its low nibble and element 8g + 4 + i in its high nibble.
//    Each nibble holds the raw GGUF nibble XOR 8, which is the 4-bit two's
//    complement of the quant (nibble - 8), so that a nibble moved to the
//    high half of a byte reads as the int8 16 * quant.
//
//  * Activations quantized by the library are written to a per-(device,
//    stream) scratch in [M][Kp] int8 rows (zero padded).  For Q8_0 the 64
//    bytes of each chunk are permuted to match the weight chunk:
//    element kk of a chunk sits at q8_perm(kk).
//
//  * Activations of the prefill GEMM (M >= kGemmMinRows) are packed into
//    its MFMA fragment layout: row group g = m / 32, K step p = k / 64,
//    half h = (k % 64) / 32; fragment (p, g, h) is 1 KiB at byte offset
//    ((p * MG + g) * 2 + h) * 1024 with MG = ceil(M / 32); inside it lane
//    l = m % 32 + 32 * ((k % 32) / 16) owns 16 bytes at l * 16 (element
//    k % 16 at byte l * 16 + k % 16).  Rows past M are zero.
#pragma once

#include <hip/hip_runtime.h>

#include <atomic>
#include <climits>
#include <cstddef>
#include <cstdint>
#include <mutex>
#include <string>

#include "mri_qmatmul.h"

namespace mri {

constexpr int kTileN = 16;        // output rows per MFMA tile
constexpr int kChunkK = 64;       // K elements per 1 KiB chunk
constexpr int kQK = 32;           // Q8_0 / Q4_0 block elements
constexpr int kQ8Bytes = 34;      // raw Q8_0 block bytes
constexpr int kQ4Bytes = 18;      // raw Q4_0 block bytes
constexpr int kQ8ScaleGroup = 8;  // blocks per scale group (16 bytes of f16)
constexpr int kBufWord3 = 0x00020000;  // raw buffer resource, dword 3 (gfx950): loads past
                                       // num_records return zeros

inline size_t round_up(size_t v, size_t m) { return (v + m - 1) / m * m; }

// Position of element kk (0..63) of a Q8_0 chunk inside the permuted
// 64-byte activation chunk: [g = 0..3][h = 0..1][8 bytes].
__host__ __device__ inline int q8_perm(int kk) {
    return ((kk >> 3) & 3) * 16 + (kk >> 5) * 8 + (kk & 7);
}

struct QMatrixDev {
    size_t n_out = 0, k_in = 0;
    size_t n_tiles = 0;     // ceil(n_out / 16)
    size_t kp = 0;          // K padded to 64
    int8_t *tiles = nullptr;  // n_tiles * (kp/64) KiB
    float *scales = nullptr;  // n_tiles * 16
    int device = 0;
};

constexpr int kQ8LapBytes = 4352;  // one Q8_0 lap block: 4 chunks + 256 bytes of scales
constexpr int kQ4LapBytes = 2304;  // one Q4_0 (W4A8) lap block: 2 KiB of nibbles + scales
constexpr int kQ8LapK = 256;       // K elements per lap block

// Q8_0 weights, or Q4_0 weights for the W4A8 path (w4).
struct Q8MatrixDev {
    size_t n_out = 0, k_in = 0;
    size_t n_blocks = 0;    // k_in / 32
    size_t n_tiles = 0;
    size_t kp = 0;          // K padded to 256
    int8_t *laps = nullptr;  // n_tiles * (kp/256) lap blocks
    int device = 0;
    bool w4 = false;
    size_t laps_per_tile() const { return kp / kQ8LapK; }
    size_t lap_bytes() const { return w4 ? kQ4LapBytes : kQ8LapBytes; }
    size_t bytes() const { return n_tiles * laps_per_tile() * lap_bytes(); }
};

// Exact f16 -> f32 decode (v_cvt_f32_f16), the f16_to_f32 of
// gguf/quantization.rs:416-459 for every finite input.
// The greedy argmax's order (sampling/mod.rs:144-151, max_by over
// partial_cmp) as one 64-bit key: the value's bits mapped to an unsigned
// order (-0 counted as +0), then the index, so equal values go to the larger
// index; NaN gets key 0, below every value (it is never chosen).
__device__ inline unsigned long long argmax_key(float v, int n) {
    if (v != v) return 0ull;
    const unsigned b = __float_as_uint(v == 0.0f ? 0.0f : v);
    const unsigned ord = (b & 0x80000000u) ? ~b : (b | 0x80000000u);
    return ((unsigned long long)ord << 32) | (unsigned)n;
}

__device__ inline float f16_bits_to_f32(unsigned bits) {
    return (float)__builtin_bit_cast(_Float16, (unsigned short)bits);
}

// ---- error handling ------------------------------------------------------
mri_status set_error(mri_status st, const std::string &msg);
mri_status hip_error(hipError_t e, const char *what);

#define MRI_HIP(call)                                               \
    do {                                                            \
        hipError_t _e = (call);                                     \
        if (_e != hipSuccess) return ::mri::hip_error(_e, #call);   \
    } while (0)

#define MRI_LAUNCHED(what)                                          \
    do {                                                            \
        hipError_t _e = hipGetLastError();                          \
        if (_e != hipSuccess) return ::mri::hip_error(_e, what);    \
    } while (0)

// ---- one-time per-device set-up --------------------------------------------
// A call site's static DeviceOnce runs its set-up (hipFuncSetAttribute, a
// device query) once per device; concurrent first calls wait for the one
// that runs it, later calls cost one acquire load.
constexpr int kMaxDevices = 64;
class DeviceOnce {
  public:
    template <class F>
    hipError_t run(F &&setup) {
        int dev = 0;
        hipError_t e = hipGetDevice(&dev);
        if (e != hipSuccess) return e;
        if (dev < 0 || dev >= kMaxDevices) return hipErrorInvalidDevice;
        if (done_[dev].load(std::memory_order_acquire)) return hipSuccess;
        std::lock_guard<std::mutex> g(mu_);
        if (done_[dev].load(std::memory_order_relaxed)) return hipSuccess;
        e = setup(dev);
        if (e == hipSuccess) done_[dev].store(true, std::memory_order_release);
        return e;
    }

  private:
    std::atomic<bool> done_[kMaxDevices] = {};
    std::mutex mu_;
};

// Number of CUs of the current device (queried once per device), or 0.
int device_cus();

// ---- per-(device, stream) scratch ----------------------------------------
// Grow-only device buffer; growth synchronizes `stream` before freeing the
// old buffer, so work already enqueued on it never sees freed memory.
mri_status scratch_get(hipStream_t stream, size_t bytes, void **ptr);

// ---- kernel launchers (defined in the .hip files) -------------------------
// quantize.hip
mri_status launch_quantize_tensor(const float *x, size_t m, size_t k,
                                  size_t ld_out, bool q8_perm_layout,
                                  int8_t *q_pad, int8_t *q_plain,
                                  float *scale, float *partials,
                                  hipStream_t s);
mri_status launch_quantize_rows(const float *x, size_t m, size_t k,
                                size_t ld_out, bool q8_perm_layout,
                                int8_t *q_pad, int8_t *q_plain,
                                float *scales, hipStream_t s);
// The same for rows of 2k, [gate | up]: quantizes their SwiGLU, silu(g) * u
// (the values the prefill SwiGLU kernel writes), into q_pad [m][ld_out].
mri_status launch_swiglu_quantize_rows(const float *gu, size_t m, size_t k, size_t ld_out,
                                       bool q8_perm_layout, int8_t *q_pad, float *scales,
                                       hipStream_t s);
mri_status launch_quantize_per_channel(const float *w, size_t n, size_t k,
                                       int8_t *data, float *scales,
                                       hipStream_t s);
mri_status launch_pad_rows(const int8_t *src, size_t m, size_t k, size_t kp,
                           int8_t *dst, hipStream_t s);
// quantize_symmetric (per tensor) of [m,k] into the packed GEMM layout.
mri_status launch_quantize_pack(const float *x, size_t m, size_t k, size_t kp,
                                int8_t *packed, int8_t *q_plain, float *scale,
                                float *partials, hipStream_t s);
// int8 rows [m][ld] (k valid) into the packed GEMM layout.
mri_status launch_pack_gemm(const int8_t *src, size_t m, size_t k, size_t ld, size_t kp,
                            int8_t *packed, hipStream_t s);
mri_status launch_dot_i8(const int8_t *a, const int8_t *b, size_t n,
                         int32_t *out, hipStream_t s);
size_t quantize_partials_count(size_t n);

// hbm_read.hip: a plain streaming read of `bytes` (16-byte aligned) device
// bytes; sink (nullable) is written only in a case that does not occur.
mri_status launch_hbm_read(const void *p, size_t bytes, int32_t *sink, hipStream_t s);
// One workgroup of 8 waves per CU, each running 8 * iters int8 32x32x32
// MFMAs on operands loaded once from src (32 KiB of int8).
mri_status launch_mfma_peak(const int8_t *src, int iters, int32_t *sink, hipStream_t s);

// repack.hip
mri_status launch_repack_int8(const int8_t *data, const float *scales,
                              QMatrixDev &w, hipStream_t s);
mri_status launch_repack_q8_0(const uint8_t *raw, Q8MatrixDev &w,
                              hipStream_t s);
// Raw Q4_0 blocks (ggml_order: low nibbles = elements 0..15; else the
// reference's interleaved order) into W4A8 lap blocks (w.w4).
mri_status launch_repack_q4_0(const uint8_t *raw, bool ggml_order, Q8MatrixDev &w,
                              hipStream_t s);

// skinny.hip: M <= 32 rows per launch (larger M loops), one wave per tile.
// act: [M][kp] int8 (Q8_0: chunk-permuted).  Activation scale of row m is
// sa_ptr[m * sa_stride] when sa_ptr != nullptr, else sa_value.
mri_status launch_skinny_int8(const int8_t *act, size_t m, const float *sa_ptr,
                              int sa_stride, float sa_value,
                              const QMatrixDev &w, float *out,
                              int32_t *acc_out, hipStream_t s);
mri_status launch_skinny_q8_0(const int8_t *act, size_t m,
                              const float *sa_ptr, const Q8MatrixDev &w,
                              float *out, int32_t *block_dots,
                              hipStream_t s);
// gemv.hip: M <= 4, K split over S waves per 16-row tile, weights streamed
// through a per-wave ring of loads.  Activations come either as one f32 row
// x (quantized in the kernel; requires gemv_fusable, M == 1; optional
// act_q_out [k] and scale_out [1]) or as quantized rows act [m][kp] (Q8_0:
// chunk-permuted) with their scales.  ops: the single-row extras below.
//
// RowOps: what the fused path (one f32 row) can do besides the projection.
// Every pointer is 16-byte aligned and holds k floats.
struct RowOps {
    const float *norm_w = nullptr;  // RMS-normalize the row with these weights and eps
    float eps = 0.0f;
    float *x_out = nullptr;         // receives a copy of x as read
    bool accum = false;             // out += the projection (a residual add)
    // The row x is the SiLU of the gate half of a SwiGLU (what silu_n below
    // stores): the projection's input is x * up elementwise.  With x =
    // g / (1 + exp(-g)) that is the SwiGLU g / (1 + exp(-g)) * u of
    // ops/activation/swiglu.rs, rounded as the separate SwiGLU kernel rounds
    // it (not with norm_w or x_out).
    const float *up = nullptr;
    // Output channels [0, silu_n) are stored as v / (1 + exp(-v)), the SiLU
    // (ops/activation/silu.rs:23-26) of a SwiGLU gate, once per channel in
    // the producing projection instead of in every workgroup of the
    // consuming one (not with accum or rope_n).
    int silu_n = 0;
    // First half of the greedy argmax of the output row (sampling/mod.rs:
    // 144-151): each 16-channel tile T writes the largest key of its outputs
    // to arg_keys[T] (argmax_key: the order of the reference's max_by, the
    // last of equal maxima, NaN never chosen; 0 for no candidate), and
    // launch_argmax_keys reduces them.
    unsigned long long *arg_keys = nullptr;
    // The row is row t of the table x points at, t the greedy token of the
    // previous decode step: the largest of the n_in_keys keys in_keys (the
    // previous step's arg_keys; argmax_key order, the index in the low
    // word, 0 when every key is 0).  The kernel reduces the keys in its
    // prologue, before it loads the row, and workgroup 0 stores t to
    // tok_out (what launch_argmax_keys computes).
    const unsigned long long *in_keys = nullptr;
    int n_in_keys = 0;
    uint32_t *tok_out = nullptr;
    // RoPE (ops/rope.rs) on output channels [0, rope_n): the pairs
    // (2i, 2i+1) of each head of hd channels rotate by the table entries
    // i % (hd/2) of rope_cos / rope_sin (one position's rows).
    const float *rope_cos = nullptr, *rope_sin = nullptr;
    int rope_n = 0, hd = 2;
    // Output channels from seg1 on go to out1[n - seg1], from seg2 on to
    // out2[n - seg2] (q | k | v of a fused projection into the KV cache).
    int seg1 = INT_MAX, seg2 = INT_MAX;
    float *out1 = nullptr, *out2 = nullptr;
    bool any() const {
        return norm_w || x_out || accum || up || arg_keys || in_keys || rope_n > 0 || out1 ||
               out2 || silu_n > 0;
    }
};
bool gemv_int8_supported(bool fused, size_t m, size_t n_tiles, size_t k, size_t kp);
// The device matrices behind the public handles (capi.cpp).
const QMatrixDev &handle_dev(const mri_qmatrix *h);
const Q8MatrixDev &handle_dev(const mri_q8_0_matrix *h);
const Q8MatrixDev &handle_dev(const mri_q4_0_matrix *h);
bool gemv_q8_supported(bool fused, size_t m, size_t n_tiles, size_t k, size_t kp);
// W4A32 (matmul_q4_0_dequant semantics) on a Q4_0 lap-block handle (w.w4):
// x f32 [m][k], 16-byte aligned, k % 4 == 0; MRI_ERR_UNSUPPORTED when the
// f32 rows of four do not fit the GEMV's LDS staging.
mri_status launch_gemv_w4a32(const float *x, size_t m, size_t k, const Q8MatrixDev &w,
                             float *out, hipStream_t st);
bool gemv_fusable(size_t m, size_t k, const float *x);
bool row_ops_ok(const float *x, const RowOps &ops);
mri_status launch_gemv_int8(const float *x, const int8_t *act, size_t m,
                            const float *sa_ptr, int sa_stride, float sa_value,
                            const QMatrixDev &w, float *out, int8_t *act_q_out,
                            float *scale_out, int32_t *acc_out, hipStream_t s,
                            const RowOps &ops = RowOps{});
mri_status launch_gemv_q8_0(const float *x, const int8_t *act, size_t m,
                            const float *sa_rows, const Q8MatrixDev &w, float *out,
                            int32_t *block_dots, float *scales_out, hipStream_t s,
                            const RowOps &ops = RowOps{});

// gemm.hip: prefill-sized M on MFMA with LDS tiles, packed activations.
constexpr size_t kGemmMinRows = 64;
inline size_t gemm_row_groups(size_t m) { return (m + 31) / 32; }
inline size_t gemm_pack_bytes(size_t m, size_t kp) { return gemm_row_groups(m) * 32 * kp; }
// Byte offset of element (m, k) in the packed layout.
__host__ __device__ inline size_t gemm_pack_offset(size_t m, size_t k, size_t mg) {
    const size_t p = k >> 6, kk = k & 63, h = kk >> 5;
    const size_t lane = (m & 31) + 32 * ((kk & 31) >> 4);
    return (((p * mg + (m >> 5)) * 2 + h) * 64 + lane) * 16 + (kk & 15);
}
// Workspace of the stream-K GEMM for m rows (0: the shape does not use
// one): int32 partial tiles plus per-tile counters.  The counters must be
// zero when the workspace is first used; every call leaves them zero.
size_t gemm_ws_bytes(size_t m, const QMatrixDev &w);
// Tile counters at the start of the GEMM workspace (gemm_ws_get), shared by
// the INT8 and Q8_0 GEMMs: zero between calls.
constexpr int kGemmWsCounters = 65536;
// gemm_q8.hip: prefill-sized matmul_q8_0_direct on LDS-staged MFMA tiles.
// ws: gemm_q8_ws_bytes(m, w) bytes of the GEMM workspace for the K split,
// or null (no K split; nothing allocated).
bool gemm_q8_supported(size_t m, const Q8MatrixDev &w);
size_t gemm_q8_ws_bytes(size_t m, const Q8MatrixDev &w);
mri_status launch_gemm_q8_0(const int8_t *act, size_t m, const float *sa_rows,
                            const Q8MatrixDev &w, float *out, void *ws, hipStream_t s);
// rows: act_packed is the caller's row-major [m][k] int8 (gemm_rows_ok).
mri_status launch_gemm_int8(const int8_t *act_packed, size_t m, const float *sa_ptr,
                            int sa_stride, float sa_value, const QMatrixDev &w,
                            float *out, int32_t *acc_out, void *ws, hipStream_t s,
                            bool rows = false);
bool gemm_rows_ok(size_t m, const QMatrixDev &w, const void *act);
// Per-(device, stream) GEMM workspace (capi.cpp), grow-only, zeroed when
// (re)allocated.
mri_status gemm_ws_get(hipStream_t stream, size_t bytes, void **ptr);

// q4_0.hip
mri_status launch_q4_0_dequant(const float *x, size_t m, size_t k, const uint8_t *w,
                               size_t n_out, bool ggml_order, float *out, hipStream_t s);

// capi.cpp: row concatenation of weight handles (whole 16-row tiles, one K)
// into a new handle, for fused projections that share their input.
mri_status concat_qmatrix(const mri_qmatrix *const *parts, int n, hipStream_t s,
                          mri_qmatrix **out);
mri_status concat_q8_0_matrix(const mri_q8_0_matrix *const *parts, int n, hipStream_t s,
                              mri_q8_0_matrix **out);
mri_status concat_q4_0_matrix(const mri_q4_0_matrix *const *parts, int n, hipStream_t s,
                              mri_q4_0_matrix **out);

// llama.hip: the decoder layer's non-matmul steps (f32 rows in HBM).
mri_status launch_embed(const float *table, const uint32_t *tokens, size_t rows, size_t d,
                        float *x, hipStream_t s);
mri_status launch_rmsnorm(const float *x, const float *w, size_t rows, size_t d, float eps,
                          float *out, hipStream_t s);
// x_out = table[tokens] (rows), out = rmsnorm(x_out): one pass.
mri_status launch_embed_rmsnorm(const float *table, const uint32_t *tokens, size_t rows,
                                size_t d, const float *w, float eps, float *x_out, float *out,
                                hipStream_t s);
// x += delta, out = rmsnorm(x): one pass.
// RMSNorm statistics of rows (rms_inv, max |normalized|) per row into
// stats[2*row], stats[2*row+1] without storing the normalized rows: mode 0
// norm x, mode 1 gather from the table x by tokens into x_out first, mode 2
// add delta into x_out (= x) first.  rmsnorm_stats_supported(d): d % 4 == 0
// and d <= 8192 (16-byte aligned rows).
bool rmsnorm_stats_supported(size_t d);
mri_status launch_rmsnorm_stats(int mode, const float *x, const float *delta,
                                const uint32_t *tokens, float *x_out, size_t rows, size_t d,
                                const float *w, float eps, float *stats, hipStream_t s);
// Quantize the normalized rows w * (x * rms_inv) from those statistics:
// form 0 per-tensor scale into the GEMM-packed layout (ld = kp), form 1
// per-tensor into [rows][ld] plain, form 2 per-row scales into [rows][ld]
// chunk-permuted (Q8_0), form 3 the f32 normalized rows into `normed`.
mri_status launch_norm_quant(int form, const float *x, const float *w, const float *stats,
                             size_t rows, size_t d, size_t ld, int8_t *q, float *scales,
                             float *normed, hipStream_t s);
// capi.cpp: the matmul dispatch on quantized rows [m][kp] (INT8 plain,
// Q8_0 / W4A8 chunk-permuted), as the entry points use it.
mri_status run_int8(const int8_t *act, size_t m, const float *sa_ptr, int sa_stride,
                    float sa_value, const QMatrixDev &w, float *out, int32_t *acc_out,
                    hipStream_t s);
// may_alloc false: no workspace is allocated (no K split in the GEMM).
mri_status run_q8(const int8_t *act, size_t m, const float *sa_rows, const Q8MatrixDev &w,
                  float *out, int32_t *block_dots, hipStream_t s, bool may_alloc = true);
mri_status launch_add_rmsnorm(float *x, const float *delta, size_t rows, size_t d,
                              const float *w, float eps, float *out, hipStream_t s);
// RoPE of q in place; rotated k and v rows into the cache at start_pos + s.
// q_stride / kv_stride: floats between consecutive rows of q and of k, v.
mri_status launch_rope_qkv(float *q, const float *k, const float *v, size_t seq, size_t n_heads,
                           size_t n_kv, size_t head_dim, size_t q_stride, size_t kv_stride,
                           const float *cos_t, const float *sin_t, size_t start_pos, float *kc,
                           float *vc, hipStream_t s);
bool attention_supported(size_t head_dim);
// Causal GQA of seq_q query rows (positions start_pos ..) against cache rows
// 0 .. start_pos + seq_q - 1.  part: attention_part_floats(...) floats of
// workspace for the split-key one-row form (nullable: one workgroup per head);
// its first words are per-head arrival counters, zeroed before the first
// call and left zero by every call.
size_t attention_part_floats(size_t n_heads, size_t head_dim, size_t max_seq);
mri_status launch_attention(const float *q, size_t q_stride, size_t seq_q, const float *kc,
                            const float *vc, size_t n_heads, size_t n_kv_heads, size_t head_dim,
                            size_t start_pos, float *out, float *part, hipStream_t s);
mri_status launch_swiglu(const float *gate, const float *up, size_t n, float *out,
                         hipStream_t s);
// rows of [gate | up] (2 * ffn floats each) -> rows of ffn.
mri_status launch_swiglu_rows(const float *gu, size_t rows, size_t ffn, float *out,
                              hipStream_t s);
mri_status launch_add(const float *a, const float *b, size_t n, float *out, hipStream_t s);
// rows == 1 runs a split form whose blocks meet through a counter in the
// stream's argmax workspace (argmax_ws_get: kArgmaxWsBytes, zeroed).
mri_status launch_argmax(const float *v, size_t rows, size_t n, uint32_t *idx, hipStream_t s);
constexpr size_t kArgmaxWsBytes = 4096;
mri_status argmax_ws_get(hipStream_t stream, void **ptr, size_t bytes = kArgmaxWsBytes);
// Reduces n keys of argmax_key (arg_keys of a one-row projection, one per
// 16-channel tile) to the index of the largest (0 when every key is 0) in
// idx[0]; with table, copies that row of table ([*][d] f32, 16-byte aligned,
// d % 4 == 0) to x_out.
mri_status launch_argmax_keys(const unsigned long long *keys, size_t n, uint32_t *idx,
                              const float *table, size_t d, float *x_out, hipStream_t s);
// One row: the argmax, then row idx of table ([*][d]) copied to x_out.
mri_status launch_argmax_embed(const float *v, size_t n, uint32_t *idx, const float *table,
                               size_t d, float *x_out, hipStream_t s);

}  // namespace mri
