/*
 * mri_qmatmul.h — C ABI of the MI355X (gfx950) quantized-matmul library.
 *
 * Drop-in boundary for mini-rust-inference's quantized matmul hot path
 * (crate llm-inference-engine, lib llm_engine).  Each entry point names the
 * reference item it replaces as src/<file>:<line>.  The reference functions
 * take host slices / Tensor<f32> and return Result<Tensor<f32>, TensorError>;
 * here every tensor argument is a DEVICE pointer (row-major, contiguous),
 * outputs are caller-owned device buffers, and work is enqueued on `stream`
 * (a hipStream_t; NULL = the default stream).  Weights are uploaded once into
 * opaque device-resident handles, the GPU counterpart of the reference's
 * long-lived QuantizedMatrix / Q8_0WeightMatrix.
 *
 * Errors mirror TensorError (src/tensor/error.rs:7-29): InvalidShape and
 * ShapeMismatch are returned in the same situations and the same check order
 * as the reference; mri_last_error() returns the thread-local `reason`.
 *
 * Numerics contract, per path (m = rows of the call, n = n_out):
 *  - Everything integer is bit-exact at every shape: quantized activations
 *    and their scales, int32 accumulators, Q8_0 / W4A8 block dots.
 *  - Per-channel INT8 f32 outputs ((f32)acc * s_a) * s_w are bit-exact at
 *    every shape (matmul_int8, _rows, _from_f32).
 *  - Q8_0 f32 outputs (matmul_q8_0_direct, its _noalloc variant) are the
 *    block terms t_b = ((f32)dot_b * s_a) * d_b added in the reference's
 *    left-to-right block order, bit-exact, for 5 <= m, except when
 *    m >= 128, m * n > 2^20 and no block_dots_out is requested.  For m <= 4
 *    (the decode GEMV adds per-wave partial sums) and in that prefill range
 *    (an FMA fold, s_a applied once per output) they are within
 *    1e-5 * max(|ref|, sum_b |t_b|) of the reference.
 *    mri_matmul_q8_0_direct_exact keeps the block order at every m.
 *  - W4A8 (extension) f32 outputs equal, bit for bit, those of
 *    mri_matmul_q8_0_direct on the expanded blocks (quant = nibble - 8,
 *    the same scale bits) at every m: the same kernels in the same order.
 *    Against the reference's order that is bit-exact where matmul_q8_0_direct
 *    is, and within the Q8_0 bound elsewhere.
 *  - Q4_0 W4A32 (matmul_q4_0_dequant and its handle form) sums in another
 *    order than the reference and is within 1e-5 * max(|ref|, sum|x_k w_k|).
 *
 * Concurrency: calls are asynchronous on `stream`.  Handles are immutable
 * after creation and may be shared by calls on any stream.  Internal scratch
 * (activation quantization, the prefill GEMMs' partial tiles and tile
 * counters) is kept per (device, stream), so concurrent calls on different
 * streams do not interfere.
 */
#ifndef MRI_QMATMUL_H
#define MRI_QMATMUL_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef enum mri_status {
    MRI_OK = 0,
    MRI_ERR_INVALID_SHAPE = 1,    /* TensorError::InvalidShape  */
    MRI_ERR_SHAPE_MISMATCH = 2,   /* TensorError::ShapeMismatch */
    MRI_ERR_INVALID_ARGUMENT = 3, /* null pointer / bad handle (no Rust analogue: borrowck) */
    MRI_ERR_HIP = 4,              /* HIP runtime error (allocation, launch) */
    MRI_ERR_UNSUPPORTED = 5       /* device is not gfx950, or a size beyond a fixed limit */
} mri_status;

/* Thread-local message for the last non-OK status on this thread
 * (TensorError's `reason`, or the HIP error string). */
const char *mri_last_error(void);
/* Library version string. */
const char *mri_version(void);

/* ===================================================================== */
/* Device-resident weights                                                */
/* ===================================================================== */

/* QuantizedMatrix, src/quant/int8/per_channel.rs:31-40: data [n_out*k_in]
 * int8 row-major, scales [n_out] f32.  Host pointers; uploaded and repacked
 * once into the kernel's tiled layout. */
typedef struct mri_qmatrix mri_qmatrix;
mri_status mri_qmatrix_create(const int8_t *data, const float *scales,
                              size_t n_out, size_t k_in, mri_qmatrix **out);
/* Same from DEVICE pointers (e.g. the output of mri_quantize_per_channel). */
mri_status mri_qmatrix_create_device(const int8_t *data_dev,
                                     const float *scales_dev, size_t n_out,
                                     size_t k_in, void *stream,
                                     mri_qmatrix **out);
/* Reads the weights back in the reference layout (host pointers). */
mri_status mri_qmatrix_read(const mri_qmatrix *w, int8_t *data, float *scales);
size_t mri_qmatrix_n_out(const mri_qmatrix *w);
size_t mri_qmatrix_k_in(const mri_qmatrix *w);
/* Device bytes held by the handle (tiled quants + scales, with padding). */
size_t mri_qmatrix_device_bytes(const mri_qmatrix *w);
void mri_qmatrix_destroy(mri_qmatrix *w);

/* Q8_0WeightMatrix::from_raw_bytes, src/ops/matmul/q8_direct.rs:80-107:
 * raw GGUF Q8_0 blocks ([f16 d][32 x i8], 34 bytes, block (n,b) at
 * (n*k_in/32 + b)*34).  InvalidShape when k_in % 32 != 0 or
 * len != n_out*(k_in/32)*34 (n_out == 0 is accepted).  Host pointer. */
typedef struct mri_q8_0_matrix mri_q8_0_matrix;
mri_status mri_q8_0_matrix_from_raw_bytes(const uint8_t *data, size_t len,
                                          size_t n_out, size_t k_in,
                                          mri_q8_0_matrix **out);
/* Same from a DEVICE pointer to the raw blocks (e.g. an uploaded GGUF slice). */
mri_status mri_q8_0_matrix_from_raw_device(const uint8_t *data_dev,
                                           size_t len, size_t n_out,
                                           size_t k_in, void *stream,
                                           mri_q8_0_matrix **out);
/* Reads the raw 34-byte blocks back (host pointer, len bytes). */
mri_status mri_q8_0_matrix_read_raw(const mri_q8_0_matrix *w, uint8_t *data,
                                    size_t len);
size_t mri_q8_0_matrix_n_out(const mri_q8_0_matrix *w);
size_t mri_q8_0_matrix_k_in(const mri_q8_0_matrix *w);
size_t mri_q8_0_matrix_device_bytes(const mri_q8_0_matrix *w);
void mri_q8_0_matrix_destroy(mri_q8_0_matrix *w);

/* ===================================================================== */
/* Quantizers (device pointers)                                          */
/* ===================================================================== */

/* quantize_symmetric, src/quant/int8/symmetric.rs:42-57: one per-tensor
 * scale over all `len` values; writes q[len] and scale[0] (device). */
mri_status mri_quantize_symmetric(const float *x, size_t len, int8_t *q,
                                  float *scale, void *stream);
/* quantize_symmetric applied to each row of [m,k] separately (the per-row
 * use in matmul_q8_0_direct, src/ops/matmul/q8_direct.rs:264). */
mri_status mri_quantize_symmetric_rows(const float *x, size_t m, size_t k,
                                       int8_t *q, float *scales, void *stream);
/* quantize_per_channel, src/quant/int8/per_channel.rs:98-128 (weight prep);
 * InvalidShape where the reference panics (len != n_out*k_in). */
mri_status mri_quantize_per_channel(const float *w, size_t len, size_t n_out,
                                    size_t k_in, int8_t *data, float *scales,
                                    void *stream);

/* ===================================================================== */
/* Hot path (device pointers)                                            */
/* ===================================================================== */

/* dot_i8_avx2, src/ops/matmul/int8_avx2.rs:136-148: *out = sum a[i]*b[i]. */
mri_status mri_dot_i8(const int8_t *a, const int8_t *b, size_t len,
                      int32_t *out, void *stream);

/* matmul_int8, src/ops/matmul/int8.rs:61-98 (also matmul_int8_avx2
 * int8_avx2.rs:174, matmul_int8_neon int8_neon.rs:158, matmul_int8_parallel
 * parallel.rs:308 — same signature and results):
 *   out[m,n] = ((f32)sum_k act_q[m,k]*w[n,k] * act_scale) * scales[n].
 * InvalidShape when act_q_len != m*k_in.  out is [m, n_out] f32;
 * acc_out (nullable) receives the [m, n_out] int32 accumulators. */
mri_status mri_matmul_int8(const int8_t *act_q, size_t act_q_len,
                           float act_scale, const mri_qmatrix *w, size_t m,
                           float *out, int32_t *acc_out, void *stream);

/* matmul_int8 with one activation scale per row (act_scales: device [m]).
 * No reference counterpart: the per-row-quantized prefill configuration. */
mri_status mri_matmul_int8_rows(const int8_t *act_q, size_t act_q_len,
                                const float *act_scales, const mri_qmatrix *w,
                                size_t m, float *out, int32_t *acc_out,
                                void *stream);

/* matmul_int8_from_f32, src/ops/matmul/int8.rs:113-143: `input` is a
 * contiguous f32 tensor with `ndim` dims (InvalidShape unless ndim == 2);
 * ShapeMismatch{expected:[m,k_in], got:[m,k]} when dims[1] != k_in; then one
 * per-tensor quantize_symmetric over the whole [m,k] and matmul_int8.
 * Optional outputs (nullable, device): act_q_out [m*k], act_scale_out [1],
 * acc_out [m*n_out]. */
mri_status mri_matmul_int8_from_f32(const float *input, const size_t *dims,
                                    size_t ndim, const mri_qmatrix *w,
                                    float *out, int8_t *act_q_out,
                                    float *act_scale_out, int32_t *acc_out,
                                    void *stream);

/* matmul_q8_0_direct, src/ops/matmul/q8_direct.rs:229-289: per-row
 * quantize_symmetric of `input` [m,k], per-block int32 dots, and
 *   out[m,n] = sum over b of t_b,  t_b = ((f32)dot[m,n,b]*s_a[m])*d[n,b].
 * The reference adds the t_b left to right in block order.  Here the
 * activation scales and block dots are bit-exact; out is bit-exact for
 * 5 <= m outside the prefill range below, and otherwise within
 * 1e-5 * max(|ref|, sum_b |t_b|): at m <= 4 (the decode GEMV splits K over
 * waves and adds their partial sums) and at m >= 128, m * n_out > 2^20
 * without block_dots_out (the LDS-tiled GEMM folds fma((f32)dot, d, acc) and
 * multiplies by s_a once).
 * InvalidShape unless ndim == 2; ShapeMismatch when dims[1] != k_in.
 * Optional outputs (nullable, device): block_dots_out [m, n_out, k_in/32]
 * int32, act_scales_out [m]. */
mri_status mri_matmul_q8_0_direct(const float *input, const size_t *dims,
                                  size_t ndim, const mri_q8_0_matrix *w,
                                  float *out, int32_t *block_dots_out,
                                  float *act_scales_out, void *stream);

/* matmul_q8_0_direct (src/ops/matmul/q8_direct.rs:229-289) with the
 * reference's evaluation order kept at every m: out is bit-identical to
 * the left-to-right block sum of q8_direct.rs:269-282 (each output's terms
 * are added by one lane in block order).  Same arguments, checks and
 * optional outputs as mri_matmul_q8_0_direct; slower at m <= 4 and at
 * prefill sizes, where that entry point uses the reordered kernels. */
mri_status mri_matmul_q8_0_direct_exact(const float *input, const size_t *dims,
                                        size_t ndim, const mri_q8_0_matrix *w,
                                        float *out, int32_t *block_dots_out,
                                        float *act_scales_out, void *stream);

/* No counterpart in the reference.  For callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc): mri_matmul_q8_0_direct with the same arguments, checks
 * and results, but its quantized activation rows and scales (m * K' + 4 * m
 * bytes, K' = k_in rounded up to 256, 0 at m = 1) are staged in a fixed
 * device array of MRI_NOALLOC_SCRATCH_BYTES per device instead of the
 * library's grow-on-demand scratch; it calls no hipMalloc / hipFree.  Larger
 * inputs return MRI_ERR_UNSUPPORTED.  All calls on one device share that
 * array: calls that overlap in time on one device (different streams or
 * threads) race and must be serialized by the caller. */
#define MRI_NOALLOC_SCRATCH_BYTES (4 << 20)
mri_status mri_matmul_q8_0_direct_noalloc(const float *input, const size_t *dims,
                                          size_t ndim, const mri_q8_0_matrix *w,
                                          float *out, int32_t *block_dots_out,
                                          float *act_scales_out, void *stream);

/* matmul_q4_0_dequant, src/ops/matmul/q4_0.rs:94-181 (W4A32): weight_q4 is
 * a DEVICE pointer to raw Q4_0 blocks ([f16 d][16 bytes], 18 bytes, element
 * 2i = low nibble of byte i minus 8, element 2i+1 = high nibble minus 8).
 * Check order as the reference: ndim != 2 -> InvalidShape; dims[1] != k ->
 * ShapeMismatch; k % 32 -> InvalidShape; len != n_out*(k/32)*18 ->
 * InvalidShape.  out is [m, n_out] f32. */
mri_status mri_matmul_q4_0_dequant(const float *input, const size_t *dims,
                                   size_t ndim, const uint8_t *weight_q4,
                                   size_t weight_len, size_t n_out, size_t k,
                                   float *out, void *stream);

/* ===================================================================== */
/* Q4_0 with int8 activations (W4A8).  An extension with no counterpart   */
/* in the reference: matmul_q8_0_direct's arithmetic                      */
/* (src/ops/matmul/q8_direct.rs:229-289) on Q4_0 weights (quant = nibble  */
/* - 8), for decode at half the Q8_0 weight bytes.  The reference-faithful */
/* Q4_0 entry point remains mri_matmul_q4_0_dequant (W4A32).              */
/* ===================================================================== */

/* Nibble order of raw Q4_0 blocks: the reference's (create_q4_0_block,
 * src/gguf/dequant.rs:706-749: element 2i = low nibble of byte i, 2i+1 =
 * high nibble) or upstream GGML's (element i = low nibble of byte i,
 * element i + 16 = high nibble), as in llama.cpp Q4_0 files. */
typedef enum {
    MRI_Q4_ORDER_INTERLEAVED = 0,
    MRI_Q4_ORDER_GGML = 1,
} mri_q4_order;

/* Uploads raw Q4_0 blocks ([f16 d][16 bytes], 18 bytes, block (n,b) at
 * (n*k_in/32 + b)*18) in nibble order `order`.  InvalidShape when
 * k_in % 32 != 0 or len != n_out*(k_in/32)*18; InvalidArgument for an
 * unknown order.  _bytes takes a host pointer, _device a device pointer. */
typedef struct mri_q4_0_matrix mri_q4_0_matrix;
mri_status mri_q4_0_matrix_from_raw_bytes(const uint8_t *data, size_t len,
                                          size_t n_out, size_t k_in, int order,
                                          mri_q4_0_matrix **out);
mri_status mri_q4_0_matrix_from_raw_device(const uint8_t *data_dev, size_t len,
                                           size_t n_out, size_t k_in, int order,
                                           void *stream, mri_q4_0_matrix **out);
size_t mri_q4_0_matrix_n_out(const mri_q4_0_matrix *w);
size_t mri_q4_0_matrix_k_in(const mri_q4_0_matrix *w);
size_t mri_q4_0_matrix_device_bytes(const mri_q4_0_matrix *w);
void mri_q4_0_matrix_destroy(mri_q4_0_matrix *w);

/* matmul_q4_0_dequant (src/ops/matmul/q4_0.rs:94-181, W4A32: f32 inputs,
 * no activation quantization) on a device-resident Q4_0 handle instead of
 * raw blocks: the weights stay in the handle's 4-bit lap-block layout and
 * are dequantized in registers by the decode GEMV, up to four rows per
 * launch.  Same checks as mri_matmul_q4_0_dequant for the input (ndim != 2
 * -> InvalidShape, dims[1] != k_in -> ShapeMismatch); input rows 16-byte
 * aligned.  Outputs within 1e-5 * max(|out|, sum_k |x_k w_k|) of the
 * reference's sequential sum.  Rows run in launches of 1, 2 or 4 (3 rows
 * are staged as 4); MRI_ERR_UNSUPPORTED when a launch's f32 rows
 * (rows * K' * 4 bytes, K' = k_in rounded up to 256) exceed 64 KiB of LDS,
 * i.e. K > 4096 at three or four rows, > 8192 at two, > 16384 at one.  The
 * kernel's LDS also holds up to 3.75 KiB of per-wave partial sums. */
mri_status mri_matmul_q4_0_dequant_matrix(const float *input, const size_t *dims, size_t ndim,
                                          const mri_q4_0_matrix *w, float *out, void *stream);

/* Per-row quantize_symmetric of `input` [m,k] (src/quant/int8/symmetric.rs:
 * 42-57), per-block exact int32 dots with the quants, and
 *   out[m,n] = sum over b of ((f32)dot[m,n,b]*s_a[m])*d[n,b],
 * i.e. mri_matmul_q8_0_direct on the blocks with quants nibble - 8: block
 * dots and activation scales bit-exact; out bit-exact for m >= 5 (block
 * order) and within 1e-5 * max(|ref|, sum_b |t_b|) for m <= 4 (per-wave
 * partial sums of the decode GEMV).
 * InvalidShape unless ndim == 2; ShapeMismatch when dims[1] != k_in.
 * Optional outputs (nullable, device):
 * block_dots_out [m, n_out, k_in/32] int32, act_scales_out [m]. */
mri_status mri_matmul_q4_0_w4a8(const float *input, const size_t *dims, size_t ndim,
                                const mri_q4_0_matrix *w, float *out,
                                int32_t *block_dots_out, float *act_scales_out,
                                void *stream);

/* mri_matmul_q4_0_dequant with the nibble order of weight_q4 given
 * (mri_q4_order): MRI_Q4_ORDER_GGML reads upstream GGML blocks (llama.cpp
 * files) with the same W4A32 arithmetic.  An option with no counterpart in
 * the reference; InvalidArgument for an unknown order, then the same checks
 * in the same order as mri_matmul_q4_0_dequant. */
mri_status mri_matmul_q4_0_dequant_ordered(const float *input, const size_t *dims,
                                           size_t ndim, const uint8_t *weight_q4,
                                           size_t weight_len, size_t n_out, size_t k,
                                           int order, float *out, void *stream);

/* Waits for all work enqueued on `stream`. */
mri_status mri_synchronize(void *stream);

/* Diagnostic, no counterpart in the reference: one kernel that streams
 * `bytes` (rounded down to 16) of device memory at p (16-byte aligned) and
 * discards them, i.e. the ceiling a one-kernel read of that size reaches on
 * this device, next to which the benchmark reports the decode GEMVs.  sink
 * (nullable, device) is never written for ordinary data. */
mri_status mri_hbm_read(const void *p, size_t bytes, int32_t *sink, void *stream);

/* Diagnostic, no counterpart in the reference: the int8 MFMA ceiling of
 * this device with operands of real data.  One workgroup of 8 waves per CU
 * (*n_cus receives the CU count) loads 32 KiB of int8 operands from src
 * (device, 16-byte aligned) once and runs iters x 8 v_mfma_i32_32x32x32_i8
 * per wave (2 * 32768 * 8 * iters int ops per wave) with no other memory
 * traffic; the benchmark times it beside the prefill GEMM. */
mri_status mri_mfma_i8_peak(const int8_t *src, int iters, int32_t *sink, int *n_cus,
                            void *stream);

#ifdef __cplusplus
}
#endif
#endif
