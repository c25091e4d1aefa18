//! Raw FFI declarations of `libmri_qmatmul.so`, the MI355X (gfx950) library
//! behind `llm_engine::ops::matmul`'s quantized entry points
//! (`src/ops/matmul/mod.rs:32-41`) and the GPU `LlamaModelInt8`
//! (`src/model/llama/forward_int8.rs:416-546`).
//!
//! Every item is one to one with `include/mri_qmatmul.h` and
//! `include/mri_llama.h`: the same names, argument order and C types
//! (`size_t` is `usize`, `int` is `c_int`, enums are `c_int` constants,
//! handles are opaque structs behind raw pointers).  A CPU test of the
//! repository parses both headers and this file and fails on any difference.
//!
//! Conventions of the C ABI: tensors are DEVICE pointers (row-major,
//! contiguous) unless a function says "host"; outputs are caller-owned;
//! `stream` is a `hipStream_t` (null = the default stream) and every call is
//! asynchronous on it.  A non-OK status leaves a thread-local message, read
//! with [`mri_last_error`] (the `reason` of the reference's `TensorError`).
//! The safe layer that maps these onto the reference's signatures
//! (`Result<Tensor<f32>, TensorError>`) lives in the engine, behind a `gpu`
//! feature; [`check`] is the status-to-`Result` step it builds on.
#![allow(non_camel_case_types)]

use core::ffi::{c_char, c_int, c_void};
use core::marker::{PhantomData, PhantomPinned};

// ---- status ---------------------------------------------------------------

/// `mri_status`: `TensorError` kinds plus the library's own.
pub type mri_status = c_int;
pub const MRI_OK: mri_status = 0;
/// `TensorError::InvalidShape`
pub const MRI_ERR_INVALID_SHAPE: mri_status = 1;
/// `TensorError::ShapeMismatch`
pub const MRI_ERR_SHAPE_MISMATCH: mri_status = 2;
/// null pointer or bad handle (no Rust analogue: the borrow checker)
pub const MRI_ERR_INVALID_ARGUMENT: mri_status = 3;
/// HIP runtime error (allocation, launch)
pub const MRI_ERR_HIP: mri_status = 4;
/// device is not gfx950, or a size beyond a fixed limit
pub const MRI_ERR_UNSUPPORTED: mri_status = 5;

/// Nibble order of raw Q4_0 blocks (`mri_q4_order`).
pub type mri_q4_order = c_int;
/// The reference's order (`create_q4_0_block`, `src/gguf/dequant.rs:706-749`).
pub const MRI_Q4_ORDER_INTERLEAVED: mri_q4_order = 0;
/// Upstream GGML's order (llama.cpp files).
pub const MRI_Q4_ORDER_GGML: mri_q4_order = 1;

/// Format of a projection weight of the GPU model (`mri_weight_format`).
pub type mri_weight_format = c_int;
/// `*const mri_qmatrix`
pub const MRI_WEIGHT_INT8: mri_weight_format = 0;
/// `*const mri_q8_0_matrix`
pub const MRI_WEIGHT_Q8_0: mri_weight_format = 1;
/// device pointer to raw Q4_0 blocks, `n_out x k_in`
pub const MRI_WEIGHT_Q4_0: mri_weight_format = 2;
/// `*const mri_q4_0_matrix` projected with int8 activations (W4A8 extension)
pub const MRI_WEIGHT_Q4_0_W4A8: mri_weight_format = 3;

/// Bytes of the fixed per-device staging of
/// [`mri_matmul_q8_0_direct_noalloc`] (`MRI_NOALLOC_SCRATCH_BYTES`).
pub const MRI_NOALLOC_SCRATCH_BYTES: usize = 4 << 20;

// ---- opaque handles ---------------------------------------------------------

/// Device-resident `QuantizedMatrix` (`src/quant/int8/per_channel.rs:31-40`).
#[repr(C)]
pub struct mri_qmatrix {
    _data: [u8; 0],
    _marker: PhantomData<(*mut u8, PhantomPinned)>,
}
/// Device-resident `Q8_0WeightMatrix` (`src/ops/matmul/q8_direct.rs:60-69`).
#[repr(C)]
pub struct mri_q8_0_matrix {
    _data: [u8; 0],
    _marker: PhantomData<(*mut u8, PhantomPinned)>,
}
/// Device-resident Q4_0 weights (W4A8 and the W4A32 handle form).
#[repr(C)]
pub struct mri_q4_0_matrix {
    _data: [u8; 0],
    _marker: PhantomData<(*mut u8, PhantomPinned)>,
}
/// GPU `LlamaModelInt8` (`src/model/llama/forward_int8.rs:416-546`).
#[repr(C)]
pub struct mri_llama {
    _data: [u8; 0],
    _marker: PhantomData<(*mut u8, PhantomPinned)>,
}
/// Device `KvCache` (`src/cache/kv_cache.rs:65`).
#[repr(C)]
pub struct mri_kv_cache {
    _data: [u8; 0],
    _marker: PhantomData<(*mut u8, PhantomPinned)>,
}

// ---- model structs ------------------------------------------------------------

/// The `LlamaConfig` fields the forward pass uses
/// (`src/model/llama/config.rs`).
#[repr(C)]
#[derive(Debug, Clone, Copy)]
pub struct mri_llama_config {
    pub dim: usize,
    pub n_heads: usize,
    pub n_kv_heads: usize,
    pub ffn_dim: usize,
    pub vocab: usize,
    pub max_seq: usize,
    pub eps: f32,
    pub rope_base: f32,
    pub n_layers: usize,
}

/// A borrowed projection weight `[n_out, k_in]`; `format` is an
/// `mri_weight_format` and says what `ptr` points at.
#[repr(C)]
#[derive(Debug, Clone, Copy)]
pub struct mri_weight_ref {
    pub format: c_int,
    pub ptr: *const c_void,
    pub n_out: usize,
    pub k_in: usize,
}

// ---- include/mri_qmatmul.h ------------------------------------------------------

extern "C" {
    pub fn mri_last_error() -> *const c_char;
    pub fn mri_version() -> *const c_char;

    // QuantizedMatrix (per_channel.rs:31-40); host pointers
    pub fn mri_qmatrix_create(
        data: *const i8,
        scales: *const f32,
        n_out: usize,
        k_in: usize,
        out: *mut *mut mri_qmatrix,
    ) -> mri_status;
    pub fn mri_qmatrix_create_device(
        data_dev: *const i8,
        scales_dev: *const f32,
        n_out: usize,
        k_in: usize,
        stream: *mut c_void,
        out: *mut *mut mri_qmatrix,
    ) -> mri_status;
    pub fn mri_qmatrix_read(w: *const mri_qmatrix, data: *mut i8, scales: *mut f32) -> mri_status;
    pub fn mri_qmatrix_n_out(w: *const mri_qmatrix) -> usize;
    pub fn mri_qmatrix_k_in(w: *const mri_qmatrix) -> usize;
    pub fn mri_qmatrix_device_bytes(w: *const mri_qmatrix) -> usize;
    pub fn mri_qmatrix_destroy(w: *mut mri_qmatrix);

    // Q8_0WeightMatrix::from_raw_bytes (q8_direct.rs:80-107)
    pub fn mri_q8_0_matrix_from_raw_bytes(
        data: *const u8,
        len: usize,
        n_out: usize,
        k_in: usize,
        out: *mut *mut mri_q8_0_matrix,
    ) -> mri_status;
    pub fn mri_q8_0_matrix_from_raw_device(
        data_dev: *const u8,
        len: usize,
        n_out: usize,
        k_in: usize,
        stream: *mut c_void,
        out: *mut *mut mri_q8_0_matrix,
    ) -> mri_status;
    pub fn mri_q8_0_matrix_read_raw(w: *const mri_q8_0_matrix, data: *mut u8, len: usize)
        -> mri_status;
    pub fn mri_q8_0_matrix_n_out(w: *const mri_q8_0_matrix) -> usize;
    pub fn mri_q8_0_matrix_k_in(w: *const mri_q8_0_matrix) -> usize;
    pub fn mri_q8_0_matrix_device_bytes(w: *const mri_q8_0_matrix) -> usize;
    pub fn mri_q8_0_matrix_destroy(w: *mut mri_q8_0_matrix);

    // quantize_symmetric (symmetric.rs:42-57), per row (q8_direct.rs:264),
    // quantize_per_channel (per_channel.rs:98-128)
    pub fn mri_quantize_symmetric(
        x: *const f32,
        len: usize,
        q: *mut i8,
        scale: *mut f32,
        stream: *mut c_void,
    ) -> mri_status;
    pub fn mri_quantize_symmetric_rows(
        x: *const f32,
        m: usize,
        k: usize,
        q: *mut i8,
        scales: *mut f32,
        stream: *mut c_void,
    ) -> mri_status;
    pub fn mri_quantize_per_channel(
        w: *const f32,
        len: usize,
        n_out: usize,
        k_in: usize,
        data: *mut i8,
        scales: *mut f32,
        stream: *mut c_void,
    ) -> mri_status;

    // dot_i8_avx2 (int8_avx2.rs:136-148)
    pub fn mri_dot_i8(
        a: *const i8,
        b: *const i8,
        len: usize,
        out: *mut i32,
        stream: *mut c_void,
    ) -> mri_status;

    // matmul_int8 (int8.rs:61-98), and its per-row-scale form
    pub fn mri_matmul_int8(
        act_q: *const i8,
        act_q_len: usize,
        act_scale: f32,
        w: *const mri_qmatrix,
        m: usize,
        out: *mut f32,
        acc_out: *mut i32,
        stream: *mut c_void,
    ) -> mri_status;
    pub fn mri_matmul_int8_rows(
        act_q: *const i8,
        act_q_len: usize,
        act_scales: *const f32,
        w: *const mri_qmatrix,
        m: usize,
        out: *mut f32,
        acc_out: *mut i32,
        stream: *mut c_void,
    ) -> mri_status;
    // matmul_int8_from_f32 (int8.rs:113-143)
    pub fn mri_matmul_int8_from_f32(
        input: *const f32,
        dims: *const usize,
        ndim: usize,
        w: *const mri_qmatrix,
        out: *mut f32,
        act_q_out: *mut i8,
        act_scale_out: *mut f32,
        acc_out: *mut i32,
        stream: *mut c_void,
    ) -> mri_status;

    // matmul_q8_0_direct (q8_direct.rs:229-289); _exact keeps the block
    // order at every row count; _noalloc stages in a fixed device array
    pub fn mri_matmul_q8_0_direct(
        input: *const f32,
        dims: *const usize,
        ndim: usize,
        w: *const mri_q8_0_matrix,
        out: *mut f32,
        block_dots_out: *mut i32,
        act_scales_out: *mut f32,
        stream: *mut c_void,
    ) -> mri_status;
    pub fn mri_matmul_q8_0_direct_exact(
        input: *const f32,
        dims: *const usize,
        ndim: usize,
        w: *const mri_q8_0_matrix,
        out: *mut f32,
        block_dots_out: *mut i32,
        act_scales_out: *mut f32,
        stream: *mut c_void,
    ) -> mri_status;
    pub fn mri_matmul_q8_0_direct_noalloc(
        input: *const f32,
        dims: *const usize,
        ndim: usize,
        w: *const mri_q8_0_matrix,
        out: *mut f32,
        block_dots_out: *mut i32,
        act_scales_out: *mut f32,
        stream: *mut c_void,
    ) -> mri_status;

    // matmul_q4_0_dequant (q4_0.rs:94-181); weight_q4 is a device pointer
    pub fn mri_matmul_q4_0_dequant(
        input: *const f32,
        dims: *const usize,
        ndim: usize,
        weight_q4: *const u8,
        weight_len: usize,
        n_out: usize,
        k: usize,
        out: *mut f32,
        stream: *mut c_void,
    ) -> mri_status;

    // Q4_0 handles (order: mri_q4_order)
    pub fn mri_q4_0_matrix_from_raw_bytes(
        data: *const u8,
        len: usize,
        n_out: usize,
        k_in: usize,
        order: c_int,
        out: *mut *mut mri_q4_0_matrix,
    ) -> mri_status;
    pub fn mri_q4_0_matrix_from_raw_device(
        data_dev: *const u8,
        len: usize,
        n_out: usize,
        k_in: usize,
        order: c_int,
        stream: *mut c_void,
        out: *mut *mut mri_q4_0_matrix,
    ) -> mri_status;
    pub fn mri_q4_0_matrix_n_out(w: *const mri_q4_0_matrix) -> usize;
    pub fn mri_q4_0_matrix_k_in(w: *const mri_q4_0_matrix) -> usize;
    pub fn mri_q4_0_matrix_device_bytes(w: *const mri_q4_0_matrix) -> usize;
    pub fn mri_q4_0_matrix_destroy(w: *mut mri_q4_0_matrix);

    // matmul_q4_0_dequant (W4A32) on a Q4_0 handle
    pub fn mri_matmul_q4_0_dequant_matrix(
        input: *const f32,
        dims: *const usize,
        ndim: usize,
        w: *const mri_q4_0_matrix,
        out: *mut f32,
        stream: *mut c_void,
    ) -> mri_status;
    // W4A8 extension: matmul_q8_0_direct's arithmetic on Q4_0 quants
    pub fn mri_matmul_q4_0_w4a8(
        input: *const f32,
        dims: *const usize,
        ndim: usize,
        w: *const mri_q4_0_matrix,
        out: *mut f32,
        block_dots_out: *mut i32,
        act_scales_out: *mut f32,
        stream: *mut c_void,
    ) -> mri_status;
    // matmul_q4_0_dequant with the nibble order of weight_q4 given
    pub fn mri_matmul_q4_0_dequant_ordered(
        input: *const f32,
        dims: *const usize,
        ndim: usize,
        weight_q4: *const u8,
        weight_len: usize,
        n_out: usize,
        k: usize,
        order: c_int,
        out: *mut f32,
        stream: *mut c_void,
    ) -> mri_status;

    pub fn mri_synchronize(stream: *mut c_void) -> mri_status;

    // diagnostics without a reference counterpart
    pub fn mri_hbm_read(p: *const c_void, bytes: usize, sink: *mut i32, stream: *mut c_void)
        -> mri_status;
    pub fn mri_mfma_i8_peak(
        src: *const i8,
        iters: c_int,
        sink: *mut i32,
        n_cus: *mut c_int,
        stream: *mut c_void,
    ) -> mri_status;
}

// ---- include/mri_llama.h ---------------------------------------------------------

extern "C" {
    // LlamaModelInt8::new (forward_int8.rs:430-444); host f32 arrays
    pub fn mri_llama_create(
        cfg: *const mri_llama_config,
        token_embd: *const f32,
        output_norm: *const f32,
        output: mri_weight_ref,
        out: *mut *mut mri_llama,
    ) -> mri_status;
    // TransformerBlockInt8::new (forward_int8.rs:168-198); w points at 7
    // weights: wq, wk, wv, wo, wgate, wup, wdown
    pub fn mri_llama_set_layer(
        model: *mut mri_llama,
        layer: usize,
        attn_norm: *const f32,
        ffn_norm: *const f32,
        w: *const mri_weight_ref,
    ) -> mri_status;
    pub fn mri_llama_destroy(model: *mut mri_llama);

    // KvCache::new (cache/kv_cache.rs:65)
    pub fn mri_kv_cache_create(
        n_layers: usize,
        max_seq: usize,
        n_kv_heads: usize,
        head_dim: usize,
        out: *mut *mut mri_kv_cache,
    ) -> mri_status;
    pub fn mri_kv_cache_destroy(cache: *mut mri_kv_cache);

    // forward_cached (forward_int8.rs:207-216, 516-529); tokens are host ids
    pub fn mri_llama_forward_cached(
        model: *mut mri_llama,
        tokens: *const u32,
        n: usize,
        start_pos: usize,
        cache: *mut mri_kv_cache,
        logits: *mut f32,
        stream: *mut c_void,
    ) -> mri_status;
    // forward_decode (forward_int8.rs:538-546)
    pub fn mri_llama_forward_decode(
        model: *mut mri_llama,
        token: u32,
        pos: usize,
        cache: *mut mri_kv_cache,
        logits: *mut f32,
        stream: *mut c_void,
    ) -> mri_status;
    // prefill, then greedy decode steps (sampling/mod.rs:144-151); prompt and
    // tokens_out are host arrays, logits_out a device buffer (nullable)
    pub fn mri_llama_generate_greedy(
        model: *mut mri_llama,
        prompt: *const u32,
        n_prompt: usize,
        n_steps: usize,
        cache: *mut mri_kv_cache,
        tokens_out: *mut u32,
        logits_out: *mut f32,
        stream: *mut c_void,
    ) -> mri_status;
    // argmax per row (sampling/mod.rs:144-151)
    pub fn mri_argmax(
        v: *const f32,
        rows: usize,
        n: usize,
        idx: *mut u32,
        stream: *mut c_void,
    ) -> mri_status;
}

// ---- HIP runtime, for the device buffers a safe layer owns --------------------------

/// The few HIP runtime entry points a safe wrapper needs to own device
/// buffers (`libamdhip64.so`); `kind` of `hipMemcpy`: 1 host to device,
/// 2 device to host.
pub mod hip {
    use core::ffi::{c_int, c_void};
    pub const HIP_MEMCPY_HOST_TO_DEVICE: c_int = 1;
    pub const HIP_MEMCPY_DEVICE_TO_HOST: c_int = 2;
    extern "C" {
        pub fn hipMalloc(ptr: *mut *mut c_void, bytes: usize) -> c_int;
        pub fn hipFree(ptr: *mut c_void) -> c_int;
        pub fn hipMemcpy(dst: *mut c_void, src: *const c_void, bytes: usize, kind: c_int)
            -> c_int;
        pub fn hipDeviceSynchronize() -> c_int;
    }
}

/// The thread-local message of the last non-OK status on this thread.
pub fn last_error() -> String {
    // SAFETY: mri_last_error returns a NUL-terminated string owned by the
    // library (thread-local), valid until the next call on this thread.
    unsafe {
        let p = mri_last_error();
        if p.is_null() {
            String::new()
        } else {
            std::ffi::CStr::from_ptr(p).to_string_lossy().into_owned()
        }
    }
}

/// `MRI_OK` as `Ok(())`, any other status as `Err((status, message))`.
pub fn check(st: mri_status) -> Result<(), (mri_status, String)> {
    if st == MRI_OK {
        Ok(())
    } else {
        Err((st, last_error()))
    }
}
