// model.cpp — LlamaModelInt8 on the GPU (include/mri_llama.h).
//
// Host-side orchestration of one forward pass: every step is a kernel (or a
// quantized projection entry point) enqueued on the caller's stream over
// activation buffers that the model handle owns, sized for max_seq rows.
// Nothing is copied back to the host except the generated token ids at the
// end of mri_llama_generate_greedy.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <string>
#include <vector>

#include "common.hpp"
#include "mri_llama.h"

struct mri_kv_cache {
    size_t n_layers = 0, max_seq = 0, kvd = 0;
    float *k = nullptr, *v = nullptr;  // [n_layers][max_seq][kvd]
};

namespace {

struct Layer {
    float *attn_norm = nullptr, *ffn_norm = nullptr;
    mri_weight_ref w[7] = {};
    // Row concatenations [wq; wk; wv] and [wgate; wup], owned by the model
    // (format 0 / null ptr when the parts cannot be fused).
    mri_weight_ref qkv{}, gu{};
    bool set = false;
};

}  // namespace

struct mri_llama {
    mri_llama_config cfg{};
    size_t hd = 0, qd = 0, kvd = 0;
    float *embd = nullptr, *out_norm = nullptr;
    mri_weight_ref output{};
    std::vector<Layer> layers;
    float *cos_t = nullptr, *sin_t = nullptr;  // [max_seq][hd/2]
    // activations for up to max_seq rows; qkv holds q, k and v (rows of
    // [q | k | v] when the projection is fused, else three row-major blocks),
    // gu likewise holds gate and up
    float *x = nullptr, *normed = nullptr, *tmp = nullptr, *qkv = nullptr, *attn = nullptr,
          *gu = nullptr, *act = nullptr;
    uint32_t *tok = nullptr;      // prompt ids [max_seq]
    uint32_t *gen = nullptr;      // generated ids [max_seq + 1]
    float *attn_part = nullptr;   // split-key decode attention partials
    float *logits_buf = nullptr;  // prefill logits for generation, grown on demand
    size_t logits_rows = 0;
    // Rows path with fused RMSNorm (fuse_norm): the RMSNorm that feeds the
    // next projections is kept as statistics (nstats: rms_inv and max |y|
    // per row) over x with weights norm_w; each projection quantizes the
    // normalized rows straight from x into qact / qscale (qform: the form
    // held there, -1 none), so the normalized f32 rows are not stored.
    bool fuse_norm = false;
    float *nstats = nullptr, *qscale = nullptr;
    int8_t *qact = nullptr;
    const float *norm_w = nullptr;
    int qform = -1;
    size_t qld = 0;
    int row_path = -1;            // decode rows take the folded path (-1: not yet known)
    // A decode row whose token is still the previous step's argmax keys: the
    // block's first projection reduces them, reads that embedding row and
    // copies it into x (RowOps in_keys); set by run_rows for one block call.
    const unsigned long long *in_keys = nullptr;
    int n_in_keys = 0;
    uint32_t *tok_out = nullptr;
    std::vector<void *> allocs;
};

namespace mri {
mri_status current_device(int *dev);
}

namespace {

using namespace mri;

std::string fmt_err(const char *f, size_t a, size_t b = 0, size_t c = 0) {
    char buf[256];
    snprintf(buf, sizeof buf, f, a, b, c);
    return buf;
}

#define TRY(call)                              \
    do {                                       \
        const mri_status _st = (call);         \
        if (_st != MRI_OK) return _st;         \
    } while (0)

mri_status dalloc(mri_llama *m, size_t bytes, void **p) {
    MRI_HIP(hipMalloc(p, bytes ? bytes : 4));
    m->allocs.push_back(*p);
    return MRI_OK;
}

template <typename T>
mri_status dalloc_t(mri_llama *m, size_t count, T **p) {
    void *v = nullptr;
    mri_status st = dalloc(m, count * sizeof(T), &v);
    *p = static_cast<T *>(v);
    return st;
}

// Shape and handle checks of one projection weight.
mri_status check_weight(const mri_weight_ref &w, size_t n_out, size_t k_in, const char *role) {
    if (!w.ptr) return set_error(MRI_ERR_INVALID_ARGUMENT, std::string(role) + ": null weight");
    if (w.n_out != n_out || w.k_in != k_in)
        return set_error(MRI_ERR_INVALID_SHAPE,
                         std::string(role) + fmt_err(": weight is [%zu, %zu], expected [%zu, ",
                                                     w.n_out, w.k_in, n_out) +
                             std::to_string(k_in) + "]");
    switch (w.format) {
    case MRI_WEIGHT_INT8: {
        auto *h = static_cast<const mri_qmatrix *>(w.ptr);
        if (mri_qmatrix_n_out(h) != n_out || mri_qmatrix_k_in(h) != k_in)
            return set_error(MRI_ERR_INVALID_SHAPE, std::string(role) + ": handle shape differs");
        return MRI_OK;
    }
    case MRI_WEIGHT_Q8_0: {
        auto *h = static_cast<const mri_q8_0_matrix *>(w.ptr);
        if (mri_q8_0_matrix_n_out(h) != n_out || mri_q8_0_matrix_k_in(h) != k_in)
            return set_error(MRI_ERR_INVALID_SHAPE, std::string(role) + ": handle shape differs");
        return MRI_OK;
    }
    case MRI_WEIGHT_Q4_0:
        if (k_in % 32)
            return set_error(MRI_ERR_INVALID_SHAPE,
                             std::string(role) + ": Q4_0 k_in must be a multiple of 32");
        return MRI_OK;
    case MRI_WEIGHT_Q4_0_W4A8: {
        auto *h = static_cast<const mri_q4_0_matrix *>(w.ptr);
        if (mri_q4_0_matrix_n_out(h) != n_out || mri_q4_0_matrix_k_in(h) != k_in)
            return set_error(MRI_ERR_INVALID_SHAPE, std::string(role) + ": handle shape differs");
        return MRI_OK;
    }
    default:
        return set_error(MRI_ERR_INVALID_ARGUMENT, std::string(role) + ": unknown weight format");
    }
}

void release_fused(mri_weight_ref &w) {
    if (w.ptr && w.format == MRI_WEIGHT_INT8)
        mri_qmatrix_destroy(static_cast<mri_qmatrix *>(const_cast<void *>(w.ptr)));
    else if (w.ptr && w.format == MRI_WEIGHT_Q8_0)
        mri_q8_0_matrix_destroy(static_cast<mri_q8_0_matrix *>(const_cast<void *>(w.ptr)));
    else if (w.ptr && w.format == MRI_WEIGHT_Q4_0_W4A8)
        mri_q4_0_matrix_destroy(static_cast<mri_q4_0_matrix *>(const_cast<void *>(w.ptr)));
    w = mri_weight_ref{};
}

// The row concatenation of parts that share one input (q/k/v, gate/up): the
// fused projection's output row is [part 0 | part 1 | ...] and every element
// equals that of the separate projection, because the parts see the same
// activations and the same activation quantization.  W4A32 Q4_0 weights
// (raw bytes, no handle), mixed formats and parts that are not whole 16-row
// tiles stay separate (*out left empty).
mri_status fuse(const mri_weight_ref *parts, int n, mri_weight_ref *out) {
    *out = mri_weight_ref{};
    size_t rows = 0;
    for (int i = 0; i < n; ++i) {
        if (parts[i].format != parts[0].format || parts[i].n_out % 16) return MRI_OK;
        rows += parts[i].n_out;
    }
    void *h = nullptr;
    if (parts[0].format == MRI_WEIGHT_INT8) {
        const mri_qmatrix *p[3];
        for (int i = 0; i < n; ++i) p[i] = static_cast<const mri_qmatrix *>(parts[i].ptr);
        mri_qmatrix *f = nullptr;
        TRY(concat_qmatrix(p, n, nullptr, &f));
        h = f;
    } else if (parts[0].format == MRI_WEIGHT_Q8_0) {
        const mri_q8_0_matrix *p[3];
        for (int i = 0; i < n; ++i) p[i] = static_cast<const mri_q8_0_matrix *>(parts[i].ptr);
        mri_q8_0_matrix *f = nullptr;
        TRY(concat_q8_0_matrix(p, n, nullptr, &f));
        h = f;
    } else if (parts[0].format == MRI_WEIGHT_Q4_0_W4A8) {
        const mri_q4_0_matrix *p[3];
        for (int i = 0; i < n; ++i) p[i] = static_cast<const mri_q4_0_matrix *>(parts[i].ptr);
        mri_q4_0_matrix *f = nullptr;
        TRY(concat_q4_0_matrix(p, n, nullptr, &f));
        h = f;
    } else {
        return MRI_OK;
    }
    *out = mri_weight_ref{parts[0].format, h, rows, parts[0].k_in};
    const hipError_t e = hipStreamSynchronize(nullptr);
    if (e != hipSuccess) {
        release_fused(*out);
        return hip_error(e, "fuse");
    }
    return MRI_OK;
}

// out[rows, n_out] = in[rows, k_in] projected by w (forward_int8.rs:72-74).
mri_status proj(const mri_weight_ref &w, const float *in, size_t rows, float *out,
                hipStream_t s) {
    const size_t dims[2] = {rows, w.k_in};
    switch (w.format) {
    case MRI_WEIGHT_INT8:
        return mri_matmul_int8_from_f32(in, dims, 2, static_cast<const mri_qmatrix *>(w.ptr), out,
                                        nullptr, nullptr, nullptr, s);
    case MRI_WEIGHT_Q8_0:
        return mri_matmul_q8_0_direct(in, dims, 2, static_cast<const mri_q8_0_matrix *>(w.ptr),
                                      out, nullptr, nullptr, s);
    case MRI_WEIGHT_Q4_0_W4A8:
        return mri_matmul_q4_0_w4a8(in, dims, 2, static_cast<const mri_q4_0_matrix *>(w.ptr),
                                    out, nullptr, nullptr, s);
    default:
        return mri_matmul_q4_0_dequant(in, dims, 2, static_cast<const uint8_t *>(w.ptr),
                                       w.n_out * (w.k_in / 32) * 18, w.n_out, w.k_in, out, s);
    }
}

// The projection of the rows RMS-normalized by the statistics in m->nstats
// (fused path): the activations are quantized from m->x in the form the
// weight's entry point uses (INT8: one scale over all rows, packed for the
// GEMM from kGemmMinRows rows; Q8_0 / W4A8: a scale per row; Q4_0: the f32
// rows themselves), once per form while the statistics stay the same.
mri_status proj_normed(mri_llama *m, const mri_weight_ref &w, size_t rows, float *out,
                       hipStream_t s) {
    const size_t d = m->cfg.dim;
    auto prepare = [&](int form, size_t ld) -> mri_status {
        if (m->qform == form && m->qld == ld) return MRI_OK;
        TRY(launch_norm_quant(form, m->x, m->norm_w, m->nstats, rows, d, ld, m->qact, m->qscale,
                              m->normed, s));
        m->qform = form;
        m->qld = ld;
        return MRI_OK;
    };
    switch (w.format) {
    case MRI_WEIGHT_INT8: {
        const QMatrixDev &dv = handle_dev(static_cast<const mri_qmatrix *>(w.ptr));
        if (dv.n_out == 0) return MRI_OK;
        const bool gemm = rows >= kGemmMinRows;
        TRY(prepare(gemm ? 0 : 1, dv.kp));
        if (!gemm) return run_int8(m->qact, rows, m->qscale, 0, 0.0f, dv, out, nullptr, s);
        void *ws = nullptr;
        if (const size_t wsb = gemm_ws_bytes(rows, dv)) TRY(gemm_ws_get(s, wsb, &ws));
        return launch_gemm_int8(m->qact, rows, m->qscale, 0, 0.0f, dv, out, nullptr, ws, s);
    }
    case MRI_WEIGHT_Q8_0:
    case MRI_WEIGHT_Q4_0_W4A8: {
        const Q8MatrixDev &dv =
            w.format == MRI_WEIGHT_Q8_0 ? handle_dev(static_cast<const mri_q8_0_matrix *>(w.ptr))
                                        : handle_dev(static_cast<const mri_q4_0_matrix *>(w.ptr));
        if (dv.n_out == 0) return MRI_OK;
        TRY(prepare(2, dv.kp));
        return run_q8(m->qact, rows, m->qscale, dv, out, nullptr, s);
    }
    default:
        TRY(prepare(3, d));
        return proj(w, m->normed, rows, out, s);
    }
}

// One decode row through the single-row GEMV, with the steps around the
// projection that it takes over (RowOps): the RMSNorm or SwiGLU that
// produces its input, a copy of the input row, and the residual add of its
// output.  row_proj_ok: the GEMV takes the weight.
bool row_proj_ok(const mri_weight_ref &w) {
    if (w.k_in == 0 || w.k_in % 4 || w.n_out == 0) return false;
    switch (w.format) {
    case MRI_WEIGHT_INT8: {
        const QMatrixDev &d = handle_dev(static_cast<const mri_qmatrix *>(w.ptr));
        return gemv_int8_supported(true, 1, d.n_tiles, d.k_in, d.kp);
    }
    case MRI_WEIGHT_Q8_0: {
        const Q8MatrixDev &d = handle_dev(static_cast<const mri_q8_0_matrix *>(w.ptr));
        return gemv_q8_supported(true, 1, d.n_tiles, d.k_in, d.kp);
    }
    case MRI_WEIGHT_Q4_0_W4A8: {
        const Q8MatrixDev &d = handle_dev(static_cast<const mri_q4_0_matrix *>(w.ptr));
        return gemv_q8_supported(true, 1, d.n_tiles, d.k_in, d.kp);
    }
    default:
        return false;
    }
}

mri_status row_proj(const mri_weight_ref &w, const float *in, const RowOps &ops, float *out,
                    hipStream_t s) {
    switch (w.format) {
    case MRI_WEIGHT_INT8:
        return launch_gemv_int8(in, nullptr, 1, nullptr, 0, 0.0f,
                                handle_dev(static_cast<const mri_qmatrix *>(w.ptr)), out,
                                nullptr, nullptr, nullptr, s, ops);
    case MRI_WEIGHT_Q8_0:
        return launch_gemv_q8_0(in, nullptr, 1, nullptr,
                                handle_dev(static_cast<const mri_q8_0_matrix *>(w.ptr)), out,
                                nullptr, nullptr, s, ops);
    case MRI_WEIGHT_Q4_0_W4A8:
        return launch_gemv_q8_0(in, nullptr, 1, nullptr,
                                handle_dev(static_cast<const mri_q4_0_matrix *>(w.ptr)), out,
                                nullptr, nullptr, s, ops);
    default:
        return set_error(MRI_ERR_INVALID_ARGUMENT, "row projection: unsupported format");
    }
}

// Whether a decode row can run every projection of the model through
// row_proj (cached until a layer changes).
bool row_path(mri_llama *m) {
    if (m->row_path >= 0) return m->row_path != 0;
    bool ok = row_proj_ok(m->output);
    for (const Layer &L : m->layers) {
        if (L.qkv.ptr) ok = ok && row_proj_ok(L.qkv);
        else ok = ok && row_proj_ok(L.w[0]) && row_proj_ok(L.w[1]) && row_proj_ok(L.w[2]);
        if (L.gu.ptr) ok = ok && row_proj_ok(L.gu);
        else ok = ok && row_proj_ok(L.w[4]) && row_proj_ok(L.w[5]);
        ok = ok && row_proj_ok(L.w[3]) && row_proj_ok(L.w[6]);
    }
    m->row_path = ok ? 1 : 0;
    return ok;
}

// TransformerBlockInt8::forward_cached (forward_int8.rs:207-216): attention
// sublayer (:291-323) and FFN sublayer (:350-357).  m->x holds the residual
// stream.  Rows path (fold false): on entry m->normed holds the block's
// attention RMSNorm; on exit m->normed holds the RMSNorm of the output with
// next_norm (the next block's attention norm, or the output norm), each
// residual add fused with the RMSNorm that follows it.  Decode row (fold):
// each RMSNorm runs in the prologue of the projection that reads it and
// each residual add in the epilogue of the projection that feeds it
// (row_proj); x_in is the block's input row (m->x, or the embedding row of
// the first block, which the first projection copies into m->x).  Either
// way the values are those of the separate steps.
mri_status block(mri_llama *m, size_t li, size_t rows, size_t start, mri_kv_cache *c,
                 const float *next_norm, bool fold, const float *x_in, hipStream_t s) {
    const mri_llama_config &g = m->cfg;
    const Layer &L = m->layers[li];
    // projections of a normalized row (fold: normalized in the GEMV from
    // xrow, the attention input and then the residual stream)
    const float *xrow = x_in;
    bool copy_x = fold && x_in != m->x;
    // the first projection of the block copies the row it reads into x (and,
    // with in_keys, first finds it from the previous step's argmax keys);
    // the later ones read x
    auto norm_ops = [&](const float *norm) {
        RowOps o;
        o.norm_w = norm;
        o.eps = g.eps;
        if (copy_x) {
            o.x_out = m->x;
            o.in_keys = m->in_keys;
            o.n_in_keys = m->n_in_keys;
            o.tok_out = m->tok_out;
            m->in_keys = nullptr;
            m->tok_out = nullptr;
        }
        copy_x = false;
        return o;
    };
    // (silu_n: one row's leading output channels stored as their SiLU)
    auto in_proj = [&](const mri_weight_ref &w, const float *norm, float *out, int silu_n = 0) {
        if (!fold) return m->fuse_norm ? proj_normed(m, w, rows, out, s)
                                       : proj(w, m->normed, rows, out, s);
        RowOps o = norm_ops(norm);
        o.silu_n = silu_n;
        const float *src = xrow;
        if (o.in_keys) xrow = m->x;
        return row_proj(w, src, o, out, s);
    };
    // rows path: m->tmp (a projection's output) added to the residual stream,
    // fused with the RMSNorm that follows
    auto out_tail = [&](const float *norm) {
        if (m->fuse_norm) {
            m->norm_w = norm;
            m->qform = -1;
            return launch_rmsnorm_stats(2, m->x, m->tmp, nullptr, m->x, rows, g.dim, norm, g.eps,
                                        m->nstats, s);
        }
        return launch_add_rmsnorm(m->x, m->tmp, rows, g.dim, norm, g.eps, m->normed, s);
    };
    // projections whose output is added to the residual stream
    // (up: in is the SiLU of a SwiGLU gate row, multiplied by up in the
    // projection; one row only)
    auto out_proj = [&](const mri_weight_ref &w, const float *in, const float *norm,
                        const float *up = nullptr) {
        if (fold) {
            RowOps o;
            o.accum = true;
            o.up = up;
            return row_proj(w, in, o, m->x, s);
        }
        TRY(proj(w, in, rows, m->tmp, s));
        return out_tail(norm);
    };
    float *kc = c->k + li * c->max_seq * c->kvd, *vc = c->v + li * c->max_seq * c->kvd;
    float *q, *k, *v;
    size_t qs, kvs;
    if (fold) {
        // q/k/v of one row with RoPE and the KV-cache writes in the GEMV
        // epilogue (what k_rope_qkv does for rows)
        if (m->hd % 2 || m->hd > 128)
            return set_error(MRI_ERR_UNSUPPORTED, "rope: head_dim must be even and <= 128");
        const size_t half = m->hd / 2;
        float *krow = kc + start * c->kvd, *vrow = vc + start * c->kvd;
        RowOps o = norm_ops(L.attn_norm);
        o.rope_cos = m->cos_t + start * half;
        o.rope_sin = m->sin_t + start * half;
        o.hd = (int)m->hd;
        q = m->qkv;
        qs = m->qd;
        if (L.qkv.ptr) {
            o.rope_n = (int)(m->qd + m->kvd);
            o.seg1 = (int)m->qd;
            o.out1 = krow;
            o.seg2 = (int)(m->qd + m->kvd);
            o.out2 = vrow;
            TRY(row_proj(L.qkv, xrow, o, q, s));
        } else {
            RowOps ok = o, ov = o;
            ok.x_out = ov.x_out = nullptr;  // copied by the first
            ok.in_keys = ov.in_keys = nullptr;
            ok.tok_out = ov.tok_out = nullptr;
            o.rope_n = (int)m->qd;
            TRY(row_proj(L.w[0], xrow, o, q, s));
            if (o.in_keys) xrow = m->x;  // the row the first found and copied
            ok.rope_n = (int)m->kvd;
            TRY(row_proj(L.w[1], xrow, ok, krow, s));
            ov.rope_n = 0;
            TRY(row_proj(L.w[2], xrow, ov, vrow, s));
        }
    } else if (L.qkv.ptr) {
        TRY(in_proj(L.qkv, L.attn_norm, m->qkv));
        q = m->qkv;
        k = q + m->qd;
        v = k + m->kvd;
        qs = kvs = m->qd + 2 * m->kvd;
    } else {
        q = m->qkv;
        k = q + rows * m->qd;
        v = k + rows * m->kvd;
        qs = m->qd;
        kvs = m->kvd;
        TRY(in_proj(L.w[0], L.attn_norm, q));
        TRY(in_proj(L.w[1], L.attn_norm, k));
        TRY(in_proj(L.w[2], L.attn_norm, v));
    }
    if (!fold)
        TRY(launch_rope_qkv(q, k, v, rows, g.n_heads, g.n_kv_heads, m->hd, qs, kvs, m->cos_t,
                            m->sin_t, start, kc, vc, s));
    TRY(launch_attention(q, qs, rows, kc, vc, g.n_heads, g.n_kv_heads, m->hd, start, m->attn,
                         m->attn_part, s));
    TRY(out_proj(L.w[3], m->attn, L.ffn_norm));
    xrow = m->x;
    // gate rows, then up rows (one row: the gate projection stores the SiLU
    // of its outputs, and the down projection's prologue multiplies by up)
    if (L.gu.ptr) TRY(in_proj(L.gu, L.ffn_norm, m->gu, (int)g.ffn_dim));
    else {
        TRY(in_proj(L.w[4], L.ffn_norm, m->gu, (int)g.ffn_dim));
        TRY(in_proj(L.w[5], L.ffn_norm, m->gu + rows * g.ffn_dim));
    }
    if (fold) return out_proj(L.w[6], m->gu, next_norm, m->gu + g.ffn_dim);
    float *act = m->gu;
    const mri_weight_ref &wd = L.w[6];
    if (L.gu.ptr && (wd.format == MRI_WEIGHT_Q8_0 || wd.format == MRI_WEIGHT_Q4_0_W4A8)) {
        // Q8_0 / W4A8 down projection: the SwiGLU rows are quantized as they
        // are formed (the rows, scales and products of launch_swiglu_rows
        // followed by matmul_q8_0_direct's own per-row quantization)
        const Q8MatrixDev &dv =
            wd.format == MRI_WEIGHT_Q8_0 ? handle_dev(static_cast<const mri_q8_0_matrix *>(wd.ptr))
                                         : handle_dev(static_cast<const mri_q4_0_matrix *>(wd.ptr));
        if (dv.k_in != g.ffn_dim)
            return set_error(MRI_ERR_SHAPE_MISMATCH, "down projection: k_in != ffn_dim");
        if (dv.n_out) {
            TRY(launch_swiglu_quantize_rows(m->gu, rows, g.ffn_dim, dv.kp, true, m->qact,
                                            m->qscale, s));
            m->qform = -1;  // qact no longer holds the normalized rows
            TRY(run_q8(m->qact, rows, m->qscale, dv, m->tmp, nullptr, s));
        }
        return out_tail(next_norm);
    }
    if (L.gu.ptr) {
        act = m->act;
        TRY(launch_swiglu_rows(m->gu, rows, g.ffn_dim, act, s));
    } else {
        TRY(launch_swiglu(act, m->gu + rows * g.ffn_dim, rows * g.ffn_dim, act, s));
    }
    return out_proj(L.w[6], act, next_norm);
}

// embed -> blocks -> rmsnorm -> output projection for `rows` token ids
// already on the device.
// Where a single folded row's embedding comes from: gathered from the ids
// on the device (kDevice), read in place at an id the host knows (kHost),
// already in m->x (kInX, written by the previous step's argmax), or read in
// place at the id the first projection finds in the previous step's argmax
// keys (kKeys: m->in_keys, which the caller sets; needs a layer).
enum class Emb { kDevice, kHost, kInX, kKeys };

// arg: for a folded row, the greedy argmax (and next embedding row) that the
// output projection's epilogue computes (the RowOps arg_* fields).
mri_status run_rows(mri_llama *m, const uint32_t *tok_dev, size_t rows, size_t start,
                    mri_kv_cache *c, float *logits, hipStream_t s, Emb emb = Emb::kDevice,
                    uint32_t host_tok = 0, const RowOps *arg = nullptr) {
    const mri_llama_config &g = m->cfg;
    const bool fold = rows == 1 && row_path(m);
    const float *first = g.n_layers ? m->layers[0].attn_norm : m->out_norm;
    const float *x_in = m->x;
    if (fold && emb == Emb::kHost) x_in = m->embd + (size_t)host_tok * g.dim;
    else if (fold && emb == Emb::kKeys && g.n_layers) x_in = m->embd;  // row found in-kernel
    else if (fold && emb == Emb::kInX) {}
    else if (fold) TRY(launch_embed(m->embd, tok_dev, 1, g.dim, m->x, s));
    else if (m->fuse_norm) {
        m->norm_w = first;
        m->qform = -1;
        TRY(launch_rmsnorm_stats(1, m->embd, nullptr, tok_dev, m->x, rows, g.dim, first, g.eps,
                                 m->nstats, s));
    } else {
        TRY(launch_embed_rmsnorm(m->embd, tok_dev, rows, g.dim, first, g.eps, m->x, m->normed, s));
    }
    for (size_t li = 0; li < g.n_layers; ++li)
        TRY(block(m, li, rows, start, c,
                  li + 1 < g.n_layers ? m->layers[li + 1].attn_norm : m->out_norm, fold,
                  li == 0 ? x_in : m->x, s));
    if (!fold)
        return m->fuse_norm ? proj_normed(m, m->output, rows, logits, s)
                            : proj(m->output, m->normed, rows, logits, s);
    RowOps o;
    o.norm_w = m->out_norm;
    o.eps = g.eps;
    if (arg) o.arg_keys = arg->arg_keys;
    return row_proj(m->output, g.n_layers ? m->x : x_in, o, logits, s);
}

mri_status check_run(mri_llama *m, size_t n, size_t start, mri_kv_cache *c) {
    if (!m || !c) return set_error(MRI_ERR_INVALID_ARGUMENT, "null model or cache");
    for (size_t li = 0; li < m->cfg.n_layers; ++li)
        if (!m->layers[li].set)
            return set_error(MRI_ERR_INVALID_ARGUMENT, fmt_err("layer %zu is not set", li));
    if (c->n_layers != m->cfg.n_layers || c->kvd != m->kvd)
        return set_error(MRI_ERR_SHAPE_MISMATCH, "KV cache shape does not match the model");
    if (n == 0) return set_error(MRI_ERR_INVALID_SHAPE, "forward: token list must not be empty");
    const size_t cap = std::min(c->max_seq, m->cfg.max_seq);
    if (start + n > cap)
        return set_error(MRI_ERR_INVALID_SHAPE,
                         fmt_err("positions %zu..%zu exceed the cache / RoPE length %zu", start,
                                 start + n - 1, cap));
    return MRI_OK;
}

mri_status check_tokens(const mri_llama *m, const uint32_t *tokens, size_t n) {
    if (!tokens) return set_error(MRI_ERR_INVALID_ARGUMENT, "null token list");
    for (size_t i = 0; i < n; ++i)
        if (tokens[i] >= m->cfg.vocab)
            return set_error(MRI_ERR_INVALID_SHAPE,
                             fmt_err("token id %zu >= vocab_size %zu", tokens[i], m->cfg.vocab));
    return MRI_OK;
}

}  // namespace

extern "C" {

mri_status mri_llama_create(const mri_llama_config *cfg, const float *token_embd,
                            const float *output_norm, mri_weight_ref output, mri_llama **out) {
    if (!cfg || !out || !token_embd || !output_norm)
        return set_error(MRI_ERR_INVALID_ARGUMENT, "null argument");
    *out = nullptr;
    const mri_llama_config g = *cfg;
    if (!g.dim || !g.n_heads || !g.n_kv_heads || !g.vocab || !g.max_seq || !g.ffn_dim)
        return set_error(MRI_ERR_INVALID_SHAPE, "llama: zero dimension");
    if (g.dim % g.n_heads || g.n_heads % g.n_kv_heads || (g.dim / g.n_heads) % 2)
        return set_error(MRI_ERR_INVALID_SHAPE,
                         "llama: dim % n_heads, n_heads % n_kv_heads and head_dim % 2 must be 0");
    const size_t hd = g.dim / g.n_heads;
    if (!attention_supported(hd))
        return set_error(MRI_ERR_UNSUPPORTED, "llama: head_dim must be 64 or 128");
    int dev;
    mri_status st = current_device(&dev);
    if (st) return st;
    TRY(check_weight(output, g.vocab, g.dim, "output"));
    auto *m = new mri_llama();
    m->cfg = g;
    m->hd = hd;
    m->qd = g.n_heads * hd;
    m->kvd = g.n_kv_heads * hd;
    m->output = output;
    m->layers.resize(g.n_layers);
    auto fail = [&](mri_status e) {
        mri_llama_destroy(m);
        return e;
    };
    const size_t R = g.max_seq;
    if ((st = dalloc_t(m, g.vocab * g.dim, &m->embd)) || (st = dalloc_t(m, g.dim, &m->out_norm)) ||
        (st = dalloc_t(m, R * hd / 2, &m->cos_t)) || (st = dalloc_t(m, R * hd / 2, &m->sin_t)) ||
        (st = dalloc_t(m, R * g.dim, &m->x)) || (st = dalloc_t(m, R * g.dim, &m->normed)) ||
        (st = dalloc_t(m, R * g.dim, &m->tmp)) ||
        (st = dalloc_t(m, R * (m->qd + 2 * m->kvd), &m->qkv)) ||
        (st = dalloc_t(m, R * m->qd, &m->attn)) || (st = dalloc_t(m, R * 2 * g.ffn_dim, &m->gu)) ||
        (st = dalloc_t(m, R * g.ffn_dim, &m->act)) || (st = dalloc_t(m, R, &m->tok)) ||
        (st = dalloc_t(m, 2 * R, &m->nstats)) || (st = dalloc_t(m, R, &m->qscale)) ||
        (st = dalloc_t(m, round_up(R, 32) * round_up(std::max(g.dim, g.ffn_dim), 256),
                       &m->qact)) ||
        (st = dalloc_t(m, R + 1, &m->gen)) ||
        (st = dalloc_t(m, attention_part_floats(g.n_heads, hd, R), &m->attn_part)))
        return fail(st);
    // the decode attention's per-head counters start at zero
    if (const hipError_t e =
            hipMemset(m->attn_part, 0, attention_part_floats(g.n_heads, hd, R) * sizeof(float)))
        return fail(hip_error(e, "hipMemset(attention workspace)"));
    m->fuse_norm = rmsnorm_stats_supported(g.dim);
    // RopeTable::new (ops/rope.rs): theta_i = 1 / base^(2i / head_dim) and
    // angle = pos * theta_i in f32, with the C library's powf / cosf / sinf.
    const size_t half = hd / 2;
    std::vector<float> ct(R * half), stb(R * half);
    for (size_t pos = 0; pos < R; ++pos)
        for (size_t i = 0; i < half; ++i) {
            const float e = (2.0f * (float)i) / (float)hd;
            const float theta = 1.0f / powf(g.rope_base, e);
            const float angle = (float)pos * theta;
            ct[pos * half + i] = cosf(angle);
            stb[pos * half + i] = sinf(angle);
        }
    hipError_t e;
    if ((e = hipMemcpy(m->cos_t, ct.data(), ct.size() * 4, hipMemcpyHostToDevice)) ||
        (e = hipMemcpy(m->sin_t, stb.data(), stb.size() * 4, hipMemcpyHostToDevice)) ||
        (e = hipMemcpy(m->embd, token_embd, g.vocab * g.dim * 4, hipMemcpyHostToDevice)) ||
        (e = hipMemcpy(m->out_norm, output_norm, g.dim * 4, hipMemcpyHostToDevice)))
        return fail(hip_error(e, "llama_create upload"));
    *out = m;
    return MRI_OK;
}

mri_status mri_llama_set_layer(mri_llama *m, size_t li, const float *attn_norm,
                               const float *ffn_norm, const mri_weight_ref w[7]) {
    if (!m || !attn_norm || !ffn_norm || !w)
        return set_error(MRI_ERR_INVALID_ARGUMENT, "null argument");
    if (li >= m->cfg.n_layers)
        return set_error(MRI_ERR_INVALID_ARGUMENT,
                         fmt_err("layer %zu of %zu", li, m->cfg.n_layers));
    const mri_llama_config &g = m->cfg;
    static const char *kRole[7] = {"wq", "wk", "wv", "wo", "wgate", "wup", "wdown"};
    const size_t shp[7][2] = {{m->qd, g.dim},      {m->kvd, g.dim},     {m->kvd, g.dim},
                              {g.dim, m->qd},      {g.ffn_dim, g.dim},  {g.ffn_dim, g.dim},
                              {g.dim, g.ffn_dim}};
    for (int i = 0; i < 7; ++i) TRY(check_weight(w[i], shp[i][0], shp[i][1], kRole[i]));
    Layer &L = m->layers[li];
    if (!L.attn_norm) {
        TRY(dalloc_t(m, g.dim, &L.attn_norm));
        TRY(dalloc_t(m, g.dim, &L.ffn_norm));
    }
    MRI_HIP(hipMemcpy(L.attn_norm, attn_norm, g.dim * 4, hipMemcpyHostToDevice));
    MRI_HIP(hipMemcpy(L.ffn_norm, ffn_norm, g.dim * 4, hipMemcpyHostToDevice));
    for (int i = 0; i < 7; ++i) L.w[i] = w[i];
    release_fused(L.qkv);
    release_fused(L.gu);
    L.set = false;
    m->row_path = -1;
    TRY(fuse(w, 3, &L.qkv));
    TRY(fuse(w + 4, 2, &L.gu));
    L.set = true;
    return MRI_OK;
}

void mri_llama_destroy(mri_llama *m) {
    if (!m) return;
    for (Layer &L : m->layers) {
        release_fused(L.qkv);
        release_fused(L.gu);
    }
    for (void *p : m->allocs) (void)hipFree(p);
    if (m->logits_buf) (void)hipFree(m->logits_buf);
    delete m;
}

mri_status mri_kv_cache_create(size_t n_layers, size_t max_seq, size_t n_kv_heads,
                               size_t head_dim, mri_kv_cache **out) {
    if (!out) return set_error(MRI_ERR_INVALID_ARGUMENT, "null argument");
    *out = nullptr;
    auto *c = new mri_kv_cache();
    c->n_layers = n_layers;
    c->max_seq = max_seq;
    c->kvd = n_kv_heads * head_dim;
    const size_t bytes = n_layers * max_seq * c->kvd * sizeof(float);
    hipError_t e;
    if ((e = hipMalloc(&c->k, bytes ? bytes : 4)) || (e = hipMalloc(&c->v, bytes ? bytes : 4)) ||
        (e = hipMemset(c->k, 0, bytes)) || (e = hipMemset(c->v, 0, bytes))) {
        mri_kv_cache_destroy(c);
        return hip_error(e, "kv_cache_create");
    }
    *out = c;
    return MRI_OK;
}

void mri_kv_cache_destroy(mri_kv_cache *c) {
    if (!c) return;
    if (c->k) (void)hipFree(c->k);
    if (c->v) (void)hipFree(c->v);
    delete c;
}

mri_status mri_llama_forward_cached(mri_llama *m, const uint32_t *tokens, size_t n,
                                    size_t start_pos, mri_kv_cache *c, float *logits,
                                    void *stream) {
    TRY(check_run(m, n, start_pos, c));
    TRY(check_tokens(m, tokens, n));
    if (!logits) return set_error(MRI_ERR_INVALID_ARGUMENT, "null logits");
    auto s = static_cast<hipStream_t>(stream);
    if (n == 1 && row_path(m))
        return run_rows(m, nullptr, 1, start_pos, c, logits, s, Emb::kHost, tokens[0]);
    MRI_HIP(hipMemcpyAsync(m->tok, tokens, n * sizeof(uint32_t), hipMemcpyHostToDevice, s));
    return run_rows(m, m->tok, n, start_pos, c, logits, s);
}

mri_status mri_llama_forward_decode(mri_llama *m, uint32_t token, size_t pos, mri_kv_cache *c,
                                    float *logits, void *stream) {
    return mri_llama_forward_cached(m, &token, 1, pos, c, logits, stream);
}

mri_status mri_llama_generate_greedy(mri_llama *m, const uint32_t *prompt, size_t n_prompt,
                                     size_t n_steps, mri_kv_cache *c, uint32_t *tokens_out,
                                     float *logits_out, void *stream) {
    TRY(check_run(m, n_prompt + n_steps, 0, c));
    if (n_prompt == 0)
        return set_error(MRI_ERR_INVALID_SHAPE, "generate: prompt must not be empty");
    TRY(check_tokens(m, prompt, n_prompt));
    if (!tokens_out) return set_error(MRI_ERR_INVALID_ARGUMENT, "null tokens_out");
    auto s = static_cast<hipStream_t>(stream);
    const size_t V = m->cfg.vocab;
    // prefill logits of every prompt row (the per-tensor activation scale of
    // the INT8 output projection covers all of them, as LlamaModelInt8::forward)
    if (m->logits_rows < n_prompt) {
        if (m->logits_buf) {
            MRI_HIP(hipStreamSynchronize(s));
            MRI_HIP(hipFree(m->logits_buf));
            m->logits_buf = nullptr;
            m->logits_rows = 0;
        }
        MRI_HIP(hipMalloc(&m->logits_buf, n_prompt * V * sizeof(float)));
        m->logits_rows = n_prompt;
    }
    MRI_HIP(hipMemcpyAsync(m->tok, prompt, n_prompt * sizeof(uint32_t), hipMemcpyHostToDevice, s));
    TRY(run_rows(m, m->tok, n_prompt, 0, c, m->logits_buf, s));
    const float *last = m->logits_buf + (n_prompt - 1) * V;
    if (logits_out)
        MRI_HIP(hipMemcpyAsync(logits_out, last, V * sizeof(float), hipMemcpyDeviceToDevice, s));
    // folded decode rows: each argmax also gathers the chosen token's
    // embedding row into m->x for the next step; after the prompt by its own
    // kernel, after each decode row in the output projection's epilogue
    const bool fold = row_path(m);
    auto pick = [&](const float *lg, uint32_t *id, bool next) {
        return fold && next ? launch_argmax_embed(lg, V, id, m->embd, m->cfg.dim, m->x, s)
                            : launch_argmax(lg, 1, V, id, s);
    };
    TRY(pick(last, m->gen, n_steps > 0));
    // the decode rows' argmax keys (one per 16-channel tile of the output
    // projection), after the split argmax's words in its workspace
    void *aws = nullptr;
    const size_t n_keys = (V + kTileN - 1) / kTileN;
    if (fold && n_steps) TRY(argmax_ws_get(s, &aws, kArgmaxWsBytes + n_keys * 8));
    auto *keys = reinterpret_cast<unsigned long long *>(static_cast<char *>(aws) + kArgmaxWsBytes);
    // With a layer, step i > 0 takes its token from step i - 1's keys in its
    // first projection's prologue (which also stores it to gen[i]); the last
    // step's keys are reduced by launch_argmax_keys.  Without layers a
    // separate reduction gathers each next embedding row.
    const bool keys_in = fold && m->cfg.n_layers > 0;
    for (size_t i = 0; i < n_steps; ++i) {
        float *lg = logits_out ? logits_out + (i + 1) * V : m->logits_buf;
        if (fold) {
            RowOps arg;
            arg.arg_keys = keys;
            Emb emb = Emb::kInX;
            if (keys_in && i > 0) {
                m->in_keys = keys;
                m->n_in_keys = (int)n_keys;
                m->tok_out = m->gen + i;
                emb = Emb::kKeys;
            }
            const mri_status st = run_rows(m, m->gen + i, 1, n_prompt + i, c, lg, s, emb, 0, &arg);
            m->in_keys = nullptr;
            m->tok_out = nullptr;
            TRY(st);
            const bool next = i + 1 < n_steps;
            if (!keys_in || !next)
                TRY(launch_argmax_keys(keys, n_keys, m->gen + i + 1, next ? m->embd : nullptr,
                                       m->cfg.dim, m->x, s));
        } else {
            TRY(run_rows(m, m->gen + i, 1, n_prompt + i, c, lg, s, Emb::kInX));
            TRY(pick(lg, m->gen + i + 1, i + 1 < n_steps));
        }
    }
    MRI_HIP(hipMemcpyAsync(tokens_out, m->gen, (n_steps + 1) * sizeof(uint32_t),
                           hipMemcpyDeviceToHost, s));
    MRI_HIP(hipStreamSynchronize(s));
    return MRI_OK;
}

mri_status mri_argmax(const float *v, size_t rows, size_t n, uint32_t *idx, void *stream) {
    if (rows && (!v || !idx)) return set_error(MRI_ERR_INVALID_ARGUMENT, "null pointer");
    if (rows && n == 0) return set_error(MRI_ERR_INVALID_SHAPE, "argmax: empty rows");
    return launch_argmax(v, rows, n, idx, static_cast<hipStream_t>(stream));
}

}  // extern "C"
