// capi.cpp — the extern "C" boundary (include/mri_qmatmul.h).
//
// Host-side validation reproduces the reference's TensorError behaviour and
// check order; everything else is dispatch to the kernels in the .hip files.
#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <map>
#include <mutex>
#include <string>
#include <utility>
#include <vector>

#include "common.hpp"

struct mri_qmatrix {
    mri::QMatrixDev d;
};
struct mri_q8_0_matrix {
    mri::Q8MatrixDev d;
};
struct mri_q4_0_matrix {
    mri::Q8MatrixDev d;  // w4: Q4_0 lap blocks
};

namespace mri {

const QMatrixDev &handle_dev(const mri_qmatrix *h) { return h->d; }
const Q8MatrixDev &handle_dev(const mri_q8_0_matrix *h) { return h->d; }
const Q8MatrixDev &handle_dev(const mri_q4_0_matrix *h) { return h->d; }

static thread_local std::string g_last_error;

mri_status set_error(mri_status st, const std::string &msg) {
    g_last_error = msg;
    return st;
}

mri_status hip_error(hipError_t e, const char *what) {
    return set_error(MRI_ERR_HIP, std::string(what) + ": " + hipGetErrorString(e));
}

static std::string fmt(const char *f, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, f);
    vsnprintf(buf, sizeof buf, f, ap);
    va_end(ap);
    return buf;
}

// ---- device checks ----------------------------------------------------------
static std::mutex g_dev_mu;
static std::map<int, int> g_dev_ok;  // device -> 1 gfx950, 0 other

mri_status current_device(int *dev) {
    MRI_HIP(hipGetDevice(dev));
    std::lock_guard<std::mutex> lk(g_dev_mu);
    auto it = g_dev_ok.find(*dev);
    if (it == g_dev_ok.end()) {
        hipDeviceProp_t prop;
        MRI_HIP(hipGetDeviceProperties(&prop, *dev));
        const int ok = std::strncmp(prop.gcnArchName, "gfx950", 6) == 0 ? 1 : 0;
        it = g_dev_ok.emplace(*dev, ok).first;
        if (!ok)
            g_last_error = std::string("device arch ") + prop.gcnArchName +
                           " is not gfx950";
    }
    if (!it->second)
        return set_error(MRI_ERR_UNSUPPORTED, "this library is built for gfx950 only");
    return MRI_OK;
}

// ---- per-(device, stream) scratch ----------------------------------------------
struct Scratch {
    void *ptr = nullptr;
    size_t bytes = 0;
};
int device_cus() {
    static std::atomic<int> cus[kMaxDevices] = {};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return 0;
    int n = cus[dev].load(std::memory_order_relaxed);
    if (n == 0) {
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
            return 0;
        cus[dev].store(n, std::memory_order_relaxed);  // every thread stores the same value
    }
    return n;
}

static std::mutex g_scratch_mu;
static std::map<std::pair<int, hipStream_t>, Scratch> g_scratch;

mri_status scratch_get(hipStream_t stream, size_t bytes, void **ptr) {
    int dev = 0;
    MRI_HIP(hipGetDevice(&dev));
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    Scratch &sc = g_scratch[{dev, stream}];
    if (sc.bytes < bytes) {
        size_t want = round_up(bytes < (1u << 20) ? (1u << 20) : bytes, 1u << 20);
        if (sc.ptr) {
            MRI_HIP(hipStreamSynchronize(stream));
            MRI_HIP(hipFree(sc.ptr));
            sc.ptr = nullptr;
            sc.bytes = 0;
        }
        MRI_HIP(hipMalloc(&sc.ptr, want));
        sc.bytes = want;
    }
    *ptr = sc.ptr;
    return MRI_OK;
}

// Per-(device, stream) workspaces of the kernels that count arrivals (the
// stream-K GEMM, the one-row argmax).  Zeroed whenever they are
// (re)allocated; the kernels leave their counters zero after every call.
static std::mutex g_ws_mu;
static std::map<std::pair<int, hipStream_t>, Scratch> g_ws, g_aws;

static mri_status zeroed_ws_get(std::map<std::pair<int, hipStream_t>, Scratch> &map,
                                hipStream_t stream, size_t bytes, void **ptr) {
    int dev = 0;
    MRI_HIP(hipGetDevice(&dev));
    std::lock_guard<std::mutex> lk(g_ws_mu);
    Scratch &sc = map[{dev, stream}];
    if (sc.bytes < bytes) {
        const size_t want = round_up(bytes, 1u << 20);
        if (sc.ptr) {
            MRI_HIP(hipStreamSynchronize(stream));
            MRI_HIP(hipFree(sc.ptr));
            sc.ptr = nullptr;
            sc.bytes = 0;
        }
        MRI_HIP(hipMalloc(&sc.ptr, want));
        MRI_HIP(hipMemset(sc.ptr, 0, want));
        sc.bytes = want;
    }
    *ptr = sc.ptr;
    return MRI_OK;
}

mri_status gemm_ws_get(hipStream_t stream, size_t bytes, void **ptr) {
    return zeroed_ws_get(g_ws, stream, bytes, ptr);
}

mri_status argmax_ws_get(hipStream_t stream, void **ptr, size_t bytes) {
    return zeroed_ws_get(g_aws, stream, std::max(bytes, kArgmaxWsBytes), ptr);
}

static inline bool aligned(const void *p, size_t a) {
    return (reinterpret_cast<uintptr_t>(p) % a) == 0;
}

// Carves consecutive 256-byte aligned regions out of one scratch block.
struct Carver {
    size_t off = 0;
    size_t take(size_t bytes) {
        size_t o = off;
        off = round_up(off + bytes, 256);
        return o;
    }
};

static std::string dims_str(const size_t *dims, size_t ndim) {
    std::string s = "[";
    for (size_t i = 0; i < ndim; ++i) {
        if (i) s += ", ";
        s += std::to_string(dims[i]);
    }
    return s + "]";
}

// matmul_int8 dispatch on prepared activations [m][kp].
mri_status run_int8(const int8_t *act, size_t m, const float *sa_ptr,
                           int sa_stride, float sa_value, const QMatrixDev &w,
                           float *out, int32_t *acc_out, hipStream_t s) {
    if (gemv_int8_supported(false, m, w.n_tiles, w.k_in, w.kp))
        return launch_gemv_int8(nullptr, act, m, sa_ptr, sa_stride, sa_value, w, out,
                                nullptr, nullptr, acc_out, s);
    return launch_skinny_int8(act, m, sa_ptr, sa_stride, sa_value, w, out, acc_out, s);
}

// matmul_q8_0_direct dispatch on quantized rows [m][kp] (chunk-permuted).
mri_status run_q8(const int8_t *act, size_t m, const float *sa_rows,
                         const Q8MatrixDev &w, float *out, int32_t *block_dots,
                         hipStream_t s, bool may_alloc) {
    if (gemv_q8_supported(false, m, w.n_tiles, w.k_in, w.kp))
        return launch_gemv_q8_0(nullptr, act, m, sa_rows, w, out, block_dots, nullptr, s);
    // prefill sizes: the LDS-tiled kernel (it has no block-dot output)
    if (!block_dots && gemm_q8_supported(m, w)) {
        void *ws = nullptr;
        const size_t wsb = may_alloc ? gemm_q8_ws_bytes(m, w) : 0;
        if (wsb) {
            const mri_status st = gemm_ws_get(s, wsb, &ws);
            if (st) return st;
        }
        return launch_gemm_q8_0(act, m, sa_rows, w, out, ws, s);
    }
    return launch_skinny_q8_0(act, m, sa_rows, w, out, block_dots, s);
}

// Returns act rows with pitch w.kp: the caller's buffer when it already has
// that layout, else a zero-padded copy in scratch.
static mri_status prepare_act(const int8_t *act_q, size_t m, const QMatrixDev &w,
                              hipStream_t s, const int8_t **act) {
    if (w.kp == w.k_in && aligned(act_q, 16)) {
        *act = act_q;
        return MRI_OK;
    }
    void *base = nullptr;
    mri_status st = scratch_get(s, m * w.kp, &base);
    if (st) return st;
    st = launch_pad_rows(act_q, m, w.k_in, w.kp, static_cast<int8_t *>(base), s);
    *act = static_cast<const int8_t *>(base);
    return st;
}

}  // namespace mri

using namespace mri;

extern "C" {

const char *mri_last_error(void) { return g_last_error.c_str(); }

const char *mri_version(void) { return "mri_qmatmul 0.1.0 (gfx950)"; }

// ===========================================================================
// weights
// ===========================================================================

static mri_status alloc_qmatrix(size_t n_out, size_t k_in, QMatrixDev &d) {
    d.n_out = n_out;
    d.k_in = k_in;
    d.n_tiles = (n_out + kTileN - 1) / kTileN;
    d.kp = round_up(k_in ? k_in : 1, kChunkK);
    MRI_HIP(hipGetDevice(&d.device));
    MRI_HIP(hipMalloc(&d.tiles, d.n_tiles * d.kp * kTileN + 256));
    MRI_HIP(hipMalloc(&d.scales, d.n_tiles * kTileN * sizeof(float) + 256));
    return MRI_OK;
}

static void free_qmatrix(QMatrixDev &d) {
    if (d.tiles) (void)hipFree(d.tiles);
    if (d.scales) (void)hipFree(d.scales);
    d.tiles = nullptr;
    d.scales = nullptr;
}

mri_status mri_qmatrix_create_device(const int8_t *data_dev, const float *scales_dev,
                                     size_t n_out, size_t k_in, void *stream,
                                     mri_qmatrix **out) {
    if (!out) return set_error(MRI_ERR_INVALID_ARGUMENT, "out is null");
    *out = nullptr;
    if (n_out * k_in && !data_dev)
        return set_error(MRI_ERR_INVALID_ARGUMENT, "data is null");
    if (n_out && !scales_dev)
        return set_error(MRI_ERR_INVALID_ARGUMENT, "scales is null");
    int dev;
    mri_status st = current_device(&dev);
    if (st) return st;
    auto *h = new mri_qmatrix();
    st = alloc_qmatrix(n_out, k_in, h->d);
    if (!st)
        st = launch_repack_int8(data_dev, scales_dev, h->d,
                                static_cast<hipStream_t>(stream));
    if (st) {
        free_qmatrix(h->d);
        delete h;
        return st;
    }
    *out = h;
    return MRI_OK;
}

mri_status mri_qmatrix_create(const int8_t *data, const float *scales, size_t n_out,
                              size_t k_in, mri_qmatrix **out) {
    if (!out) return set_error(MRI_ERR_INVALID_ARGUMENT, "out is null");
    *out = nullptr;
    if (n_out * k_in && !data) return set_error(MRI_ERR_INVALID_ARGUMENT, "data is null");
    if (n_out && !scales) return set_error(MRI_ERR_INVALID_ARGUMENT, "scales is null");
    int dev;
    mri_status st = current_device(&dev);
    if (st) return st;
    int8_t *dd = nullptr;
    float *ds = nullptr;
    MRI_HIP(hipMalloc(&dd, n_out * k_in + 16));
    hipError_t e = hipMalloc(&ds, n_out * sizeof(float) + 16);
    if (e != hipSuccess) {
        (void)hipFree(dd);
        return hip_error(e, "hipMalloc");
    }
    e = hipMemcpy(dd, data, n_out * k_in, hipMemcpyHostToDevice);
    if (e == hipSuccess) e = hipMemcpy(ds, scales, n_out * sizeof(float), hipMemcpyHostToDevice);
    if (e != hipSuccess) st = hip_error(e, "hipMemcpy");
    if (!st) st = mri_qmatrix_create_device(dd, ds, n_out, k_in, nullptr, out);
    if (!st) {
        e = hipStreamSynchronize(nullptr);
        if (e != hipSuccess) st = hip_error(e, "hipStreamSynchronize");
    }
    (void)hipFree(dd);
    (void)hipFree(ds);
    if (st && *out) {
        mri_qmatrix_destroy(*out);
        *out = nullptr;
    }
    return st;
}

mri_status mri_qmatrix_read(const mri_qmatrix *w, int8_t *data, float *scales) {
    if (!w) return set_error(MRI_ERR_INVALID_ARGUMENT, "null handle");
    const QMatrixDev &d = w->d;
    const size_t P = d.kp / kChunkK;
    std::vector<int8_t> tiles(d.n_tiles * P * 1024);
    std::vector<float> sc(d.n_tiles * kTileN);
    MRI_HIP(hipDeviceSynchronize());
    if (!tiles.empty()) MRI_HIP(hipMemcpy(tiles.data(), d.tiles, tiles.size(), hipMemcpyDeviceToHost));
    if (!sc.empty()) MRI_HIP(hipMemcpy(sc.data(), d.scales, sc.size() * 4, hipMemcpyDeviceToHost));
    for (size_t n = 0; n < d.n_out; ++n) {
        const size_t T = n / kTileN, r = n % kTileN;
        for (size_t k = 0; k < d.k_in; ++k) {
            const size_t p = k / kChunkK, g = (k % kChunkK) / 16, j = k % 16;
            const size_t lane = g * 16 + r;
            if (data) data[n * d.k_in + k] = tiles[((p * d.n_tiles + T) * 64 + lane) * 16 + j];
        }
        if (scales) scales[n] = sc[n];
    }
    return MRI_OK;
}

size_t mri_qmatrix_n_out(const mri_qmatrix *w) { return w ? w->d.n_out : 0; }
size_t mri_qmatrix_k_in(const mri_qmatrix *w) { return w ? w->d.k_in : 0; }
size_t mri_qmatrix_device_bytes(const mri_qmatrix *w) {
    return w ? w->d.n_tiles * w->d.kp * kTileN + w->d.n_tiles * kTileN * 4 : 0;
}

void mri_qmatrix_destroy(mri_qmatrix *w) {
    if (!w) return;
    free_qmatrix(w->d);
    delete w;
}

static mri_status q8_check(size_t len, size_t n_out, size_t k_in) {
    if (k_in % kQK)
        return set_error(MRI_ERR_INVALID_SHAPE,
                         fmt("Q8_0WeightMatrix: k_in=%zu is not a multiple of 32", k_in));
    const size_t nb = k_in / kQK;
    const size_t expected = n_out * nb * kQ8Bytes;
    if (len != expected)
        return set_error(MRI_ERR_INVALID_SHAPE,
                         fmt("Q8_0WeightMatrix: data.len()=%zu != expected %zu "
                             "(n_out=%zu, n_blocks=%zu, block_size=34)",
                             len, expected, n_out, nb));
    return MRI_OK;
}

mri_status mri_q8_0_matrix_from_raw_device(const uint8_t *data_dev, size_t len,
                                           size_t n_out, size_t k_in, void *stream,
                                           mri_q8_0_matrix **out) {
    if (!out) return set_error(MRI_ERR_INVALID_ARGUMENT, "out is null");
    *out = nullptr;
    mri_status st = q8_check(len, n_out, k_in);
    if (st) return st;
    if (len && !data_dev) return set_error(MRI_ERR_INVALID_ARGUMENT, "data is null");
    int dev;
    st = current_device(&dev);
    if (st) return st;
    auto *h = new mri_q8_0_matrix();
    Q8MatrixDev &d = h->d;
    d.n_out = n_out;
    d.k_in = k_in;
    d.n_blocks = k_in / kQK;
    d.n_tiles = (n_out + kTileN - 1) / kTileN;
    d.kp = round_up(k_in ? k_in : 1, kQK * kQ8ScaleGroup);
    d.device = dev;
    const hipError_t e = hipMalloc(&d.laps, d.bytes() + 256);
    if (e != hipSuccess) st = hip_error(e, "hipMalloc");
    if (!st) st = launch_repack_q8_0(data_dev, d, static_cast<hipStream_t>(stream));
    if (st) {
        mri_q8_0_matrix_destroy(h);
        return st;
    }
    *out = h;
    return MRI_OK;
}

mri_status mri_q8_0_matrix_from_raw_bytes(const uint8_t *data, size_t len, size_t n_out,
                                          size_t k_in, mri_q8_0_matrix **out) {
    if (!out) return set_error(MRI_ERR_INVALID_ARGUMENT, "out is null");
    *out = nullptr;
    mri_status st = q8_check(len, n_out, k_in);
    if (st) return st;
    if (len && !data) return set_error(MRI_ERR_INVALID_ARGUMENT, "data is null");
    int dev;
    st = current_device(&dev);
    if (st) return st;
    uint8_t *dd = nullptr;
    MRI_HIP(hipMalloc(&dd, len + 16));
    hipError_t e = hipMemcpy(dd, data, len, hipMemcpyHostToDevice);
    if (e != hipSuccess) st = hip_error(e, "hipMemcpy");
    if (!st) st = mri_q8_0_matrix_from_raw_device(dd, len, n_out, k_in, nullptr, out);
    if (!st) {
        e = hipStreamSynchronize(nullptr);
        if (e != hipSuccess) st = hip_error(e, "hipStreamSynchronize");
    }
    (void)hipFree(dd);
    if (st && *out) {
        mri_q8_0_matrix_destroy(*out);
        *out = nullptr;
    }
    return st;
}

mri_status mri_q8_0_matrix_read_raw(const mri_q8_0_matrix *w, uint8_t *data, size_t len) {
    if (!w) return set_error(MRI_ERR_INVALID_ARGUMENT, "null handle");
    const Q8MatrixDev &d = w->d;
    if (len != d.n_out * d.n_blocks * kQ8Bytes)
        return set_error(MRI_ERR_INVALID_SHAPE, "read_raw: wrong length");
    const size_t G = d.laps_per_tile();
    std::vector<uint8_t> laps(d.bytes());
    MRI_HIP(hipDeviceSynchronize());
    if (!laps.empty()) MRI_HIP(hipMemcpy(laps.data(), d.laps, laps.size(), hipMemcpyDeviceToHost));
    for (size_t n = 0; n < d.n_out; ++n) {
        const size_t T = n / kTileN, r = n % kTileN;
        for (size_t b = 0; b < d.n_blocks; ++b) {
            const uint8_t *lap = laps.data() + (T * G + b / 8) * kQ8LapBytes;
            uint8_t *blk = data + (n * d.n_blocks + b) * kQ8Bytes;
            const uint8_t *dv = lap + 4096 + r * 16 + (b % 8) * 2;
            blk[0] = dv[0];
            blk[1] = dv[1];
            const size_t c = (b / 2) % 4, h = b % 2;
            for (size_t g = 0; g < 4; ++g)
                for (size_t j = 0; j < 8; ++j)
                    blk[2 + g * 8 + j] = lap[(c * 64 + g * 16 + r) * 16 + h * 8 + j];
        }
    }
    return MRI_OK;
}

size_t mri_q8_0_matrix_n_out(const mri_q8_0_matrix *w) { return w ? w->d.n_out : 0; }
size_t mri_q8_0_matrix_k_in(const mri_q8_0_matrix *w) { return w ? w->d.k_in : 0; }
size_t mri_q8_0_matrix_device_bytes(const mri_q8_0_matrix *w) {
    if (!w) return 0;
    return w->d.bytes();
}

void mri_q8_0_matrix_destroy(mri_q8_0_matrix *w) {
    if (!w) return;
    if (w->d.laps) (void)hipFree(w->d.laps);
    delete w;
}

mri_status mri_q4_0_matrix_from_raw_device(const uint8_t *data_dev, size_t len, size_t n_out,
                                           size_t k_in, int order, void *stream,
                                           mri_q4_0_matrix **out) {
    if (!out) return set_error(MRI_ERR_INVALID_ARGUMENT, "out is null");
    *out = nullptr;
    if (order != MRI_Q4_ORDER_INTERLEAVED && order != MRI_Q4_ORDER_GGML)
        return set_error(MRI_ERR_INVALID_ARGUMENT, fmt("unknown Q4_0 nibble order %d", order));
    if (k_in % kQK)
        return set_error(MRI_ERR_INVALID_SHAPE,
                         fmt("Q4_0 weights: k_in=%zu is not a multiple of 32", k_in));
    const size_t expected = n_out * (k_in / kQK) * kQ4Bytes;
    if (len != expected)
        return set_error(MRI_ERR_INVALID_SHAPE,
                         fmt("Q4_0 weights: data.len()=%zu != expected %zu", len, expected));
    if (len && !data_dev) return set_error(MRI_ERR_INVALID_ARGUMENT, "data is null");
    int dev;
    mri_status st = current_device(&dev);
    if (st) return st;
    auto *h = new mri_q4_0_matrix();
    Q8MatrixDev &d = h->d;
    d.n_out = n_out;
    d.k_in = k_in;
    d.n_blocks = k_in / kQK;
    d.n_tiles = (n_out + kTileN - 1) / kTileN;
    d.kp = round_up(k_in ? k_in : 1, kQ8LapK);
    d.device = dev;
    d.w4 = true;
    const hipError_t e = hipMalloc(&d.laps, d.bytes() + 256);
    if (e != hipSuccess) st = hip_error(e, "hipMalloc");
    if (!st)
        st = launch_repack_q4_0(data_dev, order == MRI_Q4_ORDER_GGML, d,
                                static_cast<hipStream_t>(stream));
    if (st) {
        mri_q4_0_matrix_destroy(h);
        return st;
    }
    *out = h;
    return MRI_OK;
}

mri_status mri_q4_0_matrix_from_raw_bytes(const uint8_t *data, size_t len, size_t n_out,
                                          size_t k_in, int order, mri_q4_0_matrix **out) {
    if (!out) return set_error(MRI_ERR_INVALID_ARGUMENT, "out is null");
    *out = nullptr;
    if (len && !data) return set_error(MRI_ERR_INVALID_ARGUMENT, "data is null");
    int dev;
    mri_status st = current_device(&dev);
    if (st) return st;
    uint8_t *dd = nullptr;
    MRI_HIP(hipMalloc(&dd, len + 16));
    hipError_t e = hipMemcpy(dd, data, len, hipMemcpyHostToDevice);
    if (e != hipSuccess) st = hip_error(e, "hipMemcpy");
    if (!st) st = mri_q4_0_matrix_from_raw_device(dd, len, n_out, k_in, order, nullptr, out);
    if (!st) {
        e = hipStreamSynchronize(nullptr);
        if (e != hipSuccess) st = hip_error(e, "hipStreamSynchronize");
    }
    (void)hipFree(dd);
    if (st && *out) {
        mri_q4_0_matrix_destroy(*out);
        *out = nullptr;
    }
    return st;
}

size_t mri_q4_0_matrix_n_out(const mri_q4_0_matrix *w) { return w ? w->d.n_out : 0; }
size_t mri_q4_0_matrix_k_in(const mri_q4_0_matrix *w) { return w ? w->d.k_in : 0; }
size_t mri_q4_0_matrix_device_bytes(const mri_q4_0_matrix *w) { return w ? w->d.bytes() : 0; }

void mri_q4_0_matrix_destroy(mri_q4_0_matrix *w) {
    if (!w) return;
    if (w->d.laps) (void)hipFree(w->d.laps);
    delete w;
}

}  // extern "C"

namespace mri {

// Row concatenation of weight handles with one k_in whose n_out are whole
// tiles (multiples of 16).  The result is a new handle; the parts are not
// modified.  INT8 (slab-major chunks): slab p of the fused matrix is the
// parts' slab p side by side, so each part is one pitched copy.  Q8_0
// (tile-major lap blocks): the parts' buffers one after the other.
mri_status concat_qmatrix(const mri_qmatrix *const *parts, int n, hipStream_t s,
                          mri_qmatrix **out) {
    *out = nullptr;
    size_t rows = 0;
    for (int i = 0; i < n; ++i) {
        if (parts[i]->d.n_out % kTileN || parts[i]->d.k_in != parts[0]->d.k_in)
            return set_error(MRI_ERR_INVALID_SHAPE, "concat: parts must be whole tiles of one K");
        rows += parts[i]->d.n_out;
    }
    auto *h = new mri_qmatrix();
    mri_status st = alloc_qmatrix(rows, parts[0]->d.k_in, h->d);
    const size_t P = h->d.kp / kChunkK;
    size_t t0 = 0;
    for (int i = 0; i < n && !st; ++i) {
        const QMatrixDev &d = parts[i]->d;
        hipError_t e = hipMemcpy2DAsync(h->d.tiles + t0 * 1024, h->d.n_tiles * 1024, d.tiles,
                                        d.n_tiles * 1024, d.n_tiles * 1024, P,
                                        hipMemcpyDeviceToDevice, s);
        if (e == hipSuccess)
            e = hipMemcpyAsync(h->d.scales + t0 * kTileN, d.scales,
                               d.n_tiles * kTileN * sizeof(float), hipMemcpyDeviceToDevice, s);
        if (e != hipSuccess) st = hip_error(e, "concat_qmatrix");
        t0 += d.n_tiles;
    }
    if (st) {
        mri_qmatrix_destroy(h);
        return st;
    }
    *out = h;
    return MRI_OK;
}

// Tile-major lap blocks (Q8_0 and W4A8 handles): the parts' buffers one
// after the other.
template <typename H, void (*Destroy)(H *)>
mri_status concat_laps(const H *const *parts, int n, hipStream_t s, H **out) {
    *out = nullptr;
    size_t rows = 0;
    for (int i = 0; i < n; ++i) {
        if (parts[i]->d.n_out % kTileN || parts[i]->d.k_in != parts[0]->d.k_in)
            return set_error(MRI_ERR_INVALID_SHAPE, "concat: parts must be whole tiles of one K");
        rows += parts[i]->d.n_out;
    }
    auto *h = new H();
    Q8MatrixDev &d = h->d;
    d = parts[0]->d;
    d.laps = nullptr;
    d.n_out = rows;
    d.n_tiles = rows / kTileN;
    hipError_t e = hipMalloc(&d.laps, d.bytes() + 256);
    size_t off = 0;
    for (int i = 0; i < n && e == hipSuccess; ++i) {
        const Q8MatrixDev &pd = parts[i]->d;
        e = hipMemcpyAsync(d.laps + off, pd.laps, pd.bytes(), hipMemcpyDeviceToDevice, s);
        off += pd.bytes();
    }
    if (e != hipSuccess) {
        Destroy(h);
        return hip_error(e, "concat");
    }
    *out = h;
    return MRI_OK;
}

mri_status concat_q8_0_matrix(const mri_q8_0_matrix *const *parts, int n, hipStream_t s,
                              mri_q8_0_matrix **out) {
    return concat_laps<mri_q8_0_matrix, mri_q8_0_matrix_destroy>(parts, n, s, out);
}

mri_status concat_q4_0_matrix(const mri_q4_0_matrix *const *parts, int n, hipStream_t s,
                              mri_q4_0_matrix **out) {
    return concat_laps<mri_q4_0_matrix, mri_q4_0_matrix_destroy>(parts, n, s, out);
}

}  // namespace mri

extern "C" {

// ===========================================================================
// quantizers
// ===========================================================================

mri_status mri_quantize_symmetric(const float *x, size_t len, int8_t *q, float *scale,
                                  void *stream) {
    if ((len && (!x || !q)) || !scale)
        return set_error(MRI_ERR_INVALID_ARGUMENT, "null pointer");
    int dev;
    mri_status st = current_device(&dev);
    if (st) return st;
    auto s = static_cast<hipStream_t>(stream);
    void *base = nullptr;
    st = scratch_get(s, 1024 * sizeof(float), &base);
    if (st) return st;
    return launch_quantize_tensor(x, 1, len, len, false, nullptr, q, scale,
                                  static_cast<float *>(base), s);
}

mri_status mri_quantize_symmetric_rows(const float *x, size_t m, size_t k, int8_t *q,
                                       float *scales, void *stream) {
    if (m && (!scales || (k && (!x || !q))))
        return set_error(MRI_ERR_INVALID_ARGUMENT, "null pointer");
    int dev;
    mri_status st = current_device(&dev);
    if (st) return st;
    return launch_quantize_rows(x, m, k, k, false, nullptr, q, scales,
                                static_cast<hipStream_t>(stream));
}

mri_status mri_quantize_per_channel(const float *w, size_t len, size_t n_out, size_t k_in,
                                    int8_t *data, float *scales, void *stream) {
    if (len != n_out * k_in)
        return set_error(MRI_ERR_INVALID_SHAPE,
                         fmt("weights.len()=%zu != n_out*k_in=%zu", len, n_out * k_in));
    if (n_out && (!scales || (k_in && (!w || !data))))
        return set_error(MRI_ERR_INVALID_ARGUMENT, "null pointer");
    int dev;
    mri_status st = current_device(&dev);
    if (st) return st;
    return launch_quantize_per_channel(w, n_out, k_in, data, scales,
                                       static_cast<hipStream_t>(stream));
}

// ===========================================================================
// hot path
// ===========================================================================

mri_status mri_dot_i8(const int8_t *a, const int8_t *b, size_t len, int32_t *out,
                      void *stream) {
    if (!out || (len && (!a || !b)))
        return set_error(MRI_ERR_INVALID_ARGUMENT, "null pointer");
    int dev;
    mri_status st = current_device(&dev);
    if (st) return st;
    return launch_dot_i8(a, b, len, out, static_cast<hipStream_t>(stream));
}

static mri_status matmul_int8_common(const char *fn, const int8_t *act_q, size_t act_q_len,
                                     const float *sa_ptr, int sa_stride, float sa_value,
                                     const mri_qmatrix *w, size_t m, float *out,
                                     int32_t *acc_out, void *stream) {
    if (!w) return set_error(MRI_ERR_INVALID_ARGUMENT, "null weight handle");
    const QMatrixDev &d = w->d;
    const size_t k = d.k_in;
    if (act_q_len != m * k)
        return set_error(MRI_ERR_INVALID_SHAPE,
                         fmt("%s: act_q.len()=%zu != m*k=%zu*%zu=%zu", fn, act_q_len, m,
                             k, m * k));
    if (m * d.n_out == 0) return MRI_OK;
    if (!out || (m * k && !act_q))
        return set_error(MRI_ERR_INVALID_ARGUMENT, "null pointer");
    int dev;
    mri_status st = current_device(&dev);
    if (st) return st;
    auto s = static_cast<hipStream_t>(stream);
    if (m >= kGemmMinRows && gemm_rows_ok(m, d, act_q)) {
        // prefill on the caller's rows as they are
        void *ws = nullptr;
        if (const size_t wsb = gemm_ws_bytes(m, d)) {
            st = gemm_ws_get(s, wsb, &ws);
            if (st) return st;
        }
        return launch_gemm_int8(act_q, m, sa_ptr, sa_stride, sa_value, d, out, acc_out, ws, s,
                                true);
    }
    if (m >= kGemmMinRows) {
        // prefill: repack the rows into the GEMM fragment layout
        void *base = nullptr;
        st = scratch_get(s, gemm_pack_bytes(m, d.kp), &base);
        if (st) return st;
        auto *packed = static_cast<int8_t *>(base);
        st = launch_pack_gemm(act_q, m, k, k, d.kp, packed, s);
        if (st) return st;
        void *ws = nullptr;
        if (const size_t wsb = gemm_ws_bytes(m, d)) {
            st = gemm_ws_get(s, wsb, &ws);
            if (st) return st;
        }
        return launch_gemm_int8(packed, m, sa_ptr, sa_stride, sa_value, d, out, acc_out, ws, s);
    }
    const int8_t *act = nullptr;
    st = prepare_act(act_q, m, d, s, &act);
    if (st) return st;
    return run_int8(act, m, sa_ptr, sa_stride, sa_value, d, out, acc_out, s);
}

mri_status mri_matmul_int8(const int8_t *act_q, size_t act_q_len, float act_scale,
                           const mri_qmatrix *w, size_t m, float *out, int32_t *acc_out,
                           void *stream) {
    return matmul_int8_common("matmul_int8", act_q, act_q_len, nullptr, 0, act_scale, w,
                              m, out, acc_out, stream);
}

mri_status mri_matmul_int8_rows(const int8_t *act_q, size_t act_q_len,
                                const float *act_scales, const mri_qmatrix *w, size_t m,
                                float *out, int32_t *acc_out, void *stream) {
    if (m && !act_scales) return set_error(MRI_ERR_INVALID_ARGUMENT, "act_scales is null");
    return matmul_int8_common("matmul_int8_rows", act_q, act_q_len, act_scales, 1, 0.0f,
                              w, m, out, acc_out, stream);
}

mri_status mri_matmul_int8_from_f32(const float *input, const size_t *dims, size_t ndim,
                                    const mri_qmatrix *w, float *out, int8_t *act_q_out,
                                    float *act_scale_out, int32_t *acc_out, void *stream) {
    if (!w) return set_error(MRI_ERR_INVALID_ARGUMENT, "null weight handle");
    if (ndim && !dims) return set_error(MRI_ERR_INVALID_ARGUMENT, "dims is null");
    if (ndim != 2)
        return set_error(MRI_ERR_INVALID_SHAPE,
                         fmt("matmul_int8_from_f32: input must be 2-D, got %zuD (shape %s)",
                             ndim, dims_str(dims, ndim).c_str()));
    const QMatrixDev &d = w->d;
    const size_t m = dims[0], k = dims[1];
    if (k != d.k_in)
        return set_error(MRI_ERR_SHAPE_MISMATCH,
                         fmt("ShapeMismatch { expected: [%zu, %zu], got: [%zu, %zu] }", m,
                             d.k_in, m, k));
    if (m * k && (!input)) return set_error(MRI_ERR_INVALID_ARGUMENT, "input is null");
    if (m * d.n_out && !out) return set_error(MRI_ERR_INVALID_ARGUMENT, "out is null");
    int dev;
    mri_status st = current_device(&dev);
    if (st) return st;
    auto s = static_cast<hipStream_t>(stream);
    if (d.n_out > 0 && gemv_fusable(m, k, input) && aligned(act_q_out, 4) &&
        gemv_int8_supported(true, m, d.n_tiles, k, d.kp))
        return launch_gemv_int8(input, nullptr, m, nullptr, 0, 0.0f, d, out, act_q_out,
                                act_scale_out, acc_out, s);
    const bool gemm = m >= kGemmMinRows;
    Carver cv;
    const size_t o_act = cv.take(gemm ? gemm_pack_bytes(m, d.kp) : m * d.kp);
    const size_t o_part = cv.take(1024 * sizeof(float));
    const size_t o_scale = cv.take(sizeof(float));
    void *base = nullptr;
    st = scratch_get(s, cv.off, &base);
    if (st) return st;
    auto *b = static_cast<uint8_t *>(base);
    int8_t *act = reinterpret_cast<int8_t *>(b + o_act);
    float *scale = act_scale_out ? act_scale_out : reinterpret_cast<float *>(b + o_scale);
    auto *partials = reinterpret_cast<float *>(b + o_part);
    if (gemm) {
        // prefill: quantize straight into the GEMM fragment layout
        st = launch_quantize_pack(input, m, k, d.kp, act, act_q_out, scale, partials, s);
        if (st) return st;
        if (d.n_out == 0) return MRI_OK;
        void *ws = nullptr;
        if (const size_t wsb = gemm_ws_bytes(m, d)) {
            st = gemm_ws_get(s, wsb, &ws);
            if (st) return st;
        }
        return launch_gemm_int8(act, m, scale, 0, 0.0f, d, out, acc_out, ws, s);
    }
    st = launch_quantize_tensor(input, m, k, d.kp, false, act, act_q_out, scale, partials, s);
    if (st) return st;
    if (m * d.n_out == 0) return MRI_OK;
    return run_int8(act, m, scale, 0, 0.0f, d, out, acc_out, s);
}

}  // extern "C"

// Staging of the no-allocation entry point (quantized activation rows and
// their scales): one copy per device, held until the process ends.  Host
// code uses the address hipGetSymbolAddress gives for the current device,
// never the array's own name.
static __device__ __align__(256) uint8_t scratch[MRI_NOALLOC_SCRATCH_BYTES];

static mri_status noalloc_scratch(void **ptr) {
    static DeviceOnce once;
    static void *addr[kMaxDevices] = {};
    int dev = 0;
    MRI_HIP(hipGetDevice(&dev));
    MRI_HIP(once.run([](int d) {
        return hipGetSymbolAddress(&addr[d], HIP_SYMBOL(scratch));
    }));
    *ptr = addr[dev];  // published by the once's release
    return MRI_OK;
}

// matmul_q8_0_direct's body, shared with the W4A8 entry point (d.w4), the
// no-allocation variant (fixed: staging in the file's device array) and the
// block-ordered variant (exact: the skinny kernel, whose lanes add each
// output's block terms in block order, at every m).
static mri_status matmul_blocks(const char *name, const float *input, const size_t *dims,
                                size_t ndim, const Q8MatrixDev &d, float *out,
                                int32_t *block_dots_out, float *act_scales_out,
                                void *stream, bool fixed = false, bool exact = false) {
    if (ndim && !dims) return set_error(MRI_ERR_INVALID_ARGUMENT, "dims is null");
    if (ndim != 2)
        return set_error(MRI_ERR_INVALID_SHAPE,
                         fmt("%s: input must be 2-D, got %zuD (shape %s)", name, ndim,
                             dims_str(dims, ndim).c_str()));
    const size_t m = dims[0], k = dims[1];
    if (k != d.k_in)
        return set_error(MRI_ERR_SHAPE_MISMATCH,
                         fmt("ShapeMismatch { expected: [%zu, %zu], got: [%zu, %zu] }", m,
                             d.k_in, m, k));
    if (m * k && !input) return set_error(MRI_ERR_INVALID_ARGUMENT, "input is null");
    if (m * d.n_out && !out) return set_error(MRI_ERR_INVALID_ARGUMENT, "out is null");
    if (m == 0) return MRI_OK;
    int dev;
    mri_status st = current_device(&dev);
    if (st) return st;
    auto s = static_cast<hipStream_t>(stream);
    if (!exact && d.n_out > 0 && gemv_fusable(m, k, input) &&
        gemv_q8_supported(true, m, d.n_tiles, k, d.kp))
        return launch_gemv_q8_0(input, nullptr, m, nullptr, d, out, block_dots_out,
                                act_scales_out, s);
    Carver cv;
    const size_t o_act = cv.take(m * d.kp);
    const size_t o_sc = cv.take(m * sizeof(float));
    void *base = nullptr;
    if (fixed) {
        if (cv.off > MRI_NOALLOC_SCRATCH_BYTES)
            return set_error(MRI_ERR_UNSUPPORTED,
                             fmt("%s: %zu rows of K = %zu need %zu bytes of staging, more than "
                                 "the %d of the no-allocation entry point",
                                 name, m, k, cv.off, MRI_NOALLOC_SCRATCH_BYTES));
        st = noalloc_scratch(&base);
    } else {
        st = scratch_get(s, cv.off, &base);
    }
    if (st) return st;
    auto *b = static_cast<uint8_t *>(base);
    int8_t *act = reinterpret_cast<int8_t *>(b + o_act);
    float *sc = act_scales_out ? act_scales_out : reinterpret_cast<float *>(b + o_sc);
    st = launch_quantize_rows(input, m, k, d.kp, true, act, nullptr, sc, s);
    if (st) return st;
    if (d.n_out == 0) return MRI_OK;
    if (exact) return launch_skinny_q8_0(act, m, sc, d, out, block_dots_out, s);
    return run_q8(act, m, sc, d, out, block_dots_out, s, !fixed);
}

extern "C" {

mri_status mri_matmul_q8_0_direct(const float *input, const size_t *dims, size_t ndim,
                                  const mri_q8_0_matrix *w, float *out,
                                  int32_t *block_dots_out, float *act_scales_out,
                                  void *stream) {
    if (!w) return set_error(MRI_ERR_INVALID_ARGUMENT, "null weight handle");
    return matmul_blocks("matmul_q8_0_direct", input, dims, ndim, w->d, out, block_dots_out,
                         act_scales_out, stream);
}

mri_status mri_matmul_q8_0_direct_exact(const float *input, const size_t *dims, size_t ndim,
                                        const mri_q8_0_matrix *w, float *out,
                                        int32_t *block_dots_out, float *act_scales_out,
                                        void *stream) {
    if (!w) return set_error(MRI_ERR_INVALID_ARGUMENT, "null weight handle");
    return matmul_blocks("matmul_q8_0_direct", input, dims, ndim, w->d, out, block_dots_out,
                         act_scales_out, stream, false, true);
}

mri_status mri_matmul_q8_0_direct_noalloc(const float *input, const size_t *dims, size_t ndim,
                                          const mri_q8_0_matrix *w, float *out,
                                          int32_t *block_dots_out, float *act_scales_out,
                                          void *stream) {
    if (!w) return set_error(MRI_ERR_INVALID_ARGUMENT, "null weight handle");
    return matmul_blocks("matmul_q8_0_direct_noalloc", input, dims, ndim, w->d, out,
                         block_dots_out, act_scales_out, stream, true);
}

mri_status mri_matmul_q4_0_w4a8(const float *input, const size_t *dims, size_t ndim,
                                const mri_q4_0_matrix *w, float *out,
                                int32_t *block_dots_out, float *act_scales_out,
                                void *stream) {
    if (!w) return set_error(MRI_ERR_INVALID_ARGUMENT, "null weight handle");
    return matmul_blocks("matmul_q4_0_w4a8", input, dims, ndim, w->d, out, block_dots_out,
                         act_scales_out, stream);
}

mri_status mri_matmul_q4_0_dequant_matrix(const float *input, const size_t *dims, size_t ndim,
                                          const mri_q4_0_matrix *w, float *out, void *stream) {
    if (!w) return set_error(MRI_ERR_INVALID_ARGUMENT, "null weight handle");
    if (ndim && !dims) return set_error(MRI_ERR_INVALID_ARGUMENT, "dims is null");
    if (ndim != 2)
        return set_error(MRI_ERR_INVALID_SHAPE,
                         fmt("matmul_q4_0_dequant: `input` must be 2-D, got %zuD (shape %s)",
                             ndim, dims_str(dims, ndim).c_str()));
    const Q8MatrixDev &d = w->d;
    const size_t m = dims[0], k_in = dims[1];
    if (k_in != d.k_in)
        return set_error(MRI_ERR_SHAPE_MISMATCH,
                         fmt("ShapeMismatch { expected: [%zu, %zu], got: [%zu, %zu] }", m, d.k_in,
                             m, k_in));
    if (m * k_in && !input) return set_error(MRI_ERR_INVALID_ARGUMENT, "input is null");
    if (m * d.n_out && !out) return set_error(MRI_ERR_INVALID_ARGUMENT, "out is null");
    if (m == 0 || d.n_out == 0) return MRI_OK;
    int dev;
    mri_status st = current_device(&dev);
    if (st) return st;
    auto s = static_cast<hipStream_t>(stream);
    if (k_in == 0) {  // empty sums
        MRI_HIP(hipMemsetAsync(out, 0, m * d.n_out * sizeof(float), s));
        return MRI_OK;
    }
    if (!aligned(input, 16) || k_in % 4)
        return set_error(MRI_ERR_INVALID_ARGUMENT,
                         "matmul_q4_0_dequant (handle): input rows must be 16-byte aligned");
    return launch_gemv_w4a32(input, m, k_in, d, out, s);
}

mri_status mri_matmul_q4_0_dequant(const float *input, const size_t *dims, size_t ndim,
                                   const uint8_t *weight_q4, size_t weight_len,
                                   size_t n_out, size_t k, float *out, void *stream) {
    return mri_matmul_q4_0_dequant_ordered(input, dims, ndim, weight_q4, weight_len, n_out, k,
                                           MRI_Q4_ORDER_INTERLEAVED, out, stream);
}

mri_status mri_matmul_q4_0_dequant_ordered(const float *input, const size_t *dims, size_t ndim,
                                           const uint8_t *weight_q4, size_t weight_len,
                                           size_t n_out, size_t k, int order, float *out,
                                           void *stream) {
    if (order != MRI_Q4_ORDER_INTERLEAVED && order != MRI_Q4_ORDER_GGML)
        return set_error(MRI_ERR_INVALID_ARGUMENT, fmt("unknown Q4_0 nibble order %d", order));
    if (ndim && !dims) return set_error(MRI_ERR_INVALID_ARGUMENT, "dims is null");
    if (ndim != 2)
        return set_error(MRI_ERR_INVALID_SHAPE,
                         fmt("matmul_q4_0_dequant: `input` must be 2-D, got %zuD (shape %s)",
                             ndim, dims_str(dims, ndim).c_str()));
    const size_t m = dims[0], k_in = dims[1];
    if (k_in != k)
        return set_error(MRI_ERR_SHAPE_MISMATCH,
                         fmt("ShapeMismatch { expected: [%zu, %zu], got: [%zu, %zu] }", m, k,
                             m, k_in));
    if (k % kQK)
        return set_error(MRI_ERR_INVALID_SHAPE,
                         fmt("matmul_q4_0_dequant: k=%zu must be a multiple of 32 (Q4_0 "
                             "block size)",
                             k));
    const size_t expected = n_out * (k / kQK) * kQ4Bytes;
    if (weight_len != expected)
        return set_error(MRI_ERR_INVALID_SHAPE,
                         fmt("matmul_q4_0_dequant: weight_q4 has %zu bytes, expected %zu "
                             "for shape [%zu, %zu]",
                             weight_len, expected, n_out, k));
    if (m * n_out == 0) return MRI_OK;
    if (!out || (k && (!input || !weight_q4)))
        return set_error(MRI_ERR_INVALID_ARGUMENT, "null pointer");
    if (!aligned(weight_q4, 2))
        return set_error(MRI_ERR_INVALID_ARGUMENT, "weight_q4 must be 2-byte aligned");
    int dev;
    mri_status st = current_device(&dev);
    if (st) return st;
    auto s = static_cast<hipStream_t>(stream);
    const float *x = input;
    if (!aligned(input, 16)) {
        void *base = nullptr;
        st = scratch_get(s, m * k * sizeof(float), &base);
        if (st) return st;
        MRI_HIP(hipMemcpyAsync(base, input, m * k * sizeof(float),
                               hipMemcpyDeviceToDevice, s));
        x = static_cast<const float *>(base);
    }
    return launch_q4_0_dequant(x, m, k, weight_q4, n_out, order == MRI_Q4_ORDER_GGML, out, s);
}

mri_status mri_hbm_read(const void *p, size_t bytes, int32_t *sink, void *stream) {
    if (bytes && !p) return set_error(MRI_ERR_INVALID_ARGUMENT, "p is null");
    if (!aligned(p, 16)) return set_error(MRI_ERR_INVALID_ARGUMENT, "p is not 16-byte aligned");
    return launch_hbm_read(p, bytes, sink, static_cast<hipStream_t>(stream));
}

mri_status mri_mfma_i8_peak(const int8_t *src, int iters, int32_t *sink, int *n_cus,
                            void *stream) {
    if (!src) return set_error(MRI_ERR_INVALID_ARGUMENT, "src is null");
    if (!aligned(src, 16)) return set_error(MRI_ERR_INVALID_ARGUMENT, "src is not 16-byte aligned");
    if (iters < 1) return set_error(MRI_ERR_INVALID_ARGUMENT, "iters < 1");
    if (n_cus) *n_cus = device_cus();
    return launch_mfma_peak(src, iters, sink, static_cast<hipStream_t>(stream));
}

mri_status mri_synchronize(void *stream) {
    MRI_HIP(hipStreamSynchronize(static_cast<hipStream_t>(stream)));
    return MRI_OK;
}

}  // extern "C"
