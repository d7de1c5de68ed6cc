// The C ABI (include/telmo_hip.h): contexts, device weights, argument checks with the
// reference's semantics, and dispatch to the kernels.
//
//   tg_matmul / tg_matmul_device   Kernels::matmul        src/kernels/mod.rs:657-688
//   tg_linear / tg_linear_device   Kernels::linear        src/kernels/mod.rs:691-701
//   tg_weights_upload              PackedWeights::from_parts  src/kernels/mod.rs:214-237
//
// Dispatch (fast mode, int8 weights): m <= 8 with the row digits fitting the GEMV's LDS -> the
// dot4 GEMV (one launch); otherwise the row quantiser then the MFMA GEMM (two launches). Other
// precisions, the exact mode, and k beyond the integer path's limit run the exact kernel.
#include <cstring>
#include <mutex>
#include <string>

#include "../../include/telmo_hip.h"
#include "tg_internal.hpp"

struct tg_ctx {
    int device = 0;
    hipStream_t stream = nullptr;
    bool own_stream = false;
    uint32_t mode = TG_MODE_FAST;
    std::mutex mu;
    std::string err;
    // Workspace of the quantised rows and their exponents, grown on demand.
    uint8_t *qa = nullptr;
    size_t qa_cap = 0;
    int32_t *exps = nullptr;
    size_t exps_cap = 0;
    // Device staging of the host-pointer entry points, grown on demand.
    float *da = nullptr, *dc = nullptr, *dbias = nullptr;
    size_t da_cap = 0, dc_cap = 0, dbias_cap = 0;
    // Pinned host staging of the same: rows are gathered here so each direction is one DMA.
    float *hst = nullptr;
    size_t hst_cap = 0;
};

struct tg_weights {
    tg::DeviceWeights d;
    int device;
};

namespace {

int fail(tg_ctx *ctx, int code, const std::string &msg) {
    if (ctx) ctx->err = msg;
    return code;
}

int hip_fail(tg_ctx *ctx, hipError_t e, const char *what) {
    return fail(ctx, TG_ERR_HIP, std::string(what) + ": " + hipGetErrorString(e));
}

#define TG_HIP(ctx, call)                                   \
    do {                                                    \
        hipError_t e_ = (call);                             \
        if (e_ != hipSuccess) return hip_fail(ctx, e_, #call); \
    } while (0)

bool valid_precision(uint32_t p) { return p <= TG_Q8_0; }

// Grows a device buffer to at least `bytes`, waiting for queued work before freeing the old one.
template <typename T>
int grow(tg_ctx *ctx, T *&buf, size_t &cap, size_t bytes) {
    if (bytes <= cap) return TG_OK;
    if (buf) {
        TG_HIP(ctx, hipStreamSynchronize(ctx->stream));
        TG_HIP(ctx, hipFree(buf));
        buf = nullptr;
        cap = 0;
    }
    size_t want = bytes < 256 ? 256 : bytes;
    void *p = nullptr;
    if (hipMalloc(&p, want) != hipSuccess) return fail(ctx, TG_ERR_NOMEM, "device allocation failed");
    buf = static_cast<T *>(p);
    cap = want;
    return TG_OK;
}

// Pinned host staging (hipHostMalloc), grown on demand; the stream is idle between host calls.
int grow_host(tg_ctx *ctx, size_t bytes) {
    if (bytes <= ctx->hst_cap) return TG_OK;
    if (ctx->hst) {
        TG_HIP(ctx, hipStreamSynchronize(ctx->stream));
        TG_HIP(ctx, hipHostFree(ctx->hst));
        ctx->hst = nullptr;
        ctx->hst_cap = 0;
    }
    void *p = nullptr;
    if (hipHostMalloc(&p, bytes, hipHostMallocDefault) != hipSuccess)
        return fail(ctx, TG_ERR_NOMEM, "pinned host allocation failed");
    ctx->hst = static_cast<float *>(p);
    ctx->hst_cap = bytes;
    return TG_OK;
}

// Copies m rows of cols floats between a strided and a packed buffer (host memory).
void copy_rows(float *dst, size_t ldd, const float *src, size_t lds, size_t m, size_t cols) {
    if (ldd == cols && lds == cols) {
        std::memcpy(dst, src, m * cols * sizeof(float));
        return;
    }
    for (size_t r = 0; r < m; r++) std::memcpy(dst + r * ldd, src + r * lds, cols * sizeof(float));
}

// The checks of Kernels::matmul (src/kernels/mod.rs:669-677), in its order.
int check_matmul(tg_ctx *ctx, const float *a, size_t a_len, size_t lda, size_t m, const tg_weights *w, float *c,
                 size_t c_len, size_t ldc, const tg_epilogue *epi) {
    const size_t k = w->d.k, n = w->d.n;
    if (lda < k || ldc < n) return fail(ctx, TG_ERR_SHAPE, "lda must be >= k and ldc >= n");
    if (a_len < (m - 1) * lda + k) return fail(ctx, TG_ERR_SHAPE, "a is too short");
    if (c_len < (m - 1) * ldc + n) return fail(ctx, TG_ERR_SHAPE, "c is too short");
    if (epi && epi->bias && epi->bias_len < n) return fail(ctx, TG_ERR_SHAPE, "bias is too short");
    if (epi && epi->act > TG_ACT_SILU) return fail(ctx, TG_ERR_ARG, "unknown activation");
    if (!a && k > 0) return fail(ctx, TG_ERR_NULL, "a is null");
    if (!c) return fail(ctx, TG_ERR_NULL, "c is null");
    return TG_OK;
}

tg::EpiArgs epi_args(const tg_epilogue *epi, const float *bias_override, bool use_override) {
    tg::EpiArgs e{nullptr, TG_ACT_NONE, 1.0f, 0};
    if (epi) {
        e.bias = use_override ? bias_override : epi->bias;
        e.act = epi->act;
        e.scale = epi->scale;
        e.accumulate = epi->accumulate != 0;
    }
    return e;
}

// Queues the product on device buffers (arguments already checked).
int run_device(tg_ctx *ctx, const float *a, size_t lda, size_t m, const tg_weights *w, float *c, size_t ldc,
               const tg::EpiArgs &epi) {
    const tg::DeviceWeights &d = w->d;
    const bool int_path = ctx->mode == TG_MODE_FAST && (d.precision == TG_INT8 || d.precision == TG_Q8_0) &&
                          d.k <= tg::MAX_K_INT;
    if (!int_path) {
        TG_HIP(ctx, tg::launch_exact(a, lda, m, d, c, ldc, epi, ctx->stream));
        return TG_OK;
    }
    if (tg::gemv_fits(m, d.k, a, lda, d.precision)) {
        TG_HIP(ctx, tg::launch_gemv_i8(a, lda, m, d, c, ldc, epi, ctx->stream));
        return TG_OK;
    }
    int rc = grow(ctx, ctx->qa, ctx->qa_cap, tg::qa_bytes(m, d.k));
    if (rc) return rc;
    rc = grow(ctx, ctx->exps, ctx->exps_cap, m * sizeof(int32_t));
    if (rc) return rc;
    TG_HIP(ctx, tg::launch_quantize_rows(a, lda, m, d.k, ctx->qa, ctx->exps, ctx->stream));
    TG_HIP(ctx, tg::launch_gemm_i8(ctx->qa, ctx->exps, m, d, c, ldc, epi, ctx->stream));
    return TG_OK;
}

int upload(tg_ctx *ctx, const uint8_t *values, size_t values_len, const float *scales, size_t n_scales,
           uint32_t precision, size_t n, size_t k, tg_weights **out, bool from_device) {
    if (!ctx || !out) return fail(ctx, TG_ERR_NULL, "null argument");
    *out = nullptr;
    if (!valid_precision(precision)) return fail(ctx, TG_ERR_ARG, "unknown precision");
    if (precision == TG_Q8_0 && k % tg::Q8_BLOCK) return fail(ctx, TG_ERR_ARG, "q8_0 needs k in multiples of 32");
    if (values_len != tg_panel_bytes(precision, n, k)) return fail(ctx, TG_ERR_ARG, "values have the wrong length");
    if (n_scales != tg_scale_count(precision, n, k)) return fail(ctx, TG_ERR_ARG, "scales have the wrong length");
    if ((values_len && !values) || (n_scales && !scales)) return fail(ctx, TG_ERR_NULL, "null values or scales");
    if (reinterpret_cast<uintptr_t>(values) % 4) return fail(ctx, TG_ERR_ALIGN, "values must be 4-byte aligned");
    std::lock_guard<std::mutex> g(ctx->mu);
    TG_HIP(ctx, hipSetDevice(ctx->device));
    tg_weights *w = new tg_weights();
    w->device = ctx->device;
    tg::DeviceWeights &d = w->d;
    d.n = n;
    d.k = k;
    d.precision = precision;
    d.panels = tg::div_ceil(n, tg::PANEL);
    d.kb = tg::div_ceil(k, tg::KBLK);
    d.n_scales = n_scales;
    const bool mfma_layout = precision == TG_INT8 || precision == TG_Q8_0;
    d.values_bytes = mfma_layout ? d.panels * d.kb * 1024 : values_len;
    // The MFMA layout is k-block-major: the panels of one k-block are contiguous.
    d.panel_stride = mfma_layout ? 1024 : k * tg::PANEL * (precision == TG_F32 ? 4 : 2);
    d.blk_stride = mfma_layout ? d.panels * 1024 : 0;
    const hipMemcpyKind kind = from_device ? hipMemcpyDeviceToDevice : hipMemcpyHostToDevice;
    auto cleanup = [&](int code, const std::string &msg) {
        if (d.values) (void)hipFree(d.values);
        if (d.scales) (void)hipFree(d.scales);
        delete w;
        return fail(ctx, code, msg);
    };
    if (d.values_bytes && hipMalloc(&d.values, d.values_bytes) != hipSuccess)
        return cleanup(TG_ERR_NOMEM, "device allocation failed");
    if (n_scales && hipMalloc(&d.scales, n_scales * sizeof(float)) != hipSuccess)
        return cleanup(TG_ERR_NOMEM, "device allocation failed");
    hipError_t e = hipSuccess;
    if (n_scales) e = hipMemcpyAsync(d.scales, scales, n_scales * sizeof(float), kind, ctx->stream);
    if (e == hipSuccess && values_len) {
        if (mfma_layout) {
            uint8_t *raw = nullptr;
            if (hipMalloc(&raw, values_len) != hipSuccess) return cleanup(TG_ERR_NOMEM, "device allocation failed");
            e = hipMemcpyAsync(raw, values, values_len, kind, ctx->stream);
            if (e == hipSuccess) e = tg::launch_repack_i8(raw, d, ctx->stream);
            if (e == hipSuccess) e = hipStreamSynchronize(ctx->stream);
            (void)hipFree(raw);
        } else {
            e = hipMemcpyAsync(d.values, values, values_len, kind, ctx->stream);
        }
    }
    if (e == hipSuccess) e = hipStreamSynchronize(ctx->stream);
    if (e != hipSuccess) return cleanup(TG_ERR_HIP, std::string("weight upload: ") + hipGetErrorString(e));
    ctx->err.clear();
    *out = w;
    return TG_OK;
}

}  // namespace

extern "C" {

int tg_ctx_create(int device, void *stream, tg_ctx **out) {
    if (!out) return TG_ERR_NULL;
    *out = nullptr;
    int count = 0;
    if (hipGetDeviceCount(&count) != hipSuccess || count == 0) return TG_ERR_HIP;
    if (device < 0 || device >= count) return TG_ERR_ARG;
    if (hipSetDevice(device) != hipSuccess) return TG_ERR_HIP;
    hipDeviceProp_t prop;
    if (hipGetDeviceProperties(&prop, device) != hipSuccess) return TG_ERR_HIP;
    if (std::string(prop.gcnArchName).rfind("gfx950", 0) != 0) return TG_ERR_UNSUPPORTED;
    tg_ctx *ctx = new tg_ctx();
    ctx->device = device;
    if (stream) {
        ctx->stream = static_cast<hipStream_t>(stream);
    } else {
        if (hipStreamCreateWithFlags(&ctx->stream, hipStreamNonBlocking) != hipSuccess) {
            delete ctx;
            return TG_ERR_HIP;
        }
        ctx->own_stream = true;
    }
    *out = ctx;
    return TG_OK;
}

void tg_ctx_destroy(tg_ctx *ctx) {
    if (!ctx) return;
    (void)hipSetDevice(ctx->device);
    (void)hipStreamSynchronize(ctx->stream);
    for (void *p : {(void *)ctx->qa, (void *)ctx->exps, (void *)ctx->da, (void *)ctx->dc, (void *)ctx->dbias})
        if (p) (void)hipFree(p);
    if (ctx->hst) (void)hipHostFree(ctx->hst);
    if (ctx->own_stream) (void)hipStreamDestroy(ctx->stream);
    delete ctx;
}

int tg_ctx_set_mode(tg_ctx *ctx, uint32_t mode) {
    if (!ctx) return TG_ERR_NULL;
    if (mode > TG_MODE_EXACT) return fail(ctx, TG_ERR_ARG, "unknown mode");
    std::lock_guard<std::mutex> g(ctx->mu);
    ctx->mode = mode;
    return TG_OK;
}

uint32_t tg_ctx_mode(const tg_ctx *ctx) { return ctx ? ctx->mode : TG_MODE_FAST; }

const char *tg_last_error(const tg_ctx *ctx) { return ctx ? ctx->err.c_str() : "null context"; }

int tg_synchronize(tg_ctx *ctx) {
    if (!ctx) return TG_ERR_NULL;
    std::lock_guard<std::mutex> g(ctx->mu);
    TG_HIP(ctx, hipSetDevice(ctx->device));
    TG_HIP(ctx, hipStreamSynchronize(ctx->stream));
    return TG_OK;
}

int tg_weights_upload(tg_ctx *ctx, const uint8_t *values, size_t values_len, const float *scales, size_t n_scales,
                      uint32_t precision, size_t n, size_t k, tg_weights **out) {
    return upload(ctx, values, values_len, scales, n_scales, precision, n, k, out, false);
}

int tg_weights_upload_device(tg_ctx *ctx, const uint8_t *values, size_t values_len, const float *scales,
                             size_t n_scales, uint32_t precision, size_t n, size_t k, tg_weights **out) {
    return upload(ctx, values, values_len, scales, n_scales, precision, n, k, out, true);
}

void tg_weights_free(tg_weights *w) {
    if (!w) return;
    (void)hipSetDevice(w->device);
    (void)hipDeviceSynchronize();
    if (w->d.values) (void)hipFree(w->d.values);
    if (w->d.scales) (void)hipFree(w->d.scales);
    delete w;
}

size_t tg_weights_bytes(const tg_weights *w) {
    return w ? tg_panel_bytes(w->d.precision, w->d.n, w->d.k) + w->d.n_scales * sizeof(float) : 0;
}
size_t tg_weights_n(const tg_weights *w) { return w ? w->d.n : 0; }
size_t tg_weights_k(const tg_weights *w) { return w ? w->d.k : 0; }
uint32_t tg_weights_precision(const tg_weights *w) { return w ? w->d.precision : 0; }

int tg_matmul_device(tg_ctx *ctx, const float *a, size_t a_len, size_t lda, size_t m, const tg_weights *w, float *c,
                     size_t c_len, size_t ldc, const tg_epilogue *epi) {
    if (!ctx || !w) return fail(ctx, TG_ERR_NULL, "null context or weights");
    if (m == 0 || w->d.n == 0) return TG_OK;
    std::lock_guard<std::mutex> g(ctx->mu);
    int rc = check_matmul(ctx, a, a_len, lda, m, w, c, c_len, ldc, epi);
    if (rc) return rc;
    if (w->device != ctx->device) return fail(ctx, TG_ERR_ARG, "weights live on another device");
    TG_HIP(ctx, hipSetDevice(ctx->device));
    rc = run_device(ctx, a, lda, m, w, c, ldc, epi_args(epi, nullptr, false));
    if (rc == TG_OK) ctx->err.clear();
    return rc;
}

int tg_linear_device(tg_ctx *ctx, const float *a, size_t a_len, size_t m, const tg_weights *w, float *c,
                     size_t c_len, const tg_epilogue *epi) {
    if (!w) return fail(ctx, TG_ERR_NULL, "null weights");
    return tg_matmul_device(ctx, a, a_len, w->d.k, m, w, c, c_len, w->d.n, epi);
}

int tg_matmul(tg_ctx *ctx, const float *a, size_t a_len, size_t lda, size_t m, const tg_weights *w, float *c,
              size_t c_len, size_t ldc, const tg_epilogue *epi) {
    if (!ctx || !w) return fail(ctx, TG_ERR_NULL, "null context or weights");
    if (m == 0 || w->d.n == 0) return TG_OK;
    std::lock_guard<std::mutex> g(ctx->mu);
    int rc = check_matmul(ctx, a, a_len, lda, m, w, c, c_len, ldc, epi);
    if (rc) return rc;
    if (w->device != ctx->device) return fail(ctx, TG_ERR_ARG, "weights live on another device");
    TG_HIP(ctx, hipSetDevice(ctx->device));
    const size_t k = w->d.k, n = w->d.n;
    // Compact device copies: a as [m][k], c as [m][n]. The rows are gathered into pinned staging
    // ([m][k] then [m][n] floats) and move in one DMA each way; only the n columns of each row of
    // c are written back, so the columns between rows are never touched.
    const bool has_bias = epi && epi->bias, acc = epi && epi->accumulate;
    if ((rc = grow(ctx, ctx->da, ctx->da_cap, m * (k ? k : 1) * sizeof(float)))) return rc;
    if ((rc = grow(ctx, ctx->dc, ctx->dc_cap, m * n * sizeof(float)))) return rc;
    if (has_bias && (rc = grow(ctx, ctx->dbias, ctx->dbias_cap, n * sizeof(float)))) return rc;
    if ((rc = grow_host(ctx, (m * k + m * n + (has_bias ? n : 0)) * sizeof(float)))) return rc;
    float *ha = ctx->hst, *hc = ha + m * k, *hb = hc + m * n;
    if (k) {
        copy_rows(ha, k, a, lda, m, k);
        TG_HIP(ctx, hipMemcpyAsync(ctx->da, ha, m * k * 4, hipMemcpyHostToDevice, ctx->stream));
    }
    if (acc) {
        copy_rows(hc, n, c, ldc, m, n);
        TG_HIP(ctx, hipMemcpyAsync(ctx->dc, hc, m * n * 4, hipMemcpyHostToDevice, ctx->stream));
    }
    if (has_bias) {
        std::memcpy(hb, epi->bias, n * 4);
        TG_HIP(ctx, hipMemcpyAsync(ctx->dbias, hb, n * 4, hipMemcpyHostToDevice, ctx->stream));
    }
    rc = run_device(ctx, ctx->da, k, m, w, ctx->dc, n, epi_args(epi, ctx->dbias, has_bias));
    if (rc) return rc;
    TG_HIP(ctx, hipMemcpyAsync(hc, ctx->dc, m * n * 4, hipMemcpyDeviceToHost, ctx->stream));
    TG_HIP(ctx, hipStreamSynchronize(ctx->stream));
    copy_rows(c, ldc, hc, n, m, n);
    ctx->err.clear();
    return TG_OK;
}

int tg_linear(tg_ctx *ctx, const float *a, size_t a_len, size_t m, const tg_weights *w, float *c, size_t c_len,
              const tg_epilogue *epi) {
    if (!w) return fail(ctx, TG_ERR_NULL, "null weights");
    return tg_matmul(ctx, a, a_len, w->d.k, m, w, c, c_len, w->d.n, epi);
}

size_t tg_quant_bytes(size_t m, size_t k) { return tg::qa_bytes(m, k); }

int tg_quantize_rows_device(tg_ctx *ctx, const float *a, size_t a_len, size_t lda, size_t m, size_t k, void *qa,
                            size_t qa_len, int32_t *exps) {
    if (!ctx) return TG_ERR_NULL;
    if (m == 0) return TG_OK;
    if ((!a && k) || !qa || !exps) return fail(ctx, TG_ERR_NULL, "null buffer");
    if (lda < k || a_len < (m - 1) * lda + k) return fail(ctx, TG_ERR_SHAPE, "a is too short");
    if (qa_len < tg_quant_bytes(m, k)) return fail(ctx, TG_ERR_SHAPE, "qa is too short");
    if (k > tg::MAX_K_INT) return fail(ctx, TG_ERR_UNSUPPORTED, "k beyond the integer path's limit");
    std::lock_guard<std::mutex> g(ctx->mu);
    TG_HIP(ctx, hipSetDevice(ctx->device));
    TG_HIP(ctx, tg::launch_quantize_rows(a, lda, m, k, static_cast<uint8_t *>(qa), exps, ctx->stream));
    return TG_OK;
}

int tg_matmul_quantized_device(tg_ctx *ctx, const void *qa, size_t qa_len, const int32_t *exps, size_t m,
                               const tg_weights *w, float *c, size_t c_len, size_t ldc, const tg_epilogue *epi) {
    if (!ctx || !w) return fail(ctx, TG_ERR_NULL, "null context or weights");
    if (m == 0 || w->d.n == 0) return TG_OK;
    const size_t n = w->d.n;
    if ((w->d.precision != TG_INT8 && w->d.precision != TG_Q8_0) || w->d.k > tg::MAX_K_INT)
        return fail(ctx, TG_ERR_UNSUPPORTED, "the staged path takes int8 or Q8_0 weights with k <= 65536");
    if (!qa || !exps || !c) return fail(ctx, TG_ERR_NULL, "null buffer");
    if (qa_len < tg_quant_bytes(m, w->d.k)) return fail(ctx, TG_ERR_SHAPE, "qa is too short");
    if (ldc < n || c_len < (m - 1) * ldc + n) return fail(ctx, TG_ERR_SHAPE, "c is too short");
    if (epi && epi->bias && epi->bias_len < n) return fail(ctx, TG_ERR_SHAPE, "bias is too short");
    if (epi && epi->act > TG_ACT_SILU) return fail(ctx, TG_ERR_ARG, "unknown activation");
    if (w->device != ctx->device) return fail(ctx, TG_ERR_ARG, "weights live on another device");
    std::lock_guard<std::mutex> g(ctx->mu);
    TG_HIP(ctx, hipSetDevice(ctx->device));
    TG_HIP(ctx, tg::launch_gemm_i8(static_cast<const uint8_t *>(qa), exps, m, w->d, c, ldc,
                                   epi_args(epi, nullptr, false), ctx->stream));
    return TG_OK;
}

int tg_pack_upload_matrix(tg_ctx *ctx, const tg_pack *pack, const char *name, size_t n, size_t k,
                          tg_weights **out) {
    if (!ctx || !pack || !name || !out) return fail(ctx, TG_ERR_NULL, "null argument");
    *out = nullptr;
    tg_pack_entry e;
    if (tg_pack_find(pack, name, &e) != TG_OK) return fail(ctx, TG_ERR_ARG, tg_pack_last_error());
    const std::string head = std::string("The pack file isn't usable. Entry ") + name;
    if (e.type != TG_ENTRY_MATRIX) return fail(ctx, TG_ERR_ARG, head + " isn't a matrix.");
    if (e.n != n || e.k != k)
        return fail(ctx, TG_ERR_SHAPE, head + " is " + std::to_string(e.n) + " x " + std::to_string(e.k) +
                                           ", and the model needs " + std::to_string(n) + " x " + std::to_string(k) +
                                           ".");
    const int rc = tg_weights_upload(ctx, static_cast<const uint8_t *>(e.data), e.bytes, e.scales, e.n_scales,
                                     e.precision, n, k, out);
    if (rc == TG_ERR_ARG || rc == TG_ERR_ALIGN) return fail(ctx, rc, head + " doesn't fit its shape.");
    return rc;
}

int tg_layer_norm_device(tg_ctx *ctx, const float *x, size_t ldx, size_t m, size_t n, const float *gamma,
                         const float *beta, float eps, float *out, size_t ldo) {
    if (!ctx) return TG_ERR_NULL;
    if (m == 0 || n == 0) return TG_OK;
    if (!x || !gamma || !beta || !out) return fail(ctx, TG_ERR_NULL, "null buffer");
    if (ldx < n || ldo < n) return fail(ctx, TG_ERR_SHAPE, "ldx and ldo must be >= n");
    if (n > (size_t)INT32_MAX) return fail(ctx, TG_ERR_UNSUPPORTED, "rows longer than 2^31 values");
    std::lock_guard<std::mutex> g(ctx->mu);
    TG_HIP(ctx, hipSetDevice(ctx->device));
    TG_HIP(ctx, tg::launch_layer_norm(x, ldx, m, n, gamma, beta, eps, out, ldo, ctx->stream));
    return TG_OK;
}

int tg_glu_device(tg_ctx *ctx, const float *x, size_t ldx, size_t m, size_t half, float *out, size_t ldo) {
    if (!ctx) return TG_ERR_NULL;
    if (m == 0 || half == 0) return TG_OK;
    if (!x || !out) return fail(ctx, TG_ERR_NULL, "null buffer");
    if (ldx < 2 * half || ldo < half) return fail(ctx, TG_ERR_SHAPE, "ldx must be >= 2 half and ldo >= half");
    std::lock_guard<std::mutex> g(ctx->mu);
    TG_HIP(ctx, hipSetDevice(ctx->device));
    TG_HIP(ctx, tg::launch_glu(x, ldx, m, half, out, ldo, ctx->stream));
    return TG_OK;
}

int tg_dwconv1d_device(tg_ctx *ctx, const float *x, size_t ldx, size_t frames, size_t batch, size_t channels,
                       const float *w, size_t kernel, const float *bias, size_t t0, size_t stride, size_t rows,
                       uint32_t act, float *out, size_t ldo) {
    if (!ctx) return TG_ERR_NULL;
    if (act != TG_ACT_NONE && act != TG_ACT_SILU) return fail(ctx, TG_ERR_ARG, "act must be TG_ACT_NONE or TG_ACT_SILU");
    if (rows == 0 || channels == 0 || batch == 0) return TG_OK;
    if (!bias || !out || (frames > 0 && !x) || (kernel > 0 && !w)) return fail(ctx, TG_ERR_NULL, "null buffer");
    if (ldo < channels || (frames > 0 && ldx < channels)) return fail(ctx, TG_ERR_SHAPE, "ldx and ldo must be >= channels");
    const size_t lim = (size_t)1 << 40;  // frame indices and sizes stay far inside int64
    // the dispatch's x extent (rows / 8 blocks of 256 work-items) must stay below 2^32 work-items
    if (frames >= lim || kernel >= ((size_t)1 << 30) || t0 >= lim || stride >= lim || rows >= ((size_t)1 << 26))
        return fail(ctx, TG_ERR_UNSUPPORTED, "frames, t0 and stride must be < 2^40, rows < 2^26, kernel < 2^30");
    if (stride > 0 && rows - 1 > (lim - t0) / stride)
        return fail(ctx, TG_ERR_UNSUPPORTED, "the last row's frame t0 + (rows - 1) stride must be < 2^40");
    if (tg::div_ceil(channels, (size_t)256) >= 65536 || batch >= 65536 ||
        tg::div_ceil(rows, (size_t)8) * tg::div_ceil(channels, (size_t)256) * batch >= ((size_t)1 << 24))
        return fail(ctx, TG_ERR_UNSUPPORTED, "more than 2^24 channels, 65535 sequences or 2^35 outputs per call");
    if (frames > 0) {
        const size_t xn = ((batch * frames - 1) * ldx + channels) * 4, on = ((batch * rows - 1) * ldo + channels) * 4;
        const uintptr_t xb = reinterpret_cast<uintptr_t>(x), ob = reinterpret_cast<uintptr_t>(out);
        if (ob < xb + xn && xb < ob + on) return fail(ctx, TG_ERR_ARG, "out must not overlap x");
    }
    std::lock_guard<std::mutex> g(ctx->mu);
    TG_HIP(ctx, hipSetDevice(ctx->device));
    TG_HIP(ctx, tg::launch_dwconv1d(x, ldx, frames, batch, channels, w, kernel, bias, t0, stride, rows,
                                    act == TG_ACT_SILU, out, ldo, ctx->stream));
    return TG_OK;
}

}  // extern "C"
