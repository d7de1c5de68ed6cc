// The C ABI (include/telmo_hip.h, which cites the reference line each entry point replaces):
// contexts, device weights, argument checks with the reference's semantics, and dispatch to the
// kernels. Among them:
//
//   tg_matmul / tg_matmul_device   Kernels::matmul        src/kernels/mod.rs:657-688
//   tg_linear / tg_linear_device   Kernels::linear        src/kernels/mod.rs:691-701
//   tg_weights_upload              PackedWeights::from_parts  src/kernels/mod.rs:214-237
//
// Dispatch (fast mode, int8 and Q8_0 weights, k <= 65536): up to 16 rows that fit a GEMV
// (gemv_fits) take the MFMA GEMV, or for int8 the dot4 GEMV, in one launch; otherwise the row
// quantiser then the MFMA GEMM, whose kernel launch_gemm_i8 picks by shape. The exact mode, other
// precisions and longer inputs run the exact kernel.
#include <cstring>
#include <algorithm>
#include <mutex>
#include <string>
#include <vector>

#include "../../include/telmo_hip.h"
#include "tg_internal.hpp"

struct tg_ctx {
    int device = 0;
    hipStream_t stream = nullptr;
    bool own_stream = false;
    uint32_t mode = TG_MODE_FAST;
    std::mutex mu;
    // The last error message. Argument checks can fail before a call takes mu, so the message has
    // a mutex of its own; tg_last_error copies it under that mutex.
    std::mutex err_mu;
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
    // The product before the GLU, when tg_linear_glu_device cannot fuse them.
    float *dg = nullptr;
    size_t dg_cap = 0;
    // The quantised-output product's f32 rows and their per-tile row maxima, grown on demand.
    float *hid = nullptr;
    size_t hid_cap = 0;
    uint32_t *tmax = nullptr;
    size_t tmax_cap = 0;
    // The accuracy guard of the product entry points (tg::RowGuard): on unless turned off; its row
    // flags and the flagged rows' old outputs, grown on demand.
    bool guard = true;
    int32_t *flags = nullptr;
    size_t flags_cap = 0;
    float *save = nullptr;
    size_t save_cap = 0;
};

struct tg_weights {
    tg::DeviceWeights d;
    int device;
};

constexpr int TDT_GRAPH_STEPS = 16;
// Steps per resident launch: the host looks at the control block between launches.
constexpr int TDT_RESIDENT_STEPS = 16384;

// A TDT prediction network and joint on the device (the joint, projection, biases and embedding
// stay the caller's), with the interleaved LSTM copies and the buffers of its decode steps.
struct tg_tdt {
    tg::TdtNet net;
    int device = 0;
    tg::DeviceWeights lstm[tg::TDT_MAX_LAYERS];  // interleaved copies (owned values and scales)
    float *lstm_b[tg::TDT_MAX_LAYERS] = {};       // interleaved biases (owned)
    tg::TdtCtl *ctl = nullptr;                    // device control block
    tg::TdtCtl *ctl_host = nullptr;               // pinned copy
    int32_t *durations = nullptr;                 // device
    float *extras = nullptr;                      // the joint's first and duration logits per row
    float *scratch = nullptr;                     // TDT_ROWS states: the other buffer of a prediction
    void *partials = nullptr;
    int32_t *tokens = nullptr;                    // device, 3 int32 per token
    size_t tokens_cap = 0;                        // tokens the buffer holds
    // TDT_GRAPH_STEPS steps captured as one graph for the arguments in key (enc_proj, lde, frames,
    // state, pred, token buffer, its capacity), replayed until the decode ends.
    hipGraph_t graph = nullptr;
    hipGraphExec_t exec = nullptr;
    uintptr_t key[7] = {};
    // The resident decode: its plan (valid when can_resident), whether decodes use it, its
    // hand-over words and the longest wait of one workgroup for another (wall-clock ticks).
    tg::TdtPlan plan;
    bool can_resident = false, use_resident = false;
    uint64_t *words = nullptr;
    uint64_t wait_ticks = 0;
    uint64_t clock_khz = 100000;  // the device's wall clock, for tg_tdt_set_resident_limits
    int launch_steps = TDT_RESIDENT_STEPS;  // steps per resident launch
    // Whether the last tg_tdt_decode_device ran resident (1), by the step kernels (0), or none yet (-1).
    int last_resident = -1;
    // The multi-stream decode's control blocks (TDT_MAX_STREAMS, device and pinned), its hand-over
    // words and the streams' entry states and predictions (restored when a launch fails), made on
    // its first call.
    tg::TdtCtl *mctl = nullptr, *mctl_host = nullptr;
    uint64_t *mwords = nullptr;
    float *mscratch = nullptr;
    uint32_t last_steps = 0;  // steps of the last resident decode (one or several streams)
};


// The scratch of tg_matmul_device_noalloc, for callers that cannot allocate: the quantised rows of
// one product (the first NOALLOC_QA_BYTES; with the accuracy guard on and an accumulating
// epilogue, the flagged rows' old outputs after them), their row exponents (NOALLOC_ROWS int32
// after that region) and the guard's row flags (NOALLOC_ROWS int32 after the exponents).
// Each GPU the library runs on holds its own copy for the life of the process. Host code never uses
// the array's name as an address: tg_ctx_create takes each device's address with
// hipGetSymbolAddress, with that device current, and the kernels get that pointer.
constexpr size_t NOALLOC_SCRATCH_BYTES = (size_t)16 << 20;
constexpr size_t NOALLOC_ROWS = 16384;
constexpr size_t NOALLOC_QA_BYTES = NOALLOC_SCRATCH_BYTES - 2 * NOALLOC_ROWS * sizeof(int32_t);
static __device__ __align__(256) uint8_t scratch[NOALLOC_SCRATCH_BYTES];

namespace {

constexpr int MAX_DEVICES = 64;
// A resident decode holds most of a GPU's CUs for its whole launch, and two resident launches on one
// GPU cannot both be resident: one decode per device at a time holds this lock (try_lock); a decode
// that finds it taken runs on the step kernels, which share the GPU with it.
std::mutex resident_mu[MAX_DEVICES];
std::mutex scratch_mu;
void *scratch_ptr[MAX_DEVICES] = {};  // device address of `scratch` per device, once taken
hipError_t scratch_err[MAX_DEVICES] = {};

// Takes the address of `scratch` on `device` (the current device) the first time; later calls
// return it. hipSuccess with *out null never happens: a failure is returned and kept.
hipError_t scratch_address(int device, void **out) {
    *out = nullptr;
    if (device < 0 || device >= MAX_DEVICES) return hipErrorInvalidDevice;
    std::lock_guard<std::mutex> g(scratch_mu);
    if (!scratch_ptr[device] && scratch_err[device] == hipSuccess) {
        void *p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !p) scratch_err[device] = e != hipSuccess ? e : hipErrorInvalidSymbol;
        else scratch_ptr[device] = p;
    }
    *out = scratch_ptr[device];
    return scratch_err[device];
}

}  // namespace

namespace {

int fail(tg_ctx *ctx, int code, const std::string &msg) {
    if (ctx) {
        std::lock_guard<std::mutex> g(ctx->err_mu);
        ctx->err = msg;
    }
    return code;
}

void clear_error(tg_ctx *ctx) {
    std::lock_guard<std::mutex> g(ctx->err_mu);
    ctx->err.clear();
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

// (rows - 1) * ld + len, the elements a strided view of rows reads, or SIZE_MAX when that does not
// fit in size_t: no buffer is that long, so the length check fails instead of wrapping.
size_t span(size_t rows, size_t ld, size_t len) {
    if (rows == 0) return 0;
    if (ld != 0 && rows - 1 > (SIZE_MAX - len) / ld) return SIZE_MAX;
    return (rows - 1) * ld + len;
}

// The checks of Kernels::matmul (src/kernels/mod.rs:669-677), in its order.
int check_matmul(tg_ctx *ctx, const float *a, size_t a_len, size_t lda, size_t m, const tg_weights *w, float *c,
                 size_t c_len, size_t ldc, const tg_epilogue *epi) {
    const size_t k = w->d.k, n = w->d.n;
    if (lda < k || ldc < n) return fail(ctx, TG_ERR_SHAPE, "lda must be >= k and ldc >= n");
    if (a_len < span(m, lda, k)) return fail(ctx, TG_ERR_SHAPE, "a is too short");
    if (c_len < span(m, ldc, n)) return fail(ctx, TG_ERR_SHAPE, "c is too short");
    if (epi && epi->bias && epi->bias_len < n) return fail(ctx, TG_ERR_SHAPE, "bias is too short");
    if (epi && epi->act > TG_ACT_SILU) return fail(ctx, TG_ERR_ARG, "unknown activation");
    if (!a && k > 0) return fail(ctx, TG_ERR_NULL, "a is null");
    if (!c) return fail(ctx, TG_ERR_NULL, "c is null");
    if (m > (size_t)INT32_MAX) return fail(ctx, TG_ERR_UNSUPPORTED, "more than 2^31 - 1 rows");
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
    // The accuracy guard: the quantiser flags the rows whose two digits drop too much (keeping their
    // old outputs when the epilogue accumulates), the GEMM runs on every row, then the exact kernel
    // rewrites the flagged rows with the reference's fused sums.
    tg::RowGuard g;
    if (ctx->guard) {
        if ((rc = grow(ctx, ctx->flags, ctx->flags_cap, m * sizeof(int32_t)))) return rc;
        g.flags = ctx->flags;
        if (epi.accumulate) {
            if ((rc = grow(ctx, ctx->save, ctx->save_cap, m * d.n * sizeof(float)))) return rc;
            g.c = c;
            g.ldc = ldc;
            g.n = d.n;
            g.save = ctx->save;
        }
    }
    TG_HIP(ctx, tg::launch_quantize_rows(a, lda, m, d.k, ctx->qa, ctx->exps, ctx->stream, tg::RowAct{}, g));
    TG_HIP(ctx, tg::launch_gemm_i8(ctx->qa, ctx->exps, m, d, c, ldc, epi, ctx->stream));
    if (ctx->guard) TG_HIP(ctx, tg::launch_exact_rows(a, lda, m, d, c, ldc, epi, g.flags, g.save, ctx->stream));
    return TG_OK;
}

int upload(tg_ctx *ctx, const uint8_t *values, size_t values_len, const float *scales, size_t n_scales,
           uint32_t precision, size_t n, size_t k, tg_weights **out, bool from_device) {
    if (!ctx || !out) return fail(ctx, TG_ERR_NULL, "null argument");
    *out = nullptr;
    if (!valid_precision(precision)) return fail(ctx, TG_ERR_ARG, "unknown precision");
    // Sizes in which the panel byte count cannot wrap (and the kernels' 32-bit n and k hold).
    if (n > (size_t)INT32_MAX || k > (size_t)INT32_MAX || (n && k > ((size_t)1 << 48) / n))
        return fail(ctx, TG_ERR_UNSUPPORTED, "n and k must be < 2^31, with at most 2^48 weights");
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
    clear_error(ctx);
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
    // Set-up of the no-allocation scratch on this device, with the device current. A failure is
    // kept and reported by tg_matmul_device_noalloc; nothing else needs the scratch.
    void *scratch_dev = nullptr;
    (void)scratch_address(device, &scratch_dev);
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
    for (void *p : {(void *)ctx->qa, (void *)ctx->exps, (void *)ctx->da, (void *)ctx->dc, (void *)ctx->dbias,
                    (void *)ctx->dg, (void *)ctx->hid, (void *)ctx->tmax, (void *)ctx->flags, (void *)ctx->save})
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

int tg_ctx_set_guard(tg_ctx *ctx, int on) {
    if (!ctx) return TG_ERR_NULL;
    std::lock_guard<std::mutex> g(ctx->mu);
    ctx->guard = on != 0;
    return TG_OK;
}

int tg_ctx_guard(const tg_ctx *ctx) { return ctx && ctx->guard ? 1 : 0; }

const char *tg_last_error(const tg_ctx *ctx) {
    // The message is copied under its lock into storage of the calling thread, so another thread
    // failing or succeeding on the context meanwhile cannot free what the caller is reading.
    thread_local std::string copy;
    if (!ctx) return "null context";
    std::lock_guard<std::mutex> g(const_cast<tg_ctx *>(ctx)->err_mu);
    copy = ctx->err;
    return copy.c_str();
}

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
    if (rc == TG_OK) clear_error(ctx);
    return rc;
}

int tg_matmul_device_noalloc(tg_ctx *ctx, const float *a, size_t a_len, size_t lda, size_t m, const tg_weights *w,
                             float *c, size_t c_len, size_t ldc, const tg_epilogue *epi) {
    if (!ctx || !w) return fail(ctx, TG_ERR_NULL, "null context or weights");
    if (m == 0 || w->d.n == 0) return TG_OK;
    std::lock_guard<std::mutex> g(ctx->mu);
    int rc = check_matmul(ctx, a, a_len, lda, m, w, c, c_len, ldc, epi);
    if (rc) return rc;
    if (w->device != ctx->device) return fail(ctx, TG_ERR_ARG, "weights live on another device");
    const tg::DeviceWeights &d = w->d;
    const bool int_path = ctx->mode == TG_MODE_FAST && (d.precision == TG_INT8 || d.precision == TG_Q8_0) &&
                          d.k <= tg::MAX_K_INT;
    const bool staged = int_path && !tg::gemv_fits(m, d.k, a, lda, d.precision);
    if (staged && (m > NOALLOC_ROWS || tg::qa_bytes(m, d.k) > NOALLOC_QA_BYTES))
        return fail(ctx, TG_ERR_UNSUPPORTED,
                    "the product's quantised rows (" + std::to_string(tg::qa_bytes(m, d.k)) + " bytes, " +
                        std::to_string(m) + " rows) exceed the no-allocation scratch (" +
                        std::to_string(NOALLOC_QA_BYTES) + " bytes, " + std::to_string(NOALLOC_ROWS) + " rows)");
    // With the guard on, an accumulating product keeps its flagged rows' old outputs (m n floats)
    // after the quantised rows.
    const size_t qa_round = (tg::qa_bytes(m, d.k) + 255) / 256 * 256;
    const bool keep = staged && ctx->guard && epi && epi->accumulate;
    if (keep && (d.n > (NOALLOC_QA_BYTES - qa_round) / sizeof(float) / m))
        return fail(ctx, TG_ERR_UNSUPPORTED,
                    "with the accuracy guard on, an accumulating product keeps m x n floats beside its quantised "
                    "rows, which exceed the no-allocation scratch (" + std::to_string(NOALLOC_QA_BYTES) +
                        " bytes); turn the guard off (tg_ctx_set_guard) or split the rows");
    TG_HIP(ctx, hipSetDevice(ctx->device));
    const tg::EpiArgs e = epi_args(epi, nullptr, false);
    if (!int_path) {
        TG_HIP(ctx, tg::launch_exact(a, lda, m, d, c, ldc, e, ctx->stream));
    } else if (!staged) {
        TG_HIP(ctx, tg::launch_gemv_i8(a, lda, m, d, c, ldc, e, ctx->stream));
    } else {
        void *base = nullptr;
        const hipError_t se = scratch_address(ctx->device, &base);
        if (se != hipSuccess) return hip_fail(ctx, se, "hipGetSymbolAddress of the no-allocation scratch");
        // Every byte the GEMM reads into a stored output is written by the quantiser first (rows
        // past m in the last 16-row block feed only outputs that are never stored), so nothing in
        // the scratch needs clearing between calls.
        uint8_t *qa = static_cast<uint8_t *>(base);
        int32_t *exps = reinterpret_cast<int32_t *>(qa + NOALLOC_QA_BYTES);
        tg::RowGuard g;
        if (ctx->guard) {
            g.flags = exps + NOALLOC_ROWS;
            if (keep) {
                g.c = c;
                g.ldc = ldc;
                g.n = d.n;
                g.save = reinterpret_cast<float *>(qa + qa_round);
            }
        }
        TG_HIP(ctx, tg::launch_quantize_rows(a, lda, m, d.k, qa, exps, ctx->stream, tg::RowAct{}, g));
        TG_HIP(ctx, tg::launch_gemm_i8(qa, exps, m, d, c, ldc, e, ctx->stream));
        if (ctx->guard) TG_HIP(ctx, tg::launch_exact_rows(a, lda, m, d, c, ldc, e, g.flags, g.save, ctx->stream));
    }
    clear_error(ctx);
    return TG_OK;
}

int tg_matmul_rowmajor_device(tg_ctx *ctx, const float *a, size_t a_len, size_t lda, size_t m, const float *b,
                              size_t b_len, size_t k, size_t n, size_t ldb, float *c, size_t c_len, size_t ldc,
                              const tg_epilogue *epi) {
    if (!ctx) return TG_ERR_NULL;
    // BView::row_major's check (src/kernels/mod.rs:341-351): the view reads whole 16-column panels.
    if (n > 0 && k > 0) {
        const size_t last = span(k, ldb, (tg::div_ceil(n, (size_t)tg::PANEL) - 1) * tg::PANEL + tg::PANEL);
        if (b_len < last) return fail(ctx, TG_ERR_SHAPE, "the matrix view reads past its buffer");
        if (!b) return fail(ctx, TG_ERR_NULL, "b is null");
    }
    if (m == 0 || n == 0) return TG_OK;
    // Kernels::matmul's checks (src/kernels/mod.rs:669-677), in its order.
    if (lda < k || ldc < n) return fail(ctx, TG_ERR_SHAPE, "lda must be >= k and ldc >= n");
    if (a_len < span(m, lda, k)) return fail(ctx, TG_ERR_SHAPE, "a is too short");
    if (c_len < span(m, ldc, n)) return fail(ctx, TG_ERR_SHAPE, "c is too short");
    if (epi && epi->bias && epi->bias_len < n) return fail(ctx, TG_ERR_SHAPE, "bias is too short");
    if (epi && epi->act > TG_ACT_SILU) return fail(ctx, TG_ERR_ARG, "unknown activation");
    if (!a && k > 0) return fail(ctx, TG_ERR_NULL, "a is null");
    if (!c) return fail(ctx, TG_ERR_NULL, "c is null");
    if (k > (size_t)INT32_MAX || n > (size_t)INT32_MAX || m > (size_t)INT32_MAX)
        return fail(ctx, TG_ERR_UNSUPPORTED, "sizes beyond 2^31");
    std::lock_guard<std::mutex> g(ctx->mu);
    TG_HIP(ctx, hipSetDevice(ctx->device));
    TG_HIP(ctx, tg::launch_rowmajor(a, lda, m, k, b, ldb, n, c, ldc, epi_args(epi, nullptr, false), ctx->stream));
    clear_error(ctx);
    return TG_OK;
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
    clear_error(ctx);
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
    if (lda < k || a_len < span(m, lda, k)) return fail(ctx, TG_ERR_SHAPE, "a is too short");
    if (m > (size_t)INT32_MAX) return fail(ctx, TG_ERR_UNSUPPORTED, "more than 2^31 - 1 rows");
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
    if (ldc < n || c_len < span(m, ldc, n)) return fail(ctx, TG_ERR_SHAPE, "c is too short");
    if (m > (size_t)INT32_MAX) return fail(ctx, TG_ERR_UNSUPPORTED, "more than 2^31 - 1 rows");
    if (epi && epi->bias && epi->bias_len < n) return fail(ctx, TG_ERR_SHAPE, "bias is too short");
    if (epi && epi->act > TG_ACT_SILU) return fail(ctx, TG_ERR_ARG, "unknown activation");
    if (w->device != ctx->device) return fail(ctx, TG_ERR_ARG, "weights live on another device");
    std::lock_guard<std::mutex> g(ctx->mu);
    TG_HIP(ctx, hipSetDevice(ctx->device));
    TG_HIP(ctx, tg::launch_gemm_i8(static_cast<const uint8_t *>(qa), exps, m, w->d, c, ldc,
                                   epi_args(epi, nullptr, false), ctx->stream));
    return TG_OK;
}

int tg_matmul_quantized_glu_device(tg_ctx *ctx, const void *qa, size_t qa_len, const int32_t *exps, size_t m,
                                   const tg_weights *w, float *out, size_t out_len, size_t ldo,
                                   const tg_epilogue *epi) {
    if (!ctx || !w) return fail(ctx, TG_ERR_NULL, "null context or weights");
    const size_t n = w->d.n, half = n / 2;
    if (n % 2) return fail(ctx, TG_ERR_SHAPE, "the product's outputs must be an even count");
    if (epi && epi->accumulate) return fail(ctx, TG_ERR_ARG, "the GLU's input is not accumulated");
    if (m == 0 || n == 0) return TG_OK;
    const bool q8 = w->d.precision == TG_Q8_0;
    if ((w->d.precision != TG_INT8 && !q8) || w->d.k > tg::MAX_K_INT || (!q8 && !tg::gemm_glu_fits(n)) ||
        ctx->mode != TG_MODE_FAST)
        return fail(ctx, TG_ERR_UNSUPPORTED,
                    "the quantised GLU product takes int8 weights with n a multiple of 64, or Q8_0 weights, k <= "
                    "65536, in fast mode");
    if (!qa || !exps || !out) return fail(ctx, TG_ERR_NULL, "null buffer");
    if (qa_len < tg_quant_bytes(m, w->d.k)) return fail(ctx, TG_ERR_SHAPE, "qa is too short");
    if (ldo < half) return fail(ctx, TG_ERR_SHAPE, "ldo must be >= n / 2");
    if (out_len < span(m, ldo, half)) return fail(ctx, TG_ERR_SHAPE, "out is too short");
    if (m > (size_t)INT32_MAX) return fail(ctx, TG_ERR_UNSUPPORTED, "more than 2^31 - 1 rows");
    if (epi && epi->bias && epi->bias_len < n) return fail(ctx, TG_ERR_SHAPE, "bias is too short");
    if (epi && epi->act > TG_ACT_SILU) return fail(ctx, TG_ERR_ARG, "unknown activation");
    if (w->device != ctx->device) return fail(ctx, TG_ERR_ARG, "weights live on another device");
    std::lock_guard<std::mutex> g(ctx->mu);
    TG_HIP(ctx, hipSetDevice(ctx->device));
    if (q8 && !tg::gemm_glu_fits(n)) {
        // Q8_0 with n not a multiple of 64: the product's [m, n] rows through the context's buffer,
        // then the GLU kernel (the bits of tg_matmul_quantized_device followed by tg_glu_device,
        // which the fused product also gives).
        int rc = grow(ctx, ctx->dg, ctx->dg_cap, m * n * sizeof(float));
        if (rc) return rc;
        TG_HIP(ctx, tg::launch_gemm_i8(static_cast<const uint8_t *>(qa), exps, m, w->d, ctx->dg, n,
                                       epi_args(epi, nullptr, false), ctx->stream));
        TG_HIP(ctx, tg::launch_glu(ctx->dg, n, m, half, out, ldo, ctx->stream));
    } else {
        TG_HIP(ctx, tg::launch_gemm_i8_glu(static_cast<const uint8_t *>(qa), exps, m, w->d, out, ldo,
                                           epi_args(epi, nullptr, false), ctx->stream));
    }
    clear_error(ctx);
    return TG_OK;
}

// Rows from which the quantised-output product leaves an activation or a scale to the quantiser
// rather than to its own epilogue (1024 -> 4096 with SiLU, measured: at 12000 rows 212 us against
// 228 for the product that gathers row maxima; at 750 rows 20.6 us in the epilogue, 21.9 in the
// quantiser, 22.2 with the row maxima).
constexpr size_t QOUT_ACT_ROWS = 2048;

int tg_matmul_quantized_to_quant_device(tg_ctx *ctx, const void *qa, size_t qa_len, const int32_t *exps, size_t m,
                                        const tg_weights *w, const tg_epilogue *epi, void *qa_out,
                                        size_t qa_out_len, int32_t *exps_out, size_t exps_out_len) {
    if (!ctx || !w) return fail(ctx, TG_ERR_NULL, "null context or weights");
    if (m == 0 || w->d.n == 0) return TG_OK;
    const size_t n = w->d.n;
    const bool q8 = w->d.precision == TG_Q8_0;
    if ((w->d.precision != TG_INT8 && !q8) || w->d.k > tg::MAX_K_INT || ctx->mode != TG_MODE_FAST)
        return fail(ctx, TG_ERR_UNSUPPORTED,
                    "the quantised-output product takes int8 or Q8_0 weights with k <= 65536 in fast mode");
    if (n > tg::MAX_K_INT) return fail(ctx, TG_ERR_UNSUPPORTED, "outputs beyond the integer path's limit (65536)");
    if (!qa || !exps || !qa_out || !exps_out) return fail(ctx, TG_ERR_NULL, "null buffer");
    if (qa_len < tg_quant_bytes(m, w->d.k)) return fail(ctx, TG_ERR_SHAPE, "qa is too short");
    if (qa_out_len < tg_quant_bytes(m, n)) return fail(ctx, TG_ERR_SHAPE, "qa_out is too short");
    if (exps_out_len < m) return fail(ctx, TG_ERR_SHAPE, "exps_out must hold m exponents");
    if (m > (size_t)INT32_MAX) return fail(ctx, TG_ERR_UNSUPPORTED, "more than 2^31 - 1 rows");
    if (epi && epi->accumulate) return fail(ctx, TG_ERR_ARG, "quantised outputs are not accumulated");
    if (epi && epi->bias && epi->bias_len < n) return fail(ctx, TG_ERR_SHAPE, "bias is too short");
    if (epi && epi->act > TG_ACT_SILU) return fail(ctx, TG_ERR_ARG, "unknown activation");
    if (w->device != ctx->device) return fail(ctx, TG_ERR_ARG, "weights live on another device");
    if (qa == qa_out || exps == exps_out) return fail(ctx, TG_ERR_ARG, "the output must not overwrite the input");
    std::lock_guard<std::mutex> g(ctx->mu);
    TG_HIP(ctx, hipSetDevice(ctx->device));
    // The f32 rows (row stride kb * 64, so every 16-byte load of the quantiser stays inside) and
    // the row maxima, grown before any launch reads them; every element read is written first.
    const size_t ldh = tg::div_ceil(n, (size_t)tg::KBLK) * tg::KBLK;
    const int strips = tg::gemm_qout_strips(m, w->d);
    const tg::EpiArgs ea = epi_args(epi, nullptr, false);
    int rc;
    if ((rc = grow(ctx, ctx->hid, ctx->hid_cap, m * ldh * sizeof(float)))) return rc;
    const bool shaped = ea.act != tg::ACT_NONE || ea.scale != 1.0f;
    if (q8 || shaped) {
        // The product's f32 rows, then the row quantiser: for Q8_0 weights (the product that gathers
        // row maxima is int8 only), and for an activation or a scale other than 1. From QOUT_ACT_ROWS
        // rows those are VALU work that the product's epilogue adds to its MFMA loop, where it is not
        // hidden; the quantiser then applies them to each input as it loads it (the same f32
        // operations on the same values), under its memory time, and the product writes only the
        // biased sums.
        const bool later = shaped && m >= QOUT_ACT_ROWS;
        const tg::EpiArgs first = later ? tg::EpiArgs{ea.bias, tg::ACT_NONE, 1.0f, 0} : ea;
        TG_HIP(ctx, tg::launch_gemm_i8(static_cast<const uint8_t *>(qa), exps, m, w->d, ctx->hid, ldh, first,
                                       ctx->stream));
        TG_HIP(ctx, tg::launch_quantize_rows(ctx->hid, ldh, m, n, static_cast<uint8_t *>(qa_out), exps_out,
                                             ctx->stream, later ? tg::RowAct{ea.act, ea.scale} : tg::RowAct{}));
    } else {
        // The identity epilogue (a bias at most): the product keeps each row's largest magnitude per
        // column strip, and the quantiser reads those instead of a pass over the row.
        if ((rc = grow(ctx, ctx->tmax, ctx->tmax_cap, m * (size_t)strips * sizeof(uint32_t)))) return rc;
        TG_HIP(ctx, tg::launch_gemm_i8_qout(static_cast<const uint8_t *>(qa), exps, m, w->d, ea, ctx->hid, ldh,
                                            ctx->tmax, ctx->stream));
        TG_HIP(ctx, tg::launch_quantize_known(ctx->hid, ldh, m, n, ctx->tmax, strips, static_cast<uint8_t *>(qa_out),
                                              exps_out, ctx->stream));
    }
    clear_error(ctx);
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

int tg_layer_norm_device(tg_ctx *ctx, const float *x, size_t x_len, size_t ldx, size_t m, size_t n,
                         const float *gamma, size_t gamma_len, const float *beta, size_t beta_len, float eps,
                         float *out, size_t out_len, size_t ldo) {
    if (!ctx) return TG_ERR_NULL;
    if (m == 0 || n == 0) return TG_OK;
    if (!x || !gamma || !beta || !out) return fail(ctx, TG_ERR_NULL, "null buffer");
    if (ldx < n || ldo < n) return fail(ctx, TG_ERR_SHAPE, "ldx and ldo must be >= n");
    // The reference's assert (src/kernels/avx512.rs:348): out, gamma and beta hold the row's n values.
    if (x_len < span(m, ldx, n)) return fail(ctx, TG_ERR_SHAPE, "x is too short");
    if (out_len < span(m, ldo, n)) return fail(ctx, TG_ERR_SHAPE, "out is too short");
    if (gamma_len < n || beta_len < n) return fail(ctx, TG_ERR_SHAPE, "gamma and beta must hold n values");
    if (n > (size_t)INT32_MAX) return fail(ctx, TG_ERR_UNSUPPORTED, "rows longer than 2^31 values");
    std::lock_guard<std::mutex> g(ctx->mu);
    TG_HIP(ctx, hipSetDevice(ctx->device));
    TG_HIP(ctx, tg::launch_layer_norm(x, ldx, m, n, gamma, beta, eps, out, ldo, ctx->stream));
    return TG_OK;
}

int tg_layer_norm_quant_device(tg_ctx *ctx, const float *x, size_t x_len, size_t ldx, size_t m, size_t n,
                               const float *gamma, size_t gamma_len, const float *beta, size_t beta_len, float eps,
                               float *out, size_t out_len, size_t ldo, void *qa, size_t qa_len, int32_t *exps,
                               size_t exps_len) {
    if (!ctx) return TG_ERR_NULL;
    if (m == 0) return TG_OK;
    if (!x || !gamma || !beta || !qa || !exps) return fail(ctx, TG_ERR_NULL, "null buffer");
    if (n == 0) return fail(ctx, TG_ERR_SHAPE, "rows of no values have no LayerNorm to quantise");
    if (ldx < n || (out && ldo < n)) return fail(ctx, TG_ERR_SHAPE, "ldx and ldo must be >= n");
    if (x_len < span(m, ldx, n)) return fail(ctx, TG_ERR_SHAPE, "x is too short");
    if (out && out_len < span(m, ldo, n)) return fail(ctx, TG_ERR_SHAPE, "out is too short");
    if (gamma_len < n || beta_len < n) return fail(ctx, TG_ERR_SHAPE, "gamma and beta must hold n values");
    if (qa_len < tg_quant_bytes(m, n)) return fail(ctx, TG_ERR_SHAPE, "qa is too short");
    if (exps_len < m) return fail(ctx, TG_ERR_SHAPE, "exps must hold m exponents");
    if (n > tg::MAX_K_INT) return fail(ctx, TG_ERR_UNSUPPORTED, "rows beyond the integer path's limit (65536)");
    if (m > (size_t)INT32_MAX) return fail(ctx, TG_ERR_UNSUPPORTED, "more than 2^31 - 1 rows");
    std::lock_guard<std::mutex> g(ctx->mu);
    TG_HIP(ctx, hipSetDevice(ctx->device));
    TG_HIP(ctx, tg::launch_layer_norm_quant(x, ldx, m, n, gamma, beta, eps, out, ldo, static_cast<uint8_t *>(qa), exps,
                                            ctx->stream));
    clear_error(ctx);
    return TG_OK;
}

int tg_layer_norm_pair_quant_device(tg_ctx *ctx, float *x, size_t x_len, size_t ldx, size_t m, size_t n,
                                    const float *gamma, size_t gamma_len, const float *beta, size_t beta_len,
                                    float eps, const float *gamma2, size_t gamma2_len, const float *beta2,
                                    size_t beta2_len, float eps2, void *qa, size_t qa_len, int32_t *exps,
                                    size_t exps_len) {
    if (!ctx) return TG_ERR_NULL;
    if (m == 0) return TG_OK;
    if (!x || !gamma || !beta || !gamma2 || !beta2 || !qa || !exps) return fail(ctx, TG_ERR_NULL, "null buffer");
    if (n == 0) return fail(ctx, TG_ERR_SHAPE, "rows of no values have no LayerNorm to quantise");
    if (ldx < n) return fail(ctx, TG_ERR_SHAPE, "ldx must be >= n");
    if (x_len < span(m, ldx, n)) return fail(ctx, TG_ERR_SHAPE, "x is too short");
    if (gamma_len < n || beta_len < n || gamma2_len < n || beta2_len < n)
        return fail(ctx, TG_ERR_SHAPE, "gamma, beta, gamma2 and beta2 must hold n values");
    if (qa_len < tg_quant_bytes(m, n)) return fail(ctx, TG_ERR_SHAPE, "qa is too short");
    if (exps_len < m) return fail(ctx, TG_ERR_SHAPE, "exps must hold m exponents");
    if (n > tg::MAX_K_INT) return fail(ctx, TG_ERR_UNSUPPORTED, "rows beyond the integer path's limit (65536)");
    if (m > (size_t)INT32_MAX) return fail(ctx, TG_ERR_UNSUPPORTED, "more than 2^31 - 1 rows");
    std::lock_guard<std::mutex> g(ctx->mu);
    TG_HIP(ctx, hipSetDevice(ctx->device));
    TG_HIP(ctx, tg::launch_layer_norm_pair(x, ldx, m, n, gamma, beta, eps, x, ldx, gamma2, beta2, eps2,
                                           static_cast<uint8_t *>(qa), exps, ctx->stream));
    clear_error(ctx);
    return TG_OK;
}

int tg_glu_device(tg_ctx *ctx, const float *x, size_t x_len, size_t ldx, size_t m, size_t half, float *out,
                  size_t out_len, size_t ldo) {
    if (!ctx) return TG_ERR_NULL;
    if (m == 0 || half == 0) return TG_OK;
    if (!x || !out) return fail(ctx, TG_ERR_NULL, "null buffer");
    if (half > SIZE_MAX / 2 || ldx < 2 * half || ldo < half)
        return fail(ctx, TG_ERR_SHAPE, "ldx must be >= 2 half and ldo >= half");
    // The reference's assert (src/kernels/avx512.rs:412): both halves of each row are there.
    if (x_len < span(m, ldx, 2 * half)) return fail(ctx, TG_ERR_SHAPE, "x is too short");
    if (out_len < span(m, ldo, half)) return fail(ctx, TG_ERR_SHAPE, "out is too short");
    std::lock_guard<std::mutex> g(ctx->mu);
    TG_HIP(ctx, hipSetDevice(ctx->device));
    TG_HIP(ctx, tg::launch_glu(x, ldx, m, half, out, ldo, ctx->stream));
    return TG_OK;
}

int tg_softmax_device(tg_ctx *ctx, float *x, size_t x_len, size_t ldx, size_t m, size_t n) {
    if (!ctx) return TG_ERR_NULL;
    if (m == 0 || n == 0) return TG_OK;
    if (!x) return fail(ctx, TG_ERR_NULL, "null buffer");
    if (ldx < n) return fail(ctx, TG_ERR_SHAPE, "ldx must be >= n");
    if (x_len < span(m, ldx, n)) return fail(ctx, TG_ERR_SHAPE, "x is too short");
    if (n > (size_t)INT32_MAX) return fail(ctx, TG_ERR_UNSUPPORTED, "rows longer than 2^31 values");
    std::lock_guard<std::mutex> g(ctx->mu);
    TG_HIP(ctx, hipSetDevice(ctx->device));
    TG_HIP(ctx, tg::launch_softmax(x, ldx, m, n, ctx->stream));
    return TG_OK;
}

int tg_average_pairs_device(tg_ctx *ctx, const float *x, size_t x_len, size_t ldx, size_t frames, size_t batch,
                            size_t n, float *out, size_t out_len, size_t ldo) {
    if (!ctx) return TG_ERR_NULL;
    const size_t rows = frames / 2;
    if (rows == 0 || batch == 0 || n == 0) return TG_OK;
    if (!x || !out) return fail(ctx, TG_ERR_NULL, "null buffer");
    if (ldx < n || ldo < n) return fail(ctx, TG_ERR_SHAPE, "ldx and ldo must be >= n");
    if (frames > SIZE_MAX / batch || rows * batch > SIZE_MAX / n)
        return fail(ctx, TG_ERR_SHAPE, "frames x batch x n overflows");
    // Rows b frames + 2 r + 1 for r < frames / 2 are read; a last odd frame is not.
    const size_t last_in = (batch - 1) * frames + 2 * rows;
    if (x_len < span(last_in, ldx, n)) return fail(ctx, TG_ERR_SHAPE, "x is too short");
    if (out_len < span(rows * batch, ldo, n)) return fail(ctx, TG_ERR_SHAPE, "out is too short");
    const uintptr_t x0 = reinterpret_cast<uintptr_t>(x), o0 = reinterpret_cast<uintptr_t>(out);
    if (x0 < o0 + span(rows * batch, ldo, n) * sizeof(float) && o0 < x0 + span(last_in, ldx, n) * sizeof(float))
        return fail(ctx, TG_ERR_ARG, "out must not overlap x");
    std::lock_guard<std::mutex> g(ctx->mu);
    TG_HIP(ctx, hipSetDevice(ctx->device));
    TG_HIP(ctx, tg::launch_average_pairs(x, ldx, frames, batch, n, out, ldo, ctx->stream));
    return TG_OK;
}

int tg_linear_glu_device(tg_ctx *ctx, const float *a, size_t a_len, size_t m, const tg_weights *w, float *out,
                         size_t out_len, size_t ldo, const tg_epilogue *epi) {
    if (!ctx || !w) return fail(ctx, TG_ERR_NULL, "null context or weights");
    const size_t k = w->d.k, n = w->d.n, half = n / 2;
    if (n % 2) return fail(ctx, TG_ERR_SHAPE, "the product's outputs must be an even count");
    if (epi && epi->accumulate) return fail(ctx, TG_ERR_ARG, "the GLU's input is not accumulated");
    if (m == 0 || n == 0) return TG_OK;
    std::lock_guard<std::mutex> g(ctx->mu);
    // tg_linear_device's checks on a and the epilogue, then the GLU output's.
    if (a_len < span(m, k, k)) return fail(ctx, TG_ERR_SHAPE, "a is too short");
    if (epi && epi->bias && epi->bias_len < n) return fail(ctx, TG_ERR_SHAPE, "bias is too short");
    if (epi && epi->act > TG_ACT_SILU) return fail(ctx, TG_ERR_ARG, "unknown activation");
    if (!a && k > 0) return fail(ctx, TG_ERR_NULL, "a is null");
    if (ldo < half) return fail(ctx, TG_ERR_SHAPE, "ldo must be >= n / 2");
    if (out_len < span(m, ldo, half)) return fail(ctx, TG_ERR_SHAPE, "out is too short");
    if (m > (size_t)INT32_MAX) return fail(ctx, TG_ERR_UNSUPPORTED, "more than 2^31 - 1 rows");
    if (!out) return fail(ctx, TG_ERR_NULL, "out is null");
    if (w->device != ctx->device) return fail(ctx, TG_ERR_ARG, "weights live on another device");
    TG_HIP(ctx, hipSetDevice(ctx->device));
    const tg::EpiArgs e = epi_args(epi, nullptr, false);
    const tg::DeviceWeights &d = w->d;
    int rc;
    if (ctx->mode == TG_MODE_FAST && d.precision == TG_INT8 && d.k <= tg::MAX_K_INT && tg::gemm_glu_fits(n) &&
        !tg::gemv_fits(m, k, a, k, d.precision)) {
        // One GEMM whose epilogue applies the GLU: the product never leaves the chip.
        if ((rc = grow(ctx, ctx->qa, ctx->qa_cap, tg::qa_bytes(m, k)))) return rc;
        if ((rc = grow(ctx, ctx->exps, ctx->exps_cap, m * sizeof(int32_t)))) return rc;
        TG_HIP(ctx, tg::launch_quantize_rows(a, k, m, k, ctx->qa, ctx->exps, ctx->stream));
        TG_HIP(ctx, tg::launch_gemm_i8_glu(ctx->qa, ctx->exps, m, d, out, ldo, e, ctx->stream));
    } else {
        // The product into the context's buffer, then the GLU.
        if ((rc = grow(ctx, ctx->dg, ctx->dg_cap, m * n * sizeof(float)))) return rc;
        if ((rc = run_device(ctx, a, k, m, w, ctx->dg, n, e))) return rc;
        TG_HIP(ctx, tg::launch_glu(ctx->dg, n, m, half, out, ldo, ctx->stream));
    }
    clear_error(ctx);
    return TG_OK;
}

int tg_dwconv1d_device(tg_ctx *ctx, const float *x, size_t x_len, size_t ldx, size_t frames, size_t batch,
                       size_t channels, const float *w, size_t w_len, size_t kernel, const float *bias,
                       size_t bias_len, size_t t0, size_t stride, size_t rows, uint32_t act, float *out,
                       size_t out_len, size_t ldo) {
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
    // The slices dwconv1d_frame indexes (src/kernels/scalar.rs:174-182): the bias and each tap's
    // channels, the input frames and the output rows.
    if (bias_len < channels) return fail(ctx, TG_ERR_SHAPE, "bias is too short");
    if (kernel > 0 && (channels > SIZE_MAX / kernel || w_len < kernel * channels))
        return fail(ctx, TG_ERR_SHAPE, "w is too short");
    if (batch > SIZE_MAX / (frames > rows ? frames : rows)) return fail(ctx, TG_ERR_SHAPE, "x is too short");
    if (frames > 0 && x_len < span(batch * frames, ldx, channels)) return fail(ctx, TG_ERR_SHAPE, "x is too short");
    if (out_len < span(batch * rows, ldo, channels)) return fail(ctx, TG_ERR_SHAPE, "out is too short");
    if (tg::div_ceil(channels, (size_t)256) >= 65536 || batch >= 65536 ||
        tg::div_ceil(rows, (size_t)8) * tg::div_ceil(channels, (size_t)256) * batch >= ((size_t)1 << 24))
        return fail(ctx, TG_ERR_UNSUPPORTED, "more than 2^24 channels, 65535 sequences or 2^35 outputs per call");
    if (frames > 0) {
        // the bytes each view spans, saturated rather than wrapped
        const size_t xs = span(batch * frames, ldx, channels), os = span(batch * rows, ldo, channels);
        const size_t xn = xs > SIZE_MAX / 4 ? SIZE_MAX : xs * 4, on = os > SIZE_MAX / 4 ? SIZE_MAX : os * 4;
        const uintptr_t xb = reinterpret_cast<uintptr_t>(x), ob = reinterpret_cast<uintptr_t>(out);
        if (xn && on && (ob >= xb ? ob - xb < xn : xb - ob < on))
            return fail(ctx, TG_ERR_ARG, "out must not overlap x");
    }
    std::lock_guard<std::mutex> g(ctx->mu);
    TG_HIP(ctx, hipSetDevice(ctx->device));
    TG_HIP(ctx, tg::launch_dwconv1d(x, ldx, frames, batch, channels, w, kernel, bias, t0, stride, rows,
                                    act == TG_ACT_SILU, out, ldo, ctx->stream));
    return TG_OK;
}

int tg_dwconv1d_quant_device(tg_ctx *ctx, const float *x, size_t x_len, size_t ldx, size_t frames, size_t batch,
                             size_t channels, const float *w, size_t w_len, size_t kernel, const float *bias,
                             size_t bias_len, uint32_t act, float *out, size_t out_len, size_t ldo, void *qa,
                             size_t qa_len, int32_t *exps, size_t exps_len) {
    if (!ctx) return TG_ERR_NULL;
    if (act != TG_ACT_NONE && act != TG_ACT_SILU) return fail(ctx, TG_ERR_ARG, "act must be TG_ACT_NONE or TG_ACT_SILU");
    if (frames == 0 || channels == 0 || batch == 0) return TG_OK;
    if (!x || !w || !bias || !qa || !exps) return fail(ctx, TG_ERR_NULL, "null buffer");
    if (!tg::dwconv_quant_fits(channels, kernel))
        return fail(ctx, TG_ERR_UNSUPPORTED, "channels must be 1 .. 2048 and kernel 1 .. 32");
    if (ldx < channels || (out && ldo < channels)) return fail(ctx, TG_ERR_SHAPE, "ldx and ldo must be >= channels");
    if (frames > (size_t)INT32_MAX || batch > (size_t)INT32_MAX / frames)
        return fail(ctx, TG_ERR_UNSUPPORTED, "more than 2^31 - 1 rows");
    const size_t total = frames * batch;
    if (bias_len < channels) return fail(ctx, TG_ERR_SHAPE, "bias is too short");
    if (w_len < kernel * channels) return fail(ctx, TG_ERR_SHAPE, "w is too short");
    if (x_len < span(total, ldx, channels)) return fail(ctx, TG_ERR_SHAPE, "x is too short");
    if (out && out_len < span(total, ldo, channels)) return fail(ctx, TG_ERR_SHAPE, "out is too short");
    if (qa_len < tg_quant_bytes(total, channels)) return fail(ctx, TG_ERR_SHAPE, "qa is too short");
    if (exps_len < total) return fail(ctx, TG_ERR_SHAPE, "exps is too short");
    if (out) {
        // the bytes each view spans (each span is below 2^31 rows of at most ldx or ldo floats)
        const size_t xs = span(total, ldx, channels), os = span(total, ldo, channels);
        const size_t xn = xs > SIZE_MAX / 4 ? SIZE_MAX : xs * 4, on = os > SIZE_MAX / 4 ? SIZE_MAX : os * 4;
        const uintptr_t xb = reinterpret_cast<uintptr_t>(x), ob = reinterpret_cast<uintptr_t>(out);
        if (ob >= xb ? ob - xb < xn : xb - ob < on) return fail(ctx, TG_ERR_ARG, "out must not overlap x");
    }
    std::lock_guard<std::mutex> g(ctx->mu);
    TG_HIP(ctx, hipSetDevice(ctx->device));
    TG_HIP(ctx, tg::launch_dwconv_quant(x, ldx, frames, batch, channels, w, kernel, bias, act == TG_ACT_SILU, out, ldo,
                                        static_cast<uint8_t *>(qa), exps, ctx->stream));
    return TG_OK;
}

/* ---- the TDT decode -------------------------------------------------------------------------- */

namespace {

void tdt_drop_graph(tg_tdt *t) {
    if (t->exec) (void)hipGraphExecDestroy(t->exec);
    if (t->graph) (void)hipGraphDestroy(t->graph);
    t->exec = nullptr;
    t->graph = nullptr;
}

void tdt_release(tg_tdt *t) {
    if (!t) return;
    tdt_drop_graph(t);
    for (int l = 0; l < tg::TDT_MAX_LAYERS; l++) {
        if (t->lstm[l].values) (void)hipFree(t->lstm[l].values);
        if (t->lstm[l].scales) (void)hipFree(t->lstm[l].scales);
        if (t->lstm_b[l]) (void)hipFree(t->lstm_b[l]);
    }
    if (t->ctl) (void)hipFree(t->ctl);
    if (t->ctl_host) (void)hipHostFree(t->ctl_host);
    if (t->durations) (void)hipFree(t->durations);
    if (t->extras) (void)hipFree(t->extras);
    if (t->scratch) (void)hipFree(t->scratch);
    if (t->partials) (void)hipFree(t->partials);
    if (t->tokens) (void)hipFree(t->tokens);
    if (t->words) (void)hipFree(t->words);
    if (t->mctl) (void)hipFree(t->mctl);
    if (t->mctl_host) (void)hipHostFree(t->mctl_host);
    if (t->mwords) (void)hipFree(t->mwords);
    if (t->mscratch) (void)hipFree(t->mscratch);
    delete t;
}

bool aligned16(const void *p) { return reinterpret_cast<uintptr_t>(p) % 16 == 0; }

// A matrix of the network: present, on the context's device, int8 or Q8_0, of the given shape.
int tdt_matrix(tg_ctx *ctx, const tg_weights *w, size_t n, size_t k, const char *what) {
    if (!w) return fail(ctx, TG_ERR_NULL, std::string(what) + " is null");
    if (w->device != ctx->device) return fail(ctx, TG_ERR_ARG, std::string(what) + " lives on another device");
    if (w->d.precision != tg::INT8 && w->d.precision != tg::Q8_0)
        return fail(ctx, TG_ERR_UNSUPPORTED, std::string(what) + ": the TDT step takes int8 or Q8_0 weights");
    if (w->d.n != n || w->d.k != k)
        return fail(ctx, TG_ERR_SHAPE, std::string(what) + " is " + std::to_string(w->d.n) + " x " +
                                           std::to_string(w->d.k) + ", and the network needs " + std::to_string(n) +
                                           " x " + std::to_string(k));
    return TG_OK;
}

// The decode's outputs from the control block: frame, on_frame, the token count and the tokens.
int tdt_results(tg_ctx *ctx, tg_tdt *tdt, const tg::TdtCtl *hc, size_t *frame, size_t *on_frame, tg_token *tokens,
                size_t cap, size_t *count) {
    const size_t n = (size_t)hc->ntok;
    *frame = (size_t)hc->t;
    *on_frame = (size_t)hc->on_frame;
    *count = n;
    const size_t copy = n < cap ? n : cap;
    if (copy) {
        std::vector<int32_t> buf(copy * 3);
        TG_HIP(ctx, hipMemcpy(buf.data(), tdt->tokens, copy * 3 * sizeof(int32_t), hipMemcpyDeviceToHost));
        for (size_t i = 0; i < copy; i++)
            tokens[i] = tg_token{(uint32_t)buf[3 * i], (uint32_t)buf[3 * i + 1], (uint32_t)buf[3 * i + 2]};
    }
    if (n > cap) return fail(ctx, TG_ERR_SHAPE, "tokens holds " + std::to_string(cap) + " entries and the decode emitted " + std::to_string(n));
    return TG_OK;
}

}  // namespace

int tg_tdt_create(tg_ctx *ctx, const tg_tdt_desc *desc, tg_tdt **out) {
    if (!ctx || !desc || !out) return fail(ctx, TG_ERR_NULL, "null argument");
    *out = nullptr;
    const size_t h = desc->hidden, layers = desc->layers, ndur = desc->n_durations, vocab = desc->vocab;
    if (layers < 1 || layers > (size_t)tg::TDT_MAX_LAYERS) return fail(ctx, TG_ERR_ARG, "layers must be 1 to 4");
    if (h == 0 || h % 4) return fail(ctx, TG_ERR_ARG, "hidden must be a positive multiple of 4");
    if (2 * h > 1984) return fail(ctx, TG_ERR_UNSUPPORTED, "hidden beyond 992 (the LSTM rows exceed the GEMV's LDS)");
    if (vocab == 0 || vocab > (size_t)INT32_MAX / 2) return fail(ctx, TG_ERR_ARG, "vocab must be positive");
    if (ndur == 0 || ndur > 64 || !desc->durations) return fail(ctx, TG_ERR_ARG, "durations must hold 1 to 64 values");
    for (size_t i = 0; i < ndur; i++)
        if (desc->durations[i] < 0) return fail(ctx, TG_ERR_ARG, "durations must be >= 0");
    if (desc->max_symbols > (size_t)INT32_MAX) return fail(ctx, TG_ERR_ARG, "max_symbols out of range");
    int rc = tdt_matrix(ctx, desc->joint, vocab + ndur, h, "joint");
    if (rc) return rc;
    for (size_t l = 0; l < layers; l++) {
        rc = tdt_matrix(ctx, desc->lstm[l], 4 * h, 2 * h, "lstm");
        if (rc) return rc;
        if (!desc->lstm_bias[l]) return fail(ctx, TG_ERR_NULL, "an LSTM bias is null");
    }
    rc = tdt_matrix(ctx, desc->proj, h, h, "proj");
    if (rc) return rc;
    if (!desc->joint_bias || !desc->embedding || !desc->proj_bias) return fail(ctx, TG_ERR_NULL, "null bias or embedding");
    if (desc->joint_bias_len < vocab + ndur || desc->proj_bias_len < h || desc->embedding_len < vocab * h)
        return fail(ctx, TG_ERR_SHAPE, "a bias or the embedding is too short");
    for (size_t l = 0; l < layers; l++)
        if (desc->lstm_bias_len[l] < 4 * h) return fail(ctx, TG_ERR_SHAPE, "an LSTM bias is too short");
    if (!aligned16(desc->embedding)) return fail(ctx, TG_ERR_ALIGN, "the embedding must be 16-byte aligned");

    std::lock_guard<std::mutex> g(ctx->mu);
    TG_HIP(ctx, hipSetDevice(ctx->device));
    tg_tdt *t = new tg_tdt();
    t->device = ctx->device;
    tg::TdtNet &net = t->net;
    net.h = h;
    net.vocab = vocab;
    net.ndur = ndur;
    net.layers = layers;
    net.blank = vocab - 1;
    net.max_symbols = desc->max_symbols;
    net.joint = &desc->joint->d;
    net.proj = &desc->proj->d;
    net.joint_b = desc->joint_bias;
    net.proj_b = desc->proj_bias;
    net.emb = desc->embedding;
    bool ok = hipMalloc(&t->ctl, sizeof(tg::TdtCtl)) == hipSuccess &&
              hipHostMalloc(&t->ctl_host, sizeof(tg::TdtCtl), hipHostMallocDefault) == hipSuccess &&
              hipMalloc(&t->durations, ndur * sizeof(int32_t)) == hipSuccess &&
              hipMalloc(&t->extras, tg::tdt_extras_bytes()) == hipSuccess &&
              hipMalloc(&t->scratch, (size_t)tg::TDT_ROWS * layers * 2 * h * sizeof(float)) == hipSuccess &&
              hipMalloc(&t->partials, tg::tdt_partials_bytes()) == hipSuccess;
    for (size_t l = 0; ok && l < layers; l++) {
        const tg::DeviceWeights &src = desc->lstm[l]->d;
        tg::DeviceWeights &dst = t->lstm[l];
        dst = src;
        dst.values = nullptr;
        dst.scales = nullptr;
        ok = hipMalloc(&dst.values, src.values_bytes) == hipSuccess &&
             hipMalloc(&dst.scales, src.n_scales * sizeof(float)) == hipSuccess &&
             hipMalloc(&t->lstm_b[l], 4 * h * sizeof(float)) == hipSuccess;
    }
    if (!ok) {
        tdt_release(t);
        return fail(ctx, TG_ERR_NOMEM, "device allocation failed");
    }
    for (size_t l = 0; l < layers; l++) {
        net.lstm[l] = &t->lstm[l];
        net.lstm_b[l] = t->lstm_b[l];
        const hipError_t e = tg::launch_tdt_interleave(desc->lstm[l]->d, desc->lstm_bias[l], t->lstm[l],
                                                       t->lstm_b[l], h, ctx->stream);
        if (e != hipSuccess) {
            tdt_release(t);
            return hip_fail(ctx, e, "tg_tdt_create");
        }
    }
    net.durations = t->durations;
    if (tg::tdt_resident_plan(net, t->plan)) {
        if (hipMalloc(&t->words, tg::tdt_resident_words(net) * sizeof(uint64_t)) != hipSuccess) {
            tdt_release(t);
            return fail(ctx, TG_ERR_NOMEM, "device allocation failed");
        }
        int khz = 0;
        if (hipDeviceGetAttribute(&khz, hipDeviceAttributeWallClockRate, ctx->device) != hipSuccess || khz <= 0)
            khz = 100000;
        t->clock_khz = (uint64_t)khz;
        t->wait_ticks = (uint64_t)khz * 1000;  // one second
        t->launch_steps = TDT_RESIDENT_STEPS;
        t->can_resident = t->use_resident = true;
        (void)tg::tdt_multi_plan(net, t->plan);
    }
    (void)hipGetLastError();  // a refused LDS attribute or occupancy query leaves the step kernels
    std::memset(t->ctl_host, 0, sizeof(tg::TdtCtl));
    hipError_t e = hipMemcpyAsync(t->ctl, t->ctl_host, sizeof(tg::TdtCtl), hipMemcpyHostToDevice, ctx->stream);
    if (e == hipSuccess)
        e = hipMemcpyAsync(t->durations, desc->durations, ndur * sizeof(int32_t), hipMemcpyHostToDevice, ctx->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(ctx->stream);
    if (e != hipSuccess) {
        tdt_release(t);
        return hip_fail(ctx, e, "tg_tdt_create");
    }
    *out = t;
    return TG_OK;
}

void tg_tdt_destroy(tg_tdt *tdt) {
    if (!tdt) return;
    (void)hipSetDevice(tdt->device);
    (void)hipDeviceSynchronize();
    tdt_release(tdt);
}

size_t tg_tdt_max_rows(const tg_tdt *tdt) { return tdt ? tg::tdt_max_rows(*tdt->net.lstm[0]) : 0; }

int tg_tdt_predict_device(tg_ctx *ctx, tg_tdt *tdt, const int32_t *tokens, size_t rows, float *states,
                          size_t states_len, float *preds, size_t preds_len) {
    if (!ctx || !tdt) return fail(ctx, TG_ERR_NULL, "null context or network");
    if (rows == 0) return TG_OK;
    if (!tokens || !states || !preds) return fail(ctx, TG_ERR_NULL, "null tokens, states or preds");
    if (tdt->device != ctx->device) return fail(ctx, TG_ERR_ARG, "the network lives on another device");
    if (rows > tg::tdt_max_rows(*tdt->net.lstm[0]))
        return fail(ctx, TG_ERR_UNSUPPORTED, "more rows than tg_tdt_max_rows");
    if (states_len < rows * tdt->net.layers * 2 * tdt->net.h) return fail(ctx, TG_ERR_SHAPE, "states is too short");
    if (preds_len < rows * tdt->net.h) return fail(ctx, TG_ERR_SHAPE, "preds is too short");
    if (!aligned16(states) || !aligned16(preds)) return fail(ctx, TG_ERR_ALIGN, "states and preds must be 16-byte aligned");
    tg::TdtTokens toks{};
    for (size_t r = 0; r < rows; r++) {
        if (tokens[r] < 0 || (size_t)tokens[r] >= tdt->net.vocab) return fail(ctx, TG_ERR_ARG, "a token is out of range");
        toks.tok[r] = tokens[r];
    }
    std::lock_guard<std::mutex> g(ctx->mu);
    TG_HIP(ctx, hipSetDevice(ctx->device));
    // The new states go to the scratch rows (other workgroups still read the old ones), then back.
    TG_HIP(ctx, tg::launch_tdt_predict(tdt->ctl, toks, rows, tdt->net, states, tdt->scratch, preds, ctx->stream));
    const size_t width = tdt->net.layers * 2 * tdt->net.h;
    TG_HIP(ctx, hipMemcpyAsync(states, tdt->scratch, rows * width * sizeof(float), hipMemcpyDeviceToDevice,
                               ctx->stream));
    return TG_OK;
}

int tg_tdt_decode_device(tg_ctx *ctx, tg_tdt *tdt, const float *enc_proj, size_t enc_len, size_t lde, size_t frames,
                         float *state, size_t state_len, float *pred, size_t pred_len, size_t *frame,
                         size_t *on_frame, tg_token *tokens, size_t cap, size_t *count) {
    if (!ctx || !tdt) return fail(ctx, TG_ERR_NULL, "null context or network");
    if (!state || !pred || !frame || !on_frame || !count || (cap && !tokens))
        return fail(ctx, TG_ERR_NULL, "null argument");
    *count = 0;
    if (tdt->device != ctx->device) return fail(ctx, TG_ERR_ARG, "the network lives on another device");
    const tg::TdtNet &net = tdt->net;
    if (frames >= ((size_t)1 << 24)) return fail(ctx, TG_ERR_UNSUPPORTED, "more than 2^24 frames");
    if (*frame >= frames) return TG_OK;  // the reference's loop does not start
    if (!enc_proj) return fail(ctx, TG_ERR_NULL, "enc_proj is null");
    if (lde < net.h || lde % 4) return fail(ctx, TG_ERR_SHAPE, "lde must be >= hidden and a multiple of 4");
    if (enc_len < span(frames, lde, net.h)) return fail(ctx, TG_ERR_SHAPE, "enc_proj is too short");
    if (state_len < net.layers * 2 * net.h) return fail(ctx, TG_ERR_SHAPE, "state is too short");
    if (pred_len < net.h) return fail(ctx, TG_ERR_SHAPE, "pred is too short");
    if (!aligned16(enc_proj) || !aligned16(state) || !aligned16(pred))
        return fail(ctx, TG_ERR_ALIGN, "enc_proj, state and pred must be 16-byte aligned");
    if (*on_frame > (size_t)INT32_MAX) return fail(ctx, TG_ERR_ARG, "on_frame out of range");
    // At most max(max_symbols, 1) tokens per frame: a token either moves on by its duration or
    // counts towards max_symbols on its frame.
    const size_t per_frame = net.max_symbols > 1 ? net.max_symbols : 1;
    const size_t most = (frames - *frame) * per_frame;
    if (most >= ((size_t)1 << 30)) return fail(ctx, TG_ERR_UNSUPPORTED, "too many possible tokens");

    std::lock_guard<std::mutex> g(ctx->mu);
    TG_HIP(ctx, hipSetDevice(ctx->device));
    if (most > tdt->tokens_cap) {
        TG_HIP(ctx, hipStreamSynchronize(ctx->stream));
        if (tdt->tokens) TG_HIP(ctx, hipFree(tdt->tokens));
        tdt->tokens = nullptr;
        tdt->tokens_cap = 0;
        if (hipMalloc(&tdt->tokens, most * 3 * sizeof(int32_t)) != hipSuccess)
            return fail(ctx, TG_ERR_NOMEM, "device allocation failed");
        tdt->tokens_cap = most;
    }
    tg::TdtCtl *hc = tdt->ctl_host;
    TG_HIP(ctx, hipStreamSynchronize(ctx->stream));  // the pinned copy is free to rewrite
    std::memset(hc, 0, sizeof(*hc));
    hc->t = (int32_t)*frame;
    hc->on_frame = (int32_t)*on_frame;
    hc->rows = tg::TDT_ROWS;
    TG_HIP(ctx, hipMemcpyAsync(tdt->ctl, hc, sizeof(*hc), hipMemcpyHostToDevice, ctx->stream));
    const size_t limit = (frames - *frame) * (per_frame + 1) + 1;
    // The resident decode when the network takes it and no other resident decode holds this device;
    // the lock is held until its last launch has ended (each launch is followed by a synchronize).
    std::unique_lock<std::mutex> rlock;
    if (tdt->use_resident && ctx->device >= 0 && ctx->device < MAX_DEVICES)
        rlock = std::unique_lock<std::mutex>(resident_mu[ctx->device], std::try_to_lock);
    tdt->last_resident = rlock.owns_lock() ? 1 : 0;
    if (rlock.owns_lock()) {
        // state and pred as the caller passed them, in the scratch rows (layers x 2h, then h), put
        // back if a launch fails: the launches write their state back even when a wait gave up.
        const size_t sw = net.layers * 2 * net.h;
        TG_HIP(ctx, hipMemcpyAsync(tdt->scratch, state, sw * sizeof(float), hipMemcpyDeviceToDevice, ctx->stream));
        TG_HIP(ctx, hipMemcpyAsync(tdt->scratch + sw, pred, net.h * sizeof(float), hipMemcpyDeviceToDevice,
                                   ctx->stream));
        auto restore = [&]() {
            (void)hipMemcpyAsync(state, tdt->scratch, sw * sizeof(float), hipMemcpyDeviceToDevice, ctx->stream);
            (void)hipMemcpyAsync(pred, tdt->scratch + sw, net.h * sizeof(float), hipMemcpyDeviceToDevice, ctx->stream);
            (void)hipStreamSynchronize(ctx->stream);
        };
        TG_HIP(ctx, tg::launch_tdt_resident_init(net, tdt->words, state, pred, ctx->stream));
        size_t steps = 0;
        while (true) {
            const hipError_t e = tg::launch_tdt_resident(tdt->ctl, net, tdt->plan, tdt->words, enc_proj, lde,
                                                         (int)frames, state, pred, tdt->tokens, (int)most,
                                                         tdt->launch_steps, tdt->wait_ticks, ctx->stream);
            if (e != hipSuccess) {
                restore();
                return hip_fail(ctx, e, "the resident decode's launch");
            }
            TG_HIP(ctx, hipMemcpyAsync(hc, tdt->ctl, sizeof(*hc), hipMemcpyDeviceToHost, ctx->stream));
            TG_HIP(ctx, hipStreamSynchronize(ctx->stream));
            if (hc->err) {
                restore();
                return fail(ctx, TG_ERR_HIP,
                            "the resident decode: a workgroup's wait passed its deadline (state and pred restored)");
            }
            if (hc->done) break;
            steps += (size_t)tdt->launch_steps;
            if (steps > limit) {
                restore();
                return fail(ctx, TG_ERR_HIP, "the decode did not finish within its step bound");
            }
        }
        tdt->last_steps = hc->step;
        return tdt_results(ctx, tdt, hc, frame, on_frame, tokens, cap, count);
    }
    // Steps run as a captured graph of TDT_GRAPH_STEPS steps, replayed in growing batches between
    // looks at the control block; a step after the end returns at once. Every step emits a token
    // or moves at least one frame, so (frames - frame) (per_frame + 1) steps always suffice.
    const uintptr_t key[7] = {reinterpret_cast<uintptr_t>(enc_proj), lde, frames, reinterpret_cast<uintptr_t>(state),
                              reinterpret_cast<uintptr_t>(pred), reinterpret_cast<uintptr_t>(tdt->tokens), most};
    if (!tdt->exec || std::memcmp(key, tdt->key, sizeof(key)) != 0) {
        tdt_drop_graph(tdt);
        TG_HIP(ctx, hipStreamBeginCapture(ctx->stream, hipStreamCaptureModeThreadLocal));
        hipError_t e = hipSuccess;
        for (int i = 0; i < TDT_GRAPH_STEPS && e == hipSuccess; i++)
            e = tg::launch_tdt_step(tdt->ctl, net, enc_proj, lde, (int)frames, state, tdt->scratch, pred,
                                    tdt->partials, tdt->extras, tdt->tokens, (int)most, ctx->stream);
        hipGraph_t g = nullptr;
        const hipError_t e2 = hipStreamEndCapture(ctx->stream, &g);
        if (e != hipSuccess || e2 != hipSuccess) {
            if (g) (void)hipGraphDestroy(g);
            return hip_fail(ctx, e != hipSuccess ? e : e2, "capturing the decode step");
        }
        tdt->graph = g;
        TG_HIP(ctx, hipGraphInstantiate(&tdt->exec, g, nullptr, nullptr, 0));
        std::memcpy(tdt->key, key, sizeof(key));
    }
    size_t steps = 0, graphs = 1;
    while (true) {
        for (size_t i = 0; i < graphs; i++) TG_HIP(ctx, hipGraphLaunch(tdt->exec, ctx->stream));
        steps += graphs * TDT_GRAPH_STEPS;
        TG_HIP(ctx, hipMemcpyAsync(hc, tdt->ctl, sizeof(*hc), hipMemcpyDeviceToHost, ctx->stream));
        TG_HIP(ctx, hipStreamSynchronize(ctx->stream));
        if (hc->done) break;
        if (steps > limit) return fail(ctx, TG_ERR_HIP, "the decode did not finish within its step bound");
        graphs = graphs < 8 ? graphs * 2 : 8;
    }
    if (hc->cur)  // the last prediction left the state in the scratch buffer
        TG_HIP(ctx, hipMemcpyAsync(state, tdt->scratch, net.layers * 2 * net.h * sizeof(float),
                                   hipMemcpyDeviceToDevice, ctx->stream));
    return tdt_results(ctx, tdt, hc, frame, on_frame, tokens, cap, count);
}

int tg_tdt_decode_streams_device(tg_ctx *ctx, tg_tdt *tdt, tg_tdt_stream *streams, size_t m) {
    if (!ctx || !tdt) return fail(ctx, TG_ERR_NULL, "null context or network");
    if (m == 0) return TG_OK;
    if (!streams) return fail(ctx, TG_ERR_NULL, "null streams");
    if (tdt->device != ctx->device) return fail(ctx, TG_ERR_ARG, "the network lives on another device");
    if (m > tg::TDT_MAX_STREAMS) {  // in groups of TDT_MAX_STREAMS
        for (size_t q0 = 0; q0 < m; q0 += tg::TDT_MAX_STREAMS) {
            const size_t n = m - q0 < tg::TDT_MAX_STREAMS ? m - q0 : tg::TDT_MAX_STREAMS;
            const int rc = tg_tdt_decode_streams_device(ctx, tdt, streams + q0, n);
            if (rc) return rc;
        }
        return TG_OK;
    }
    const tg::TdtNet &net = tdt->net;
    const size_t per_frame = net.max_symbols > 1 ? net.max_symbols : 1;
    size_t most[tg::TDT_MAX_STREAMS] = {}, total = 0, bound = 0;
    bool any = false;
    for (size_t q = 0; q < m; q++) {
        tg_tdt_stream &st = streams[q];
        st.count = 0;
        if (!st.state || !st.pred || (st.cap && !st.tokens)) return fail(ctx, TG_ERR_NULL, "null argument");
        if (st.frames >= ((size_t)1 << 24)) return fail(ctx, TG_ERR_UNSUPPORTED, "more than 2^24 frames");
        if (st.frame >= st.frames) continue;  // the reference's loop does not start
        if (!st.enc_proj) return fail(ctx, TG_ERR_NULL, "enc_proj is null");
        if (st.lde < net.h || st.lde % 4) return fail(ctx, TG_ERR_SHAPE, "lde must be >= hidden and a multiple of 4");
        if (st.enc_len < span(st.frames, st.lde, net.h)) return fail(ctx, TG_ERR_SHAPE, "enc_proj is too short");
        if (st.state_len < net.layers * 2 * net.h) return fail(ctx, TG_ERR_SHAPE, "state is too short");
        if (st.pred_len < net.h) return fail(ctx, TG_ERR_SHAPE, "pred is too short");
        if (!aligned16(st.enc_proj) || !aligned16(st.state) || !aligned16(st.pred))
            return fail(ctx, TG_ERR_ALIGN, "enc_proj, state and pred must be 16-byte aligned");
        if (st.on_frame > (size_t)INT32_MAX) return fail(ctx, TG_ERR_ARG, "on_frame out of range");
        most[q] = (st.frames - st.frame) * per_frame;
        if (most[q] >= ((size_t)1 << 30)) return fail(ctx, TG_ERR_UNSUPPORTED, "too many possible tokens");
        total += most[q];
        bound = std::max(bound, (st.frames - st.frame) * (per_frame + 1) + 1);
        any = true;
    }
    if (!any) return TG_OK;
    // The streams' states must not share memory: each stream's launch writes its own.
    for (size_t q = 0; q < m; q++)
        for (size_t r = q + 1; r < m; r++)
            if (streams[q].frame < streams[q].frames && streams[r].frame < streams[r].frames &&
                (streams[q].state == streams[r].state || streams[q].pred == streams[r].pred))
                return fail(ctx, TG_ERR_ARG, "two streams share a state or prediction");
    {
        std::unique_lock<std::mutex> g(ctx->mu);
        std::unique_lock<std::mutex> rlock;
        if (tdt->use_resident && tdt->plan.multi && m > 1 && ctx->device >= 0 && ctx->device < MAX_DEVICES)
            rlock = std::unique_lock<std::mutex>(resident_mu[ctx->device], std::try_to_lock);
        if (rlock.owns_lock()) {
            TG_HIP(ctx, hipSetDevice(ctx->device));
            const size_t sw = net.layers * 2 * net.h, M = tg::TDT_MAX_STREAMS;
            if (!tdt->mctl) {
                if (hipMalloc(&tdt->mctl, M * sizeof(tg::TdtCtl)) != hipSuccess ||
                    hipHostMalloc(&tdt->mctl_host, M * sizeof(tg::TdtCtl), hipHostMallocDefault) != hipSuccess ||
                    hipMalloc(&tdt->mwords, tg::tdt_multi_words(net) * sizeof(uint64_t)) != hipSuccess ||
                    hipMalloc(&tdt->mscratch, M * (sw + net.h) * sizeof(float)) != hipSuccess)
                    return fail(ctx, TG_ERR_NOMEM, "device allocation failed");
            }
            if (total > tdt->tokens_cap) {
                TG_HIP(ctx, hipStreamSynchronize(ctx->stream));
                if (tdt->tokens) TG_HIP(ctx, hipFree(tdt->tokens));
                tdt->tokens = nullptr;
                tdt->tokens_cap = 0;
                if (hipMalloc(&tdt->tokens, total * 3 * sizeof(int32_t)) != hipSuccess)
                    return fail(ctx, TG_ERR_NOMEM, "device allocation failed");
                tdt->tokens_cap = total;
            }
            // Streams that start past their frames take no part: the launch sees the others only.
            size_t idx[tg::TDT_MAX_STREAMS], k = 0, off = 0;
            tg::TdtStream ts[tg::TDT_MAX_STREAMS];
            size_t toff[tg::TDT_MAX_STREAMS];
            for (size_t q = 0; q < m; q++) {
                if (streams[q].frame >= streams[q].frames) continue;
                idx[k] = q;
                toff[k] = off;
                ts[k] = tg::TdtStream{streams[q].enc_proj, streams[q].lde, (int)streams[q].frames, streams[q].state,
                                      streams[q].pred, tdt->tokens + off * 3, (int)most[q]};
                off += most[q];
                k++;
            }
            tg::TdtCtl *hc = tdt->mctl_host;
            TG_HIP(ctx, hipStreamSynchronize(ctx->stream));
            std::memset(hc, 0, M * sizeof(tg::TdtCtl));
            uint32_t preds[tg::TDT_MAX_STREAMS] = {};
            for (size_t j = 0; j < k; j++) {
                hc[j].t = (int32_t)streams[idx[j]].frame;
                hc[j].on_frame = (int32_t)streams[idx[j]].on_frame;
                hc[j].rows = tg::TDT_ROWS;
            }
            TG_HIP(ctx, hipMemcpyAsync(tdt->mctl, hc, M * sizeof(tg::TdtCtl), hipMemcpyHostToDevice, ctx->stream));
            for (size_t j = 0; j < k; j++) {
                float *sc = tdt->mscratch + j * (sw + net.h);
                TG_HIP(ctx, hipMemcpyAsync(sc, ts[j].state, sw * sizeof(float), hipMemcpyDeviceToDevice, ctx->stream));
                TG_HIP(ctx, hipMemcpyAsync(sc + sw, ts[j].pred, net.h * sizeof(float), hipMemcpyDeviceToDevice,
                                           ctx->stream));
            }
            auto restore = [&]() {
                for (size_t j = 0; j < k; j++) {
                    const float *sc = tdt->mscratch + j * (sw + net.h);
                    (void)hipMemcpyAsync(ts[j].state, sc, sw * sizeof(float), hipMemcpyDeviceToDevice, ctx->stream);
                    (void)hipMemcpyAsync(ts[j].pred, sc + sw, net.h * sizeof(float), hipMemcpyDeviceToDevice,
                                         ctx->stream);
                }
                (void)hipStreamSynchronize(ctx->stream);
            };
            TG_HIP(ctx, tg::launch_tdt_multi_init(net, tdt->mwords, k, ts, preds, ctx->stream));
            tdt->last_resident = 2;
            size_t steps = 0;
            while (true) {
                const hipError_t e = tg::launch_tdt_multi(tdt->mctl, net, tdt->plan, tdt->mwords, k, ts,
                                                          tdt->launch_steps, tdt->wait_ticks, ctx->stream);
                if (e != hipSuccess) {
                    restore();
                    return hip_fail(ctx, e, "the multi-stream decode's launch");
                }
                TG_HIP(ctx, hipMemcpyAsync(hc, tdt->mctl, M * sizeof(tg::TdtCtl), hipMemcpyDeviceToHost, ctx->stream));
                TG_HIP(ctx, hipStreamSynchronize(ctx->stream));
                if (hc[0].err) {
                    restore();
                    return fail(ctx, TG_ERR_HIP,
                                "the multi-stream decode: a workgroup's wait passed its deadline (states and "
                                "predictions restored)");
                }
                bool done = true;
                for (size_t j = 0; j < k; j++) done = done && hc[j].done;
                if (done) break;
                steps += (size_t)tdt->launch_steps;
                if (steps > bound) {
                    restore();
                    return fail(ctx, TG_ERR_HIP, "the decode did not finish within its step bound");
                }
            }
            tdt->last_steps = hc[0].step;
            int rc = TG_OK;
            for (size_t j = 0; j < k; j++) {
                tg_tdt_stream &st = streams[idx[j]];
                const size_t n = (size_t)hc[j].ntok, copy = n < st.cap ? n : st.cap;
                st.frame = (size_t)hc[j].t;
                st.on_frame = (size_t)hc[j].on_frame;
                st.count = n;
                if (copy) {
                    std::vector<int32_t> buf(copy * 3);
                    TG_HIP(ctx, hipMemcpy(buf.data(), tdt->tokens + toff[j] * 3, copy * 3 * sizeof(int32_t),
                                          hipMemcpyDeviceToHost));
                    for (size_t i = 0; i < copy; i++)
                        st.tokens[i] = tg_token{(uint32_t)buf[3 * i], (uint32_t)buf[3 * i + 1], (uint32_t)buf[3 * i + 2]};
                }
                if (n > st.cap && rc == TG_OK)
                    rc = fail(ctx, TG_ERR_SHAPE, "tokens holds " + std::to_string(st.cap) +
                                                     " entries and the decode emitted " + std::to_string(n));
            }
            if (rc == TG_OK) clear_error(ctx);
            return rc;
        }
    }
    // One stream at a time (resident where it can, else by the step kernels): the same results.
    for (size_t q = 0; q < m; q++) {
        tg_tdt_stream &st = streams[q];
        const int rc = tg_tdt_decode_device(ctx, tdt, st.enc_proj, st.enc_len, st.lde, st.frames, st.state,
                                            st.state_len, st.pred, st.pred_len, &st.frame, &st.on_frame, st.tokens,
                                            st.cap, &st.count);
        if (rc) return rc;
    }
    return TG_OK;
}

int tg_tdt_set_resident(tg_ctx *ctx, tg_tdt *tdt, int on) {
    if (!ctx || !tdt) return fail(ctx, TG_ERR_NULL, "null context or network");
    if (on && !tdt->can_resident)
        return fail(ctx, TG_ERR_UNSUPPORTED,
                    "the network does not run resident (int8 matrices, vocab < 65535, the panels in LDS, cooperative launch)");
    std::lock_guard<std::mutex> g(ctx->mu);
    tdt->use_resident = on != 0;
    return TG_OK;
}

int tg_tdt_is_resident(const tg_tdt *tdt) { return tdt && tdt->use_resident ? 1 : 0; }

int tg_tdt_last_resident(const tg_tdt *tdt) { return tdt ? tdt->last_resident : -1; }

size_t tg_tdt_last_steps(const tg_tdt *tdt) { return tdt ? tdt->last_steps : 0; }

int tg_tdt_set_resident_limits(tg_ctx *ctx, tg_tdt *tdt, uint32_t steps_per_launch, uint64_t wait_us) {
    if (!ctx || !tdt) return fail(ctx, TG_ERR_NULL, "null context or network");
    if (steps_per_launch > (uint32_t)TDT_RESIDENT_STEPS)
        return fail(ctx, TG_ERR_ARG, "at most 16384 steps per resident launch");
    if (wait_us > (uint64_t)60 * 1000 * 1000) return fail(ctx, TG_ERR_ARG, "a wait of at most 60 s");
    std::lock_guard<std::mutex> g(ctx->mu);
    tdt->launch_steps = steps_per_launch ? (int)steps_per_launch : TDT_RESIDENT_STEPS;
    const uint64_t ticks = wait_us ? wait_us * tdt->clock_khz / 1000 : tdt->clock_khz * 1000;
    tdt->wait_ticks = ticks ? ticks : 1;
    return TG_OK;
}

}  // extern "C"
