/*
 * telmo_hip.h - C ABI of the MI355X (gfx950) int8-weight matrix product.
 *
 * A drop-in for telmo's matrix-product operator surface. Plain pointers and sizes only; every
 * entry point returns a status (TG_OK = 0, negative on error) and never aborts or throws across
 * the boundary. Reference interfaces each entry point replaces (paths in the telmo repository):
 *
 *   Precision                    src/quant.rs:20-83
 *   quant::encode / decode       src/quant.rs:200-303
 *   PackedWeights::from_parts    src/kernels/mod.rs:214-237   -> tg_weights_upload
 *   PackedWeights::bytes         src/kernels/mod.rs:301-303   -> tg_weights_bytes
 *   Act, Epilogue                src/kernels/mod.rs:366-398   -> tg_epilogue
 *   Kernels::matmul              src/kernels/mod.rs:657-688   -> tg_matmul, tg_matmul_device
 *   Kernels::linear              src/kernels/mod.rs:691-701   -> tg_linear, tg_linear_device
 *   Kernels::glu (row kernel)    src/kernels/mod.rs:463-464   -> tg_glu_device
 *   Kernels::layer_norm          src/kernels/mod.rs:458       -> tg_layer_norm_device
 *   Kernels::dwconv1d_frame + silu  src/kernels/mod.rs:464-475  -> tg_dwconv1d_device
 *   BView::row_major + matmul    src/kernels/mod.rs:320-339, 657-688 -> tg_matmul_rowmajor_device
 *   Parakeet::predict_rows       src/parakeet.rs:1524-1577    -> tg_tdt_predict_device
 *   Parakeet::decode_inner       src/parakeet.rs:1412-1513    -> tg_tdt_decode_device
 *   Pack::open / from_bytes      src/pack.rs:79-96            -> tg_pack_open, tg_pack_from_bytes
 *   Pack::parse (the checks)     src/pack.rs:98-259           -> tg_pack_open, tg_pack_last_error
 *   Pack::model / meta / entries src/pack.rs:248-265          -> tg_pack_model, tg_pack_meta, tg_pack_entry_at
 *   Pack::matrix                 src/pack.rs:279-305          -> tg_pack_find + tg_pack_upload_matrix
 *
 * Error behaviour follows the reference's asserts (src/kernels/mod.rs:669-677): m == 0 or n == 0
 * is a no-op that succeeds before any other check; then lda >= k, ldc >= n, the lengths of a and
 * c, and the bias length (>= n) are checked and give TG_ERR_SHAPE; k == 0 stores the epilogue of
 * a zero sum. The reference panics where this returns an error; a Rust shim maps the codes back.
 */
#ifndef TELMO_HIP_H
#define TELMO_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct tg_ctx tg_ctx;
typedef struct tg_weights tg_weights;

/* Weight precisions, in the order of src/quant.rs:22-30. */
enum { TG_F32 = 0, TG_F16 = 1, TG_BF16 = 2, TG_INT8 = 3, TG_Q8_0 = 4 };

/* Epilogue activations, src/kernels/mod.rs:368-372. */
enum { TG_ACT_NONE = 0, TG_ACT_RELU = 1, TG_ACT_SILU = 2 };

/* Numerics of a context.
 * TG_MODE_FAST: int8 and Q8_0 weights run the two-digit int8 path: the MFMA GEMM, or for m <= 16
 *   decode rows the MFMA GEMV (for int8, the dot4 GEMV for m <= 8 rows it cannot take).
 *   Activations are split per row into two int8 digits of a 15-bit fixed-point value; sums are
 *   exact in i32 (per 32-input block for Q8_0, whose block sums are scaled and added in f32 in
 *   block order); results are bit-identical for any m, kernel, tiling or split, and within about
 *   1e-4 row-normwise of the reference's fused f32 sums (gate 1e-3). Other precisions run the
 *   exact kernel.
 * TG_MODE_EXACT: one lane per output sums fmaf(a, widen(w), acc) in input order, bit-identical
 *   to the reference's AVX2 / AVX-512 / NEON kernels, epilogue included. Slow; for validation. */
enum { TG_MODE_FAST = 0, TG_MODE_EXACT = 1 };

/* Status codes. */
enum {
    TG_OK = 0,
    TG_ERR_NULL = -1,        /* a required pointer is null */
    TG_ERR_SHAPE = -2,       /* a precondition of Kernels::matmul fails */
    TG_ERR_ALIGN = -3,       /* a buffer is not aligned as required */
    TG_ERR_HIP = -4,         /* a HIP runtime call failed (see tg_last_error) */
    TG_ERR_UNSUPPORTED = -5, /* precision, mode or size this library does not run */
    TG_ERR_NOMEM = -6,       /* device allocation failed */
    TG_ERR_ARG = -7          /* an argument is out of its range (precision, act, sizes of the weights) */
};

/* Epilogue: c = (accumulate ? c : 0) + scale * act(sum + bias). bias may be null; when set it
 * holds bias_len >= n values (host memory for host entry points, device memory for _device ones). */
typedef struct tg_epilogue {
    const float *bias;
    size_t bias_len;
    uint32_t act;
    float scale;
    int32_t accumulate;
} tg_epilogue;

/* ---- contexts ---------------------------------------------------------------------------- */

/* A context on HIP device `device`. `stream` is a hipStream_t to run on, or null for a stream of
 * the context's own. Calls on one context are serialised; contexts are independent. */
int tg_ctx_create(int device, void *stream, tg_ctx **out);
void tg_ctx_destroy(tg_ctx *ctx);
int tg_ctx_set_mode(tg_ctx *ctx, uint32_t mode);
uint32_t tg_ctx_mode(const tg_ctx *ctx);
/* The accuracy guard of the product entry points (tg_matmul, tg_linear and their _device and
 * _noalloc forms) in fast mode, on by default; no counterpart in the reference, whose f32 sums have
 * no data-dependent error. The fast path keeps 15 bits of each row relative to its largest value.
 * When a product takes the GEMM (not the decode GEMV of a few aligned rows), its quantiser also
 * measures what the two digits drop: with x = a 2^e the scaled inputs, v = rint(x) and d =
 * rint(256 (x - v)), a row whose 256 sum d^2 exceeds sum v^2 (a relative rounding of the row above
 * 2^-12, where the fast path's row-normwise error could approach 1e-3: an outlier far above the
 * rest of a long row) is flagged, and the exact kernel rewrites that row's outputs with the
 * reference's fused sums (its bits), the epilogue accumulating onto the row as it was before the
 * call. Unflagged rows keep the fast path's bits. Off: every row takes the fast path. */
int tg_ctx_set_guard(tg_ctx *ctx, int on);
int tg_ctx_guard(const tg_ctx *ctx);
/* The message of the last failed call on this context ("" if none), copied into storage of the
 * calling thread: valid until that thread's next tg_last_error call. */
const char *tg_last_error(const tg_ctx *ctx);
/* Waits for all work queued on the context's stream; TG_ERR_HIP if the device reports an error. */
int tg_synchronize(tg_ctx *ctx);

/* ---- weights ------------------------------------------------------------------------------ */

/* Uploads a matrix in telmo's panel layout (n outputs, k inputs; values_len bytes as
 * tg_panel_bytes gives, scales as tg_scale_count gives). Host pointers. The device copy is the
 * library's own and lives until tg_weights_free; int8 and Q8_0 values are re-laid out on the
 * device for the MFMA and dot4 kernels. Mirrors PackedWeights::from_parts, whose refusals
 * (wrong lengths, Q8_0 with k not a multiple of 32) give TG_ERR_ARG. n and k must be below 2^31
 * with at most 2^48 weights (TG_ERR_UNSUPPORTED), checked before the lengths so that no byte
 * count wraps. */
int tg_weights_upload(tg_ctx *ctx, const uint8_t *values, size_t values_len, const float *scales,
                      size_t n_scales, uint32_t precision, size_t n, size_t k, tg_weights **out);
/* The same with values and scales already in device memory (read during the call only). */
int tg_weights_upload_device(tg_ctx *ctx, const uint8_t *values, size_t values_len, const float *scales,
                             size_t n_scales, uint32_t precision, size_t n, size_t k, tg_weights **out);
void tg_weights_free(tg_weights *w);
/* Bytes of weight data in the panel layout, scales included (PackedWeights::bytes). */
size_t tg_weights_bytes(const tg_weights *w);
size_t tg_weights_n(const tg_weights *w);
size_t tg_weights_k(const tg_weights *w);
uint32_t tg_weights_precision(const tg_weights *w);

/* ---- the matrix product ------------------------------------------------------------------- */

/* c[m, n] = epilogue(a[m, k] * w^T) with a rows lda apart and c rows ldc apart. Host pointers;
 * copies a (and c when accumulating) to the device, runs, copies c back, and returns when done.
 * a_len and c_len are the lengths of the caller's slices, as the reference checks them; a span
 * (m - 1) * ld + k that does not fit in size_t counts as too long for any slice. m must be below
 * 2^31 (TG_ERR_UNSUPPORTED). */
int tg_matmul(tg_ctx *ctx, const float *a, size_t a_len, size_t lda, size_t m, const tg_weights *w, float *c,
              size_t c_len, size_t ldc, const tg_epilogue *epi);
/* tg_matmul with lda = k and ldc = n. */
int tg_linear(tg_ctx *ctx, const float *a, size_t a_len, size_t m, const tg_weights *w, float *c, size_t c_len,
              const tg_epilogue *epi);

/* The same on device pointers, queued on the context's stream and returning at once. Buffers
 * must stay valid until the stream reaches the work (tg_synchronize). a and c must not overlap.
 * Captured graphs: a call that takes the GEMM quantises a into the context's workspace, which a
 * later call needing more of it frees and reallocates. A HIP graph captured around a call keeps the
 * workspace's address, so once any call on that context has grown the workspace the graph must not
 * be replayed (it would write freed memory): capture after the largest call, or capture
 * tg_matmul_device_noalloc or the staged calls below on buffers of the caller's. */
int tg_matmul_device(tg_ctx *ctx, const float *a, size_t a_len, size_t lda, size_t m, const tg_weights *w,
                     float *c, size_t c_len, size_t ldc, const tg_epilogue *epi);
int tg_linear_device(tg_ctx *ctx, const float *a, size_t a_len, size_t m, const tg_weights *w, float *c,
                     size_t c_len, const tg_epilogue *epi);

/* tg_matmul_device without any allocation: no counterpart in the reference; for callers that
 * cannot allocate (code under HIP graph capture, serving loops, harnesses that forbid hipMalloc).
 * The same checks, kernels and bits as tg_matmul_device; the quantised rows of a product that
 * takes the GEMM go to a scratch array of the library's (16 MiB per GPU, held until the process
 * ends) instead of the context's grown workspace, and so do the accuracy guard's flags and, for an
 * accumulating product, its rows' old outputs (m n floats after the quantised rows). Products whose
 * quantised rows exceed it (tg_quant_bytes(m, k) > 16 MiB - 128 KiB, or m > 16384), or with the guard
 * on whose old outputs do not fit beside them, give TG_ERR_UNSUPPORTED. Every call on a
 * GPU shares that GPU's scratch, so calls that overlap on one GPU (other contexts or streams)
 * race: serialise them. Device pointers, queued on the stream. */
int tg_matmul_device_noalloc(tg_ctx *ctx, const float *a, size_t a_len, size_t lda, size_t m, const tg_weights *w,
                             float *c, size_t c_len, size_t ldc, const tg_epilogue *epi);

/* c = epi(a . b) with b a row-major [k, ldb] f32 matrix whose first n columns are used: the
 * reference's BView::row_major right-hand side (src/kernels/mod.rs:320-339, the attention path's
 * f32 activations) through Kernels::matmul (657-688) / matmul_serial (732-765). The sums are the
 * reference's fused ones, fmaf over the inputs in order, whatever the context's mode. As
 * BView::check (341-351) requires, b holds whole 16-column panels: b_len >= (ceil(n / 16) - 1) 16
 * + (k - 1) ldb + 16 floats (TG_ERR_SHAPE otherwise); then matmul's checks. Device pointers. */
int tg_matmul_rowmajor_device(tg_ctx *ctx, const float *a, size_t a_len, size_t lda, size_t m, const float *b,
                              size_t b_len, size_t k, size_t n, size_t ldb, float *c, size_t c_len, size_t ldc,
                              const tg_epilogue *epi);

/* ---- the staged int8 path ------------------------------------------------------------------
 * The fast int8 product in its two stages, for callers that reuse one quantised input across
 * several weights or time the GEMM alone. Rows are quantised into an opaque buffer of
 * tg_quant_bytes(m, k) bytes plus m int32 row exponents (device memory, caller-owned). No
 * counterpart in the reference, whose sums are all f32. */
size_t tg_quant_bytes(size_t m, size_t k);
int tg_quantize_rows_device(tg_ctx *ctx, const float *a, size_t a_len, size_t lda, size_t m, size_t k, void *qa,
                            size_t qa_len, int32_t *exps);
/* c = epilogue(product of the quantised rows and int8 or Q8_0 weights w) on the MFMA GEMM, any
 * m >= 1. TG_ERR_UNSUPPORTED for other weights or k beyond the integer path's limit (65536). */
int tg_matmul_quantized_device(tg_ctx *ctx, const void *qa, size_t qa_len, const int32_t *exps, size_t m,
                               const tg_weights *w, float *c, size_t c_len, size_t ldc, const tg_epilogue *epi);

/* tg_linear_glu_device on quantised rows: out = glu(epi(qa . w)), the GLU in the GEMM's epilogue,
 * for a convolution module whose pointwise_conv1 input comes out of tg_layer_norm_quant_device.
 * int8 weights with n a multiple of 64, or Q8_0 weights with any even n (with n not a multiple of
 * 64 the product goes into a context buffer and then the GLU kernel); either way the bits of the
 * two calls. Fast mode (TG_ERR_UNSUPPORTED otherwise); no accumulation. */
int tg_matmul_quantized_glu_device(tg_ctx *ctx, const void *qa, size_t qa_len, const int32_t *exps, size_t m,
                                   const tg_weights *w, float *out, size_t out_len, size_t ldo,
                                   const tg_epilogue *epi);

/* The product of quantised rows whose outputs go out quantised in turn: epi(qa . w) as
 * tg_matmul_quantized_device computes it, then the two-digit quantisation tg_quantize_rows_device
 * makes of those f32 rows, into qa_out (tg_quant_bytes(m, n) bytes) and exps_out (m), bit-identical
 * to the two calls. For a feed-forward block's first product, whose only reader is the second
 * (src/parakeet.rs:1024-1060: ff_in with SiLU into s.big, then ff_out), which then takes qa_out
 * through tg_matmul_quantized_device. The f32 rows go through a context workspace of about 4 m n
 * bytes, grown on first use. Without activation or scale an int8 product also leaves each row's
 * largest |y| per tile column, so the quantiser streams the rows once without a reduction. With
 * them, or with Q8_0 weights, the product's f32 rows go through the row quantiser, and from 2048 rows
 * the activation and scale are applied by the quantiser as it loads the product's biased sums, off
 * the MFMA loop (below that, in the product's epilogue). int8 or Q8_0 weights, fast
 * mode, no accumulation
 * (TG_ERR_ARG), n <= 65536. Calls on one context share the workspace; they run in order on its
 * stream. Device pointers, queued on the stream. No counterpart in the reference, whose sums are all
 * f32. */
int tg_matmul_quantized_to_quant_device(tg_ctx *ctx, const void *qa, size_t qa_len, const int32_t *exps, size_t m,
                                        const tg_weights *w, const tg_epilogue *epi, void *qa_out,
                                        size_t qa_out_len, int32_t *exps_out, size_t exps_out_len);

/* out = glu(epi(a . w)): the convolution module's pointwise_conv1 followed by its GLU
 * (src/parakeet.rs:1087-1104, src/granite.rs:881-899: Kernels::linear into [m, n], then
 * out[r, j] = g[r, j] * sigmoid(g[r, n / 2 + j]) for j < n / 2 through Kernels::glu), giving
 * exactly what tg_linear_device followed by tg_glu_device writes. For int8 weights in fast mode
 * with n a multiple of 64, past the GEMV sizes, the GLU runs in the GEMM's epilogue and the
 * [m, n] product never reaches memory; otherwise the two steps run through a context-owned
 * buffer. out is [m, ldo] (ldo >= n / 2, out_len >= (m - 1) ldo + n / 2); epi may carry a bias
 * of n values, an activation and a scale, applied before the GLU, but not accumulate
 * (TG_ERR_ARG). n odd: TG_ERR_SHAPE. a holds m rows of k; a and out must not overlap. Device
 * pointers, queued on the stream. No single counterpart in the reference, which runs the two
 * kernels one after the other. */
int tg_linear_glu_device(tg_ctx *ctx, const float *a, size_t a_len, size_t m, const tg_weights *w, float *out,
                         size_t out_len, size_t ldo, const tg_epilogue *epi);

/* ---- row kernels -------------------------------------------------------------------------- */

/* out[r, j] = x[r, j] * sigmoid(x[r, half + j]) for j < half (the GLU of a convolution module),
 * with the exp of the reference's SIMD kernels. x_len and out_len are the buffers' lengths in
 * floats, checked against the rows the call reads and writes (TG_ERR_SHAPE), as the reference
 * asserts its slices (src/kernels/avx512.rs:412). Device pointers, queued on the stream. */
int tg_glu_device(tg_ctx *ctx, const float *x, size_t x_len, size_t ldx, size_t m, size_t half, float *out,
                  size_t out_len, size_t ldo);

/* softmax of each of m rows of n values, in place: Kernels::softmax as the reference's AVX-512
 * kernel computes it (src/kernels/mod.rs:460, src/kernels/avx512.rs:382-407): the row maximum,
 * e = exp(x - max) with the SIMD exp, sixteen partial sums of e (partial j over e[j], e[j + 16], ...
 * in order) folded by halves, then e * (1 / sum). Granite's self-conditioning applies it to the CTC
 * head's logits (src/granite.rs:1040-1069). x holds (m - 1) ldx + n floats (TG_ERR_SHAPE
 * otherwise). Device pointer, queued on the stream. */
int tg_softmax_device(tg_ctx *ctx, float *x, size_t x_len, size_t ldx, size_t m, size_t n);

/* Granite's strided-block pooling (src/granite.rs:918-931, the "pool" step of block_span): for each
 * of batch equal-length sequences of frames rows of x, output row r < frames / 2 of that sequence
 * (row b (frames / 2) + r of out) is (x[b frames + 2 r] + x[b frames + 2 r + 1]) / 2 over n values,
 * a last odd frame dropped. out must not overlap x (TG_ERR_ARG). Device pointers, queued on the
 * stream. */
int tg_average_pairs_device(tg_ctx *ctx, const float *x, size_t x_len, size_t ldx, size_t frames, size_t batch,
                            size_t n, float *out, size_t out_len, size_t ldo);

/* out[r, :] = LayerNorm(x[r, :]) * gamma + beta over n values per row, with the summation order of
 * the reference's AVX-512 layer_norm (src/kernels/avx512.rs:346-380). gamma and beta hold at least
 * n floats and x and out (m - 1) ld + n, as the reference asserts (avx512.rs:348; TG_ERR_SHAPE
 * otherwise); out may equal x. Device pointers, queued on the stream. */
int tg_layer_norm_device(tg_ctx *ctx, const float *x, size_t x_len, size_t ldx, size_t m, size_t n,
                         const float *gamma, size_t gamma_len, const float *beta, size_t beta_len, float eps,
                         float *out, size_t out_len, size_t ldo);

/* tg_layer_norm_device followed by tg_quantize_rows_device of its outputs, in one pass: the
 * quantised rows (qa, tg_quant_bytes(m, n) bytes) and their m exponents (exps) that
 * tg_matmul_quantized_device takes, bit-identical to the two calls. out, when not null, also gets
 * the f32 LayerNorm (and may equal x); the reference's callers (src/parakeet.rs:1023, 1052, 1085,
 * 1138) need only the product of the LayerNorm, so they pass null and the f32 rows never reach
 * memory. n <= 65536. Device pointers, queued on the stream. */
int tg_layer_norm_quant_device(tg_ctx *ctx, const float *x, size_t x_len, size_t ldx, size_t m, size_t n,
                               const float *gamma, size_t gamma_len, const float *beta, size_t beta_len, float eps,
                               float *out, size_t out_len, size_t ldo, void *qa, size_t qa_len, int32_t *exps,
                               size_t exps_len);

/* A stack's layer boundary in one call: x = LayerNorm(x; gamma, beta, eps) in place, as
 * tg_layer_norm_device writes it (a layer's last LayerNorm, norm_out, src/parakeet.rs:1168-1170),
 * then the quantised rows of LayerNorm(x; gamma2, beta2, eps2), as tg_layer_norm_quant_device
 * writes them (the next layer's first, norm_ff1, src/parakeet.rs:1026; the layers run in turn at
 * 893-894): bit-identical to those two calls.
 * Rows of at most 1024 values (a multiple of 4, 16-byte aligned) below 2048 rows take one launch
 * that reads each row once; other shapes run the two calls. n <= 65536. Device pointers, queued on
 * the stream. No counterpart in the reference, which runs the two LayerNorms as two calls. */
int tg_layer_norm_pair_quant_device(tg_ctx *ctx, float *x, size_t x_len, size_t ldx, size_t m, size_t n,
                                    const float *gamma, size_t gamma_len, const float *beta, size_t beta_len,
                                    float eps, const float *gamma2, size_t gamma2_len, const float *beta2,
                                    size_t beta2_len, float eps2, void *qa, size_t qa_len, int32_t *exps,
                                    size_t exps_len);

/* Depthwise 1-D convolution of frames x channels rows, "same" zero padding: output row r is frame
 * t = t0 + r * stride, out[r, c] = bias[c] + sum over taps j in order of w[j * channels + c] *
 * x[t + j - kernel/2, c], each term a rounded product and a rounded sum, taps outside [0, frames)
 * skipped: the reference's dwconv1d_frame (src/kernels/scalar.rs:164-187) called once per output
 * frame, as the conv modules do (src/parakeet.rs:1107-1122 with t = r; src/granite.rs:900-915
 * with t = stride * (out_start + r) - lo). act TG_ACT_SILU then applies the caller's
 * (k.silu)(row) (v / (1 + exp(0 - v)), src/kernels/avx512.rs:308-311, 432-443); TG_ACT_NONE leaves
 * the sums. w holds kernel x channels floats, bias channels floats. batch equal-length sequences
 * may be laid one after another (sequence b: input rows b * frames .., output rows b * rows ..),
 * each convolved on its own; batch = 1 is the reference's call. out must not overlap x. Device
 * pointers, queued on the stream. */
int tg_dwconv1d_device(tg_ctx *ctx, const float *x, size_t x_len, size_t ldx, size_t frames, size_t batch,
                       size_t channels, const float *w, size_t w_len, size_t kernel, const float *bias,
                       size_t bias_len, size_t t0, size_t stride, size_t rows, uint32_t act, float *out,
                       size_t out_len, size_t ldo);

/* The conv module's depthwise convolution + SiLU whose output only the next pointwise product reads
 * (Parakeet::layer, src/parakeet.rs:1105-1134: dwconv1d_frame for every frame, silu, then
 * conv_pw2): tg_dwconv1d_device over whole sequences (t0 = 0, stride = 1, rows = frames) whose
 * output rows are written quantised, qa and exps holding exactly what tg_quantize_rows_device
 * writes for those rows (k = channels), ready for tg_matmul_quantized_device. out (nullable) also
 * receives the f32 rows. Sequences are stacked along the rows (batch of them, frames rows each);
 * qa_len >= tg_quant_bytes(batch * frames, channels), exps_len >= batch * frames. channels 1 ..
 * 2048 and kernel 1 .. 32, else TG_ERR_UNSUPPORTED (the caller then makes the two calls). No
 * reference counterpart of its own: the fusion of two calls the reference makes in a row. */
int tg_dwconv1d_quant_device(tg_ctx *ctx, const float *x, size_t x_len, size_t ldx, size_t frames, size_t batch,
                             size_t channels, const float *w, size_t w_len, size_t kernel, const float *bias,
                             size_t bias_len, uint32_t act, float *out, size_t out_len, size_t ldo, void *qa,
                             size_t qa_len, int32_t *exps, size_t exps_len);

/* ---- the TDT decoder (src/parakeet.rs:1412-1577) --------------------------------------------
 * Parakeet's prediction network (embedding, LSTM layers, projection) and joint, decoded greedily
 * with every step on the device. The matrices are tg_weights of int8 or Q8_0 values. The network
 * keeps its own copies of the LSTM matrices and biases (rows interleaved so a unit's four gates meet
 * in one output quad); the joint, projection, their biases and the embedding stay the caller's and
 * must outlive the network. Every call on a network uses the network's scratch rows and decode
 * control block, so calls on one network must not overlap on the device: issue them through one
 * context, or synchronise between contexts. */
typedef struct tg_tdt tg_tdt;
typedef struct {
    size_t hidden;                 /* pred_hidden h: a multiple of 4, at most 992 */
    size_t vocab;                  /* tokens, the blank last (blank_token_id = vocab - 1) */
    const int32_t *durations;      /* host, n_durations values >= 0 (the TDT durations) */
    size_t n_durations;            /* 1 to 64 */
    size_t max_symbols;            /* max_symbols_per_step */
    size_t layers;                 /* LSTM layers, 1 to 4 */
    const tg_weights *joint;       /* (vocab + n_durations) x h */
    const float *joint_bias;       /* device, vocab + n_durations */
    const float *embedding;        /* device, vocab x h, 16-byte aligned */
    const tg_weights *lstm[4];     /* 4h x 2h: gates i, f, g, o of [x; h_l] */
    const float *lstm_bias[4];     /* device, 4h */
    const tg_weights *proj;        /* h x h */
    const float *proj_bias;        /* device, h */
    /* lengths in floats of the device buffers above, checked against what the network reads */
    size_t joint_bias_len, embedding_len, lstm_bias_len[4], proj_bias_len;
} tg_tdt_desc;
/* One emitted token (parakeet.rs Token): its id, its frame (relative to enc_proj's first row) and
 * its duration. */
typedef struct {
    uint32_t id, frame, duration;
} tg_token;
int tg_tdt_create(tg_ctx *ctx, const tg_tdt_desc *desc, tg_tdt **out);
void tg_tdt_destroy(tg_tdt *tdt);
/* Rows tg_tdt_predict_device takes at once (16 for Parakeet's h = 640). */
size_t tg_tdt_max_rows(const tg_tdt *tdt);
/* predict_rows (src/parakeet.rs:1524-1577): for each row r, the token's embedding runs through the
 * LSTM layers with row r's state (states: rows x layers x [h, c] of h floats each, updated in place),
 * and preds[r] = proj(h_last) + bias. Gate math as the reference's: sigmoid = 1 / (1 + exp(-x)),
 * tanh, c = f c + i g, h = o tanh(c). states_len and preds_len (floats) must cover rows of each
 * (TG_ERR_SHAPE). Device pointers, 16-byte aligned; queued on the stream. */
int tg_tdt_predict_device(tg_ctx *ctx, tg_tdt *tdt, const int32_t *tokens, size_t rows, float *states,
                          size_t states_len, float *preds, size_t preds_len);
/* decode_inner (src/parakeet.rs:1412-1513) from frame *frame with *on_frame tokens already on it:
 * per frame t, logits = joint(relu(enc_proj[t] + pred)) + bias; the token and duration are the
 * argmaxes of the vocabulary and duration logits; a blank moves max(duration, 1) frames, a token
 * is emitted, runs through the prediction network (state: layers x [h, c], and pred, updated in
 * place) and moves by its duration, or after max_symbols tokens of duration 0 by one frame. Runs
 * until t >= frames and returns the emitted tokens (at most cap into tokens; *count is the number
 * emitted, TG_ERR_SHAPE when it exceeds cap) with *frame and *on_frame where the loop stopped.
 * enc_proj: frames rows of h floats at stride lde, on the device; enc_len, state_len and pred_len
 * (floats) must cover what the decode reads (TG_ERR_SHAPE). Blocks until the decode ends. */
int tg_tdt_decode_device(tg_ctx *ctx, tg_tdt *tdt, const float *enc_proj, size_t enc_len, size_t lde, size_t frames,
                         float *state, size_t state_len, float *pred, size_t pred_len, size_t *frame,
                         size_t *on_frame, tg_token *tokens, size_t cap, size_t *count);
/* How tg_tdt_decode_device runs its steps (no counterpart in the reference, whose decode loop runs
 * on the host). Resident (the default where the network allows it: every matrix int8, or every one
 * Q8_0, vocab < 65535,
 * the panels fit the workgroups' LDS and the device takes cooperative launches): one launch makes
 * the steps with the matrices held in LDS across the device's CUs. Otherwise each step is four
 * kernels, replayed as a graph. Both give the same tokens, states and predictions.
 * tg_tdt_set_resident(on = 1) fails with TG_ERR_UNSUPPORTED when the network cannot run resident;
 * on = 0 selects the step kernels. tg_tdt_is_resident returns 1 when decodes run resident. */
int tg_tdt_set_resident(tg_ctx *ctx, tg_tdt *tdt, int on);
int tg_tdt_is_resident(const tg_tdt *tdt);
/* A resident launch holds most of the GPU's CUs until the decode ends, and two of them cannot be
 * resident on one GPU at once: within a process, one resident decode runs per device at a time,
 * and a decode that starts while another holds the device runs on the step kernels instead (same
 * results). Separate processes must not run resident decodes on the same GPU; give each process
 * its own GPU or call tg_tdt_set_resident(ctx, tdt, 0) in all but one.
 * tg_tdt_last_resident: 1 when the last tg_tdt_decode_device on this network ran resident, 0 when
 * it ran on the step kernels, -1 before the first. */
int tg_tdt_last_resident(const tg_tdt *tdt);
/* Steps the last resident decode on this network made (one step scores one window of frames). */
size_t tg_tdt_last_steps(const tg_tdt *tdt);

/* One stream of tg_tdt_decode_streams_device: tg_tdt_decode_device's arguments for that stream. */
typedef struct {
    const float *enc_proj; /* device, frames rows of hidden floats at stride lde */
    size_t enc_len, lde, frames;
    float *state;          /* device, updated in place */
    size_t state_len;
    float *pred;           /* device, updated in place */
    size_t pred_len;
    size_t frame, on_frame; /* in: where the stream's loop starts; out: where it stopped */
    tg_token *tokens;      /* host, cap entries */
    size_t cap;
    size_t count;          /* out: the tokens the stream emitted */
} tg_tdt_stream;
/* m independent greedy decodes (streams; parakeet.rs:1412-1513 per stream, as a caller decoding
 * several utterances at once calls decode_inner for each), each giving exactly what
 * tg_tdt_decode_device gives for it. Up to 8 streams run resident in one launch (no counterpart in
 * the reference): the joint scores 16 / m frames of each stream's window per step, each stream's
 * window is walked on its own, and the streams that emitted a token run the prediction network
 * together as rows of one MFMA product with the matrices in LDS (on Parakeet's decoder a step of 8
 * streams takes about three single-stream steps, so 8 streams decode 2.3 times one stream's tokens
 * per second). More than 8 streams go in groups of 8. Without the resident multi-stream
 * decode (Q8_0 or mixed matrices, the device's resident lock held elsewhere, tg_tdt_set_resident(0),
 * one stream) the streams are decoded one after another. tg_tdt_last_resident then reports 2 for a
 * multi-stream launch. Streams must not share state or pred. Blocks until every stream ends; on an
 * error (tokens past cap: TG_ERR_SHAPE) the other streams' results are still written. */
int tg_tdt_decode_streams_device(tg_ctx *ctx, tg_tdt *tdt, tg_tdt_stream *streams, size_t m);
/* Limits of the resident decode (no counterpart in the reference; for tests and tuning): the most
 * steps one launch makes before the host looks at the control block and relaunches (1 to 16384; 0
 * restores 16384), and the longest one workgroup waits for another, in microseconds (0 restores
 * one second). A wait that passes its limit ends the launch in every workgroup; the decode then
 * fails with TG_ERR_HIP and leaves state and pred as they were passed (*frame, *on_frame and the
 * tokens untouched), so the call can be repeated, resident or on the step kernels. */
int tg_tdt_set_resident_limits(tg_ctx *ctx, tg_tdt *tdt, uint32_t steps_per_launch, uint64_t wait_us);

/* ---- packs: the reference's weight files (src/pack.rs) -------------------------------------
 * A pack is "TELMOPAK", a u32 version (1) and 4 zero bytes; entries' data at multiples of 64
 * bytes; a JSON index; the index's offset and length (u64) and "TELMOIDX". Opening maps the file
 * read-only and checks the index as Pack::parse does, with its messages; entries are views into
 * the mapping until tg_pack_close. No device is needed except for tg_pack_upload_matrix. */
typedef struct tg_pack tg_pack;

enum { TG_ENTRY_MATRIX = 0, TG_ENTRY_F32 = 1, TG_ENTRY_BYTES = 2 };

typedef struct tg_pack_entry {
    const char *name;
    uint32_t type;        /* TG_ENTRY_* */
    uint32_t precision;   /* matrices: TG_F32 .. TG_Q8_0 */
    size_t n, k;          /* matrices: outputs, inputs */
    size_t rank;          /* f32 tensors: dimensions (at most 8) */
    size_t shape[8];
    const void *data;     /* panel values, tensor data or bytes */
    size_t bytes;
    const float *scales;  /* matrices with scales (int8, Q8_0), else null */
    size_t n_scales;
} tg_pack_entry;

/* TG_ERR_ARG for a file that is not a usable pack (message from tg_pack_last_error). */
int tg_pack_open(const char *path, tg_pack **out);
/* A pack held in memory (copied). */
int tg_pack_from_bytes(const void *data, size_t len, tg_pack **out);
void tg_pack_close(tg_pack *pack);
/* The message of this thread's last failed tg_pack_* call ("" if none). */
const char *tg_pack_last_error(void);
/* Whether the entries are a mapping of the file (else a copy in memory). */
int tg_pack_is_mapped(const tg_pack *pack);
const char *tg_pack_model(const tg_pack *pack);
/* A metadata value, or null if the key is absent. */
const char *tg_pack_meta(const tg_pack *pack, const char *key);
size_t tg_pack_meta_count(const tg_pack *pack);
int tg_pack_meta_at(const tg_pack *pack, size_t i, const char **key, const char **value);
size_t tg_pack_entry_count(const tg_pack *pack);
int tg_pack_entry_at(const tg_pack *pack, size_t i, tg_pack_entry *out);
/* The named entry; TG_ERR_ARG "Entry <name> is missing." when there is none. */
int tg_pack_find(const tg_pack *pack, const char *name, tg_pack_entry *out);
/* Pack::matrix then tg_weights_upload: the named matrix, which must be n x k, uploaded once
 * (TG_ERR_ARG if it is missing or not a matrix, TG_ERR_SHAPE if its shape differs). */
int tg_pack_upload_matrix(tg_ctx *ctx, const tg_pack *pack, const char *name, size_t n, size_t k,
                          tg_weights **out);

/* ---- the panel layout (host utilities, no device needed) ---------------------------------- */

size_t tg_panel_bytes(uint32_t precision, size_t n, size_t k);
size_t tg_scale_count(uint32_t precision, size_t n, size_t k);
int tg_fits(uint32_t precision, size_t k);
/* quant::encode of row-major f32 rows w[n][k] (Rows::F32). */
int tg_encode(const float *w, size_t n, size_t k, uint32_t precision, uint8_t *values, size_t values_len,
              float *scales, size_t n_scales);
/* The reference's test generator, random(len, seed) (src/kernels/mod.rs:795-805): xorshift64
 * (shifts 13, 7, 17) from the state seed * 0x9E3779B97F4A7C15 | 1, each step's top 24 bits mapped to
 * [-1, 1). Not part of the product path: exported so that harnesses draw telmo's seeded inputs. */
void tg_random(float *out, size_t len, uint64_t seed);
/* quant::decode into row-major out[n][k]. */
int tg_decode(const uint8_t *values, size_t values_len, const float *scales, size_t n_scales, uint32_t precision,
              size_t n, size_t k, float *out);

#ifdef __cplusplus
}
#endif

#endif /* TELMO_HIP_H */
