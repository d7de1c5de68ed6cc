/*
 * Oracle for telmo's int8-weight matrix product: a plain-C restatement of the reference's
 * CPU algorithm. TEST INFRASTRUCTURE ONLY. Only tests/, __graft_entry__.smoke() and the
 * bench's cpu_baseline leg load this library, and only to check results against. The product
 * path (telmo_amd/) never links, loads or calls it.
 *
 * Built with -ffp-contract=off so that every `a * b + c` below is two roundings, and
 * every fused step is an explicit fmaf().
 *
 * What each part follows (paths relative to the reference repository):
 *   or_random             src/kernels/mod.rs:795-805   (xorshift test generator)
 *   or_f32_to_f16 ...     src/quant.rs:91-164          (RNE half / bfloat16 conversions)
 *   or_quantize_q8_0_block src/quant.rs:176-187
 *   or_quantize_row_int8  src/quant.rs:189-198
 *   or_encode_*           src/quant.rs:200-269         (the 16-output panel layout)
 *   or_decode             src/quant.rs:271-303
 *   or_widen              src/kernels/scalar.rs:54-107 (== avx512.rs:220-265, bit for bit)
 *   or_tile               src/kernels/scalar.rs:26-49 (unfused) and avx512.rs:70-105,
 *                         avx2.rs:62-107 (fused, sums in input order)
 *   or_exp_simd           src/kernels/avx512.rs:279-304 == avx2.rs:305-331 (same steps)
 *   or_glu                src/kernels/avx512.rs:410-430
 *   or_layer_norm         src/kernels/avx512.rs:346-380 (AVX-512 summation order)
 *   or_softmax            src/kernels/avx512.rs:382-407 (AVX-512 order; the bits of rows holding a
 *                         NaN depend on the register maximum's fold, which the reference leaves to
 *                         the compiler: those rows are parity unpinned)
 *   or_dwconv1d_frame     src/kernels/scalar.rs:164-187 (== avx512.rs:445-459, the same loop)
 *   or_dwconv1d           src/parakeet.rs:1107-1122, src/granite.rs:900-915 (one frame per
 *                         output row, then silu, avx512.rs:308-311 and 432-443)
 *   or_tdt_predict        src/parakeet.rs:1524-1577 (predict_rows), its products by the fast path's
 *                         integer oracle, sigmoid as parakeet.rs:1678-1680, libm expf / tanhf
 *   or_tdt_decode         src/parakeet.rs:1412-1513 (decode_inner), argmax as parakeet.rs:1682-1691
 *   or_store              src/kernels/scalar.rs:110-124 (unfused, libm exp) and
 *                         avx512.rs:313-343 (fused ISAs)
 *   or_matmul             src/kernels/mod.rs:530-688   (gemm_panels with KC = 256, the
 *                         direct-narrow rule, matmul's preconditions and early return)
 *
 * Pinning (tests/test_oracle_*.py): the quant known answers of src/quant.rs:305-455, every
 * half bit pattern, numpy's float16 conversion on random values, exact-rational FMA sums for
 * the fused tile, an f64 triple loop within 1e-5*sqrt(k)*(1+|w|) (src/kernels/mod.rs:962-1005),
 * widen == decode for every int8 value and every scale exponent (mod.rs:1130-1183), and
 * exp/sigmoid accuracy against math.exp (mod.rs:1261-1277), the depthwise convolution against
 * an f64 direct sum (mod.rs:1279-1300), exact integer correlations (numpy) and numpy's per-op
 * float32 rounding.
 *
 * The second half of the file is the integer oracle of telmo_amd's fast path (two int8
 * digits per activation, exact i32 sums, one shared dequantisation). It has no counterpart
 * in the reference; tests pin it with numpy int64 products and invariants of the digit split.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#define PANEL 16
#define Q8_BLOCK 32
#define KC 256

enum { P_F32 = 0, P_F16 = 1, P_BF16 = 2, P_INT8 = 3, P_Q8_0 = 4 };
enum { ACT_NONE = 0, ACT_RELU = 1, ACT_SILU = 2 };
enum { OR_OK = 0, OR_ERR_SHAPE = -2, OR_ERR_ARG = -7 };

static float from_bits(uint32_t b) { float f; memcpy(&f, &b, 4); return f; }
static uint32_t to_bits(float f) { uint32_t b; memcpy(&b, &f, 4); return b; }
static size_t div_ceil(size_t a, size_t b) { return (a + b - 1) / b; }

/* ---------------------------------------------------------------- test generator */

void or_random(float *out, size_t len, uint64_t seed) {
    uint64_t s = seed * 0x9E3779B97F4A7C15ull | 1u;
    for (size_t i = 0; i < len; i++) {
        s ^= s << 13;
        s ^= s >> 7;
        s ^= s << 17;
        out[i] = ((float)(s >> 40) / (float)(1ull << 24)) * 2.0f - 1.0f;
    }
}

/* ---------------------------------------------------------------- precisions */

size_t or_value_bytes(int p) {
    switch (p) {
    case P_F32: return 4;
    case P_F16: case P_BF16: return 2;
    case P_INT8: case P_Q8_0: return 1;
    default: return 0;
    }
}

size_t or_panel_bytes(int p, size_t n, size_t k) { return div_ceil(n, PANEL) * k * PANEL * or_value_bytes(p); }

size_t or_scale_count(int p, size_t n, size_t k) {
    size_t panels = div_ceil(n, PANEL);
    if (p == P_INT8) return panels * PANEL;
    if (p == P_Q8_0) return panels * div_ceil(k, Q8_BLOCK) * PANEL;
    return 0;
}

int or_fits(int p, size_t k) { return p != P_Q8_0 || k % Q8_BLOCK == 0; }

uint16_t or_f32_to_f16(float x) {
    uint32_t bits = to_bits(x);
    uint16_t sign = (uint16_t)((bits >> 16) & 0x8000);
    int32_t exp = (int32_t)((bits >> 23) & 0xff);
    uint32_t man = bits & 0x7fffff;
    if (exp == 0xff) {
        uint16_t nan = man != 0 ? (uint16_t)(0x200 | (man >> 13)) : 0;
        return sign | 0x7c00 | nan;
    }
    int32_t e = exp - 127 + 15;
    if (e >= 0x1f) return sign | 0x7c00;
    if (e <= 0) {
        uint32_t shift = (uint32_t)(126 - exp);
        if (shift > 24) return sign;
        uint32_t full = man | 0x800000;
        uint32_t m = full >> shift;
        uint32_t rem = full & ((1u << shift) - 1);
        uint32_t half = 1u << (shift - 1);
        if (rem > half || (rem == half && (m & 1))) m += 1;
        return sign | (uint16_t)m;
    }
    uint32_t h = ((uint32_t)e << 10) | (man >> 13);
    uint32_t rem = man & 0x1fff;
    if (rem > 0x1000 || (rem == 0x1000 && (h & 1))) h += 1;
    return sign | (uint16_t)h;
}

float or_f16_to_f32(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000) << 16;
    uint32_t exp = (h >> 10) & 0x1f, man = h & 0x3ff;
    if (exp == 0 && man == 0) return from_bits(sign);
    if (exp == 0) {
        float v = (float)man * (1.0f / (float)(1u << 24));
        return sign ? -v : v;
    }
    if (exp == 0x1f && man != 0) return from_bits(sign | 0x7fc00000u | (man << 13));
    if (exp == 0x1f) return from_bits(sign | 0x7f800000u);
    return from_bits(sign | ((exp + 112) << 23) | (man << 13));
}

uint16_t or_f32_to_bf16(float x) {
    uint32_t bits = to_bits(x);
    if (isnan(x)) return (uint16_t)((bits >> 16) | 0x40);
    return (uint16_t)((bits + 0x7fff + ((bits >> 16) & 1)) >> 16);
}

float or_bf16_to_f32(uint16_t h) { return from_bits((uint32_t)h << 16); }

/* Rust's `f32 as i8`: saturating, NaN to 0. */
static int8_t as_i8(float v) {
    if (isnan(v)) return 0;
    if (v >= 127.0f) return 127;
    if (v <= -128.0f) return -128;
    return (int8_t)v;
}

/* The largest magnitude, NaN-ignoring like Rust's f32::max. */
static float amax_of(const float *x, size_t len) {
    float m = 0.0f;
    for (size_t i = 0; i < len; i++) m = fmaxf(m, fabsf(x[i]));
    return m;
}

float or_quantize_q8_0_block(const float *x, size_t len, int8_t *q) {
    float d = amax_of(x, len) / 127.0f;
    float id = d != 0.0f ? 1.0f / d : 0.0f;
    for (size_t i = 0; i < len; i++) q[i] = as_i8(roundf(x[i] * id));
    return or_f16_to_f32(or_f32_to_f16(d));
}

float or_quantize_row_int8(const float *x, size_t len, int8_t *q) {
    float d = amax_of(x, len) / 127.0f;
    float id = d != 0.0f ? 1.0f / d : 0.0f;
    for (size_t i = 0; i < len; i++) {
        float v = roundf(x[i] * id);
        if (!isnan(v)) v = v < -127.0f ? -127.0f : (v > 127.0f ? 127.0f : v);
        q[i] = as_i8(v);
    }
    return d;
}

/* The panel layout. `w` is row-major [n][k] f32 (Rows::F32) or, with `d` set, Q8_0 blocks
 * (Rows::Q8_0: d holds n*k/32 scales and q the n*k values). */
static int encode(const float *w, const float *d, const int8_t *qsrc, size_t n, size_t k, int p,
                  uint8_t *values, float *scales) {
    if (!or_fits(p, k) || or_value_bytes(p) == 0) return OR_ERR_ARG;
    size_t vb = or_value_bytes(p), blocks = div_ceil(k, Q8_BLOCK);
    memset(values, 0, or_panel_bytes(p, n, k));
    size_t ns = or_scale_count(p, n, k);
    for (size_t i = 0; i < ns; i++) scales[i] = 0.0f;
    float *row = (float *)calloc(k ? k : 1, sizeof(float));
    int8_t *q = (int8_t *)calloc(k ? k : 1, 1);
    for (size_t o = 0; o < n; o++) {
        size_t pp = o / PANEL, j = o % PANEL;
        uint8_t *panel = values + pp * k * PANEL * vb;
        if (d && p == P_Q8_0) {
            memcpy(q, qsrc + o * k, k);
            for (size_t b = 0; b < blocks; b++) scales[(pp * blocks + b) * PANEL + j] = d[o * blocks + b];
        } else {
            if (d) {
                for (size_t i = 0; i < k; i++) row[i] = (float)qsrc[o * k + i] * d[o * blocks + i / Q8_BLOCK];
            } else {
                memcpy(row, w + o * k, k * sizeof(float));
            }
            if (p == P_INT8) {
                scales[pp * PANEL + j] = or_quantize_row_int8(row, k, q);
            } else if (p == P_Q8_0) {
                for (size_t b = 0; b < blocks; b++) {
                    size_t lo = b * Q8_BLOCK, hi = (b + 1) * Q8_BLOCK < k ? (b + 1) * Q8_BLOCK : k;
                    scales[(pp * blocks + b) * PANEL + j] = or_quantize_q8_0_block(row + lo, hi - lo, q + lo);
                }
            }
        }
        for (size_t i = 0; i < k; i++) {
            uint8_t *at = panel + (i * PANEL + j) * vb;
            switch (p) {
            case P_F32: { uint32_t b = to_bits(row[i]); memcpy(at, &b, 4); break; }
            case P_F16: { uint16_t h = or_f32_to_f16(row[i]); memcpy(at, &h, 2); break; }
            case P_BF16: { uint16_t h = or_f32_to_bf16(row[i]); memcpy(at, &h, 2); break; }
            default: at[0] = (uint8_t)q[i]; break;
            }
        }
    }
    free(row);
    free(q);
    return OR_OK;
}

int or_encode_f32(const float *w, size_t n, size_t k, int p, uint8_t *values, float *scales) {
    return encode(w, NULL, NULL, n, k, p, values, scales);
}

int or_encode_q8(const float *d, const int8_t *q, size_t n, size_t k, int p, uint8_t *values, float *scales) {
    return encode(NULL, d, q, n, k, p, values, scales);
}

static float decode_value(const uint8_t *values, const float *scales, size_t k, int p, size_t o, size_t i) {
    size_t vb = or_value_bytes(p), blocks = div_ceil(k, Q8_BLOCK);
    size_t pp = o / PANEL, j = o % PANEL;
    const uint8_t *b = values + ((pp * k + i) * PANEL + j) * vb;
    switch (p) {
    case P_F32: { uint32_t u; memcpy(&u, b, 4); return from_bits(u); }
    case P_F16: { uint16_t h; memcpy(&h, b, 2); return or_f16_to_f32(h); }
    case P_BF16: { uint16_t h; memcpy(&h, b, 2); return or_bf16_to_f32(h); }
    case P_INT8: return (float)(int8_t)b[0] * scales[pp * PANEL + j];
    default: return (float)(int8_t)b[0] * scales[(pp * blocks + i / Q8_BLOCK) * PANEL + j];
    }
}

void or_decode(const uint8_t *values, const float *scales, size_t n, size_t k, int p, float *out) {
    for (size_t o = 0; o < n; o++)
        for (size_t i = 0; i < k; i++) out[o * k + i] = decode_value(values, scales, k, p, o, i);
}

/* ---------------------------------------------------------------- kernels */

/* `k` inputs of one panel to f32 (`k * 16` values). `scales` is the panel's 16 scales for
 * int8, or the 16 scales of the first block of 32 inputs for Q8_0. */
void or_widen(int p, size_t k, const uint8_t *src, const float *scales, float *out) {
    for (size_t i = 0; i < k; i++) {
        for (size_t j = 0; j < PANEL; j++) {
            size_t e = i * PANEL + j;
            switch (p) {
            case P_F32: { uint32_t u; memcpy(&u, src + e * 4, 4); out[e] = from_bits(u); break; }
            case P_F16: { uint16_t h; memcpy(&h, src + e * 2, 2); out[e] = or_f16_to_f32(h); break; }
            case P_BF16: { uint16_t h; memcpy(&h, src + e * 2, 2); out[e] = or_bf16_to_f32(h); break; }
            case P_INT8: out[e] = (float)(int8_t)src[e] * scales[j]; break;
            default: out[e] = (float)(int8_t)src[e] * scales[i / Q8_BLOCK * PANEL + j]; break;
            }
        }
    }
}

/* A rows x 16 tile of a * b into out (row stride 16), continuing from out when `load`. Each
 * output is the sum of its products in input order: fused (fmaf) or, for the scalar ISA,
 * a rounded product then a rounded add. */
void or_tile(int fused, size_t k, const float *a, size_t lda, size_t rows, const float *b, size_t k_stride,
             float *out, int load) {
    for (size_t r = 0; r < rows; r++) {
        float *acc = out + r * PANEL;
        if (!load)
            for (size_t j = 0; j < PANEL; j++) acc[j] = 0.0f;
        for (size_t i = 0; i < k; i++) {
            float av = a[r * lda + i];
            const float *bp = b + i * k_stride;
            for (size_t j = 0; j < PANEL; j++) acc[j] = fused ? fmaf(av, bp[j], acc[j]) : acc[j] + av * bp[j];
        }
    }
}

/* x86 MAXPS / MINPS of (a, b): a if a > b (a < b), else b. A NaN in either gives b. */
static float x86_max(float a, float b) { return a > b ? a : b; }
static float x86_min(float a, float b) { return a < b ? a : b; }

/* e^x with the steps of the reference's 8- and 16-lane SIMD exp: clamp, n = rint(x log2 e),
 * two-part Cody-Waite reduction, a degree-6 polynomial in fused steps, then times 2^n. */
float or_exp_simd(float x) {
    x = x86_min(x86_max(x, -87.33654f), 88.37626f);
    float n = rintf(x * 1.44269504088896340736f);
    float r = fmaf(-n, 0.6933594f, x);
    r = fmaf(-n, -2.1219444e-4f, r);
    float p = 1.9875691e-4f;
    p = fmaf(p, r, 1.3982e-3f);
    p = fmaf(p, r, 8.333452e-3f);
    p = fmaf(p, r, 4.1665796e-2f);
    p = fmaf(p, r, 0.16666665f);
    p = fmaf(p, r, 0.5f);
    p = fmaf(p, r * r, r);
    p = p + 1.0f;
    float pow2n = from_bits((uint32_t)((int32_t)n + 127) << 23);
    return p * pow2n;
}

float or_silu_simd(float v) { return v / (1.0f + or_exp_simd(0.0f - v)); }

/* glu: out = a / (1 + exp(0 - b)) with the SIMD exp (src/kernels/avx512.rs:410-430). */
void or_glu(const float *a, const float *b, float *out, size_t n) {
    for (size_t i = 0; i < n; i++) out[i] = a[i] / (1.0f + or_exp_simd(0.0f - b[i]));
}

/* Sum of sixteen partials as the reduction of a 512-bit register: halves added lane by lane
 * (j + 8, then j + 4, j + 2, j + 1). */
static float reduce16(const float *p) {
    float h8[8], h4[4], h2[2];
    for (int j = 0; j < 8; j++) h8[j] = p[j] + p[j + 8];
    for (int j = 0; j < 4; j++) h4[j] = h8[j] + h8[j + 4];
    for (int j = 0; j < 2; j++) h2[j] = h4[j] + h4[j + 2];
    return h2[0] + h2[1];
}

/* layer_norm of one row, AVX-512 (src/kernels/avx512.rs:346-380): sixteen partial sums over the
 * row in steps of 16 (masked tail lanes add zero), reduced; mean = sum / n; partial fma(d, d, q)
 * with d = x - mean (zero in masked lanes); rstd = 1 / sqrt(q / n + eps); out = fma((x - mean) *
 * rstd, gamma, beta). */
void or_layer_norm(const float *x, size_t n, float *out, const float *gamma, const float *beta, float eps) {
    float s[16] = {0}, q[16] = {0};
    for (size_t i = 0; i < n; i += 16)
        for (size_t j = 0; j < 16; j++) s[j] = s[j] + (i + j < n ? x[i + j] : 0.0f);
    const float mean = reduce16(s) / (float)n;
    for (size_t i = 0; i < n; i += 16)
        for (size_t j = 0; j < 16; j++) {
            const float d = i + j < n ? x[i + j] - mean : 0.0f;
            q[j] = fmaf(d, d, q[j]);
        }
    const float rstd = 1.0f / sqrtf(reduce16(q) / (float)n + eps);
    for (size_t i = 0; i < n; i++) {
        const float d = (x[i] - mean) * rstd;
        out[i] = fmaf(d, gamma[i], beta[i]);
    }
}

/* softmax of one row in place, AVX-512 (src/kernels/avx512.rs:382-407): sixteen lane maxima from
 * -inf (x86 MAXPS, masked tail lanes loading -inf), folded by halves with the lower lane first;
 * e = exp_simd(x - max) stored over x; sixteen partial sums of e from +0 in steps of 16 (masked
 * tail lanes keep their partial), reduced as reduce16; inv = 1 / sum; x = e * inv. */
void or_softmax(float *x, size_t n) {
    float mx[16], s[16] = {0};
    for (int j = 0; j < 16; j++) mx[j] = -INFINITY;
    for (size_t i = 0; i < n; i += 16)
        for (size_t j = 0; j < 16; j++) mx[j] = x86_max(mx[j], i + j < n ? x[i + j] : -INFINITY);
    for (int h = 8; h >= 1; h >>= 1)
        for (int j = 0; j < h; j++) mx[j] = x86_max(mx[j], mx[j + h]);
    const float vmax = mx[0];
    for (size_t i = 0; i < n; i += 16)
        for (size_t j = 0; j < 16 && i + j < n; j++) {
            const float e = or_exp_simd(x[i + j] - vmax);
            x[i + j] = e;
            s[j] = s[j] + e;
        }
    const float inv = 1.0f / reduce16(s);
    for (size_t i = 0; i < n; i++) x[i] = x[i] * inv;
}

/* One output frame of the depthwise convolution (src/kernels/scalar.rs:164-187): out = bias, then
 * for each tap j in order whose source frame t + j - kernel/2 lies in [0, frames), out[c] =
 * out[c] + w[j * channels + c] * input[src * channels + c], a rounded product then a rounded sum. */
void or_dwconv1d_frame(const float *input, size_t channels, size_t frames, size_t t, const float *w, size_t kernel,
                       const float *bias, float *out) {
    memcpy(out, bias, channels * sizeof(float));
    const size_t half = kernel / 2;
    for (size_t j = 0; j < kernel; j++) {
        if (t + j < half || t + j - half >= frames) continue;
        const float *row = input + (t + j - half) * channels;
        const float *wj = w + j * channels;
        for (size_t c = 0; c < channels; c++) out[c] = out[c] + wj[c] * row[c];
    }
}

/* The conv modules' loop: output row r (stride ldo) is or_dwconv1d_frame at t = t0 + r * stride
 * over the frames of input (stride ldx), then, when silu is set, v / (1 + exp(0 - v)) with the
 * SIMD exp (src/kernels/avx512.rs:308-311). */
void or_dwconv1d(const float *input, size_t ldx, size_t frames, size_t channels, const float *w, size_t kernel,
                 const float *bias, size_t t0, size_t stride, size_t rows, int silu, float *out, size_t ldo) {
    float *dense = malloc((frames ? frames : 1) * channels * sizeof(float));
    for (size_t f = 0; f < frames; f++) memcpy(dense + f * channels, input + f * ldx, channels * sizeof(float));
    for (size_t r = 0; r < rows; r++) {
        float *o = out + r * ldo;
        or_dwconv1d_frame(dense, channels, frames, t0 + r * stride, w, kernel, bias, o);
        if (silu)
            for (size_t c = 0; c < channels; c++) o[c] = or_silu_simd(o[c]);
    }
    free(dense);
}

float or_activate_scalar(float v, int act) {
    switch (act) {
    case ACT_RELU: return fmaxf(v, 0.0f);
    case ACT_SILU: return v / (1.0f + expf(-v));
    default: return v;
    }
}

/* The epilogue over `cols` columns: c = (accumulate ? c : 0) + scale * act(acc + bias). */
void or_store(int fused, const float *acc, float *c, size_t cols, const float *bias, int act, float scale,
              int accumulate) {
    for (size_t j = 0; j < cols; j++) {
        float v;
        if (fused) {
            v = acc[j];
            if (bias) v = v + bias[j];
            if (act == ACT_RELU) v = x86_max(v, 0.0f);
            else if (act == ACT_SILU) v = or_silu_simd(v);
        } else {
            v = acc[j] + (bias ? bias[j] : 0.0f);
            v = or_activate_scalar(v, act);
        }
        v = v * scale;
        c[j] = accumulate ? c[j] + v : v;
    }
}

/* Kernels::matmul over packed weights: c[m, n] = epilogue(a[m, k] * w^T). Returns 0, or
 * OR_ERR_SHAPE where the reference asserts. Sums run in gemm_panels' order: per panel, KC
 * blocks of inputs continue the stored partial sums, so each output is summed in input order
 * whatever the blocking; tile_rows only groups rows. Panels are split across OpenMP threads
 * as the reference splits them across its pool, which changes no result. */
int or_matmul(int fused, const float *a, size_t a_len, size_t lda, size_t m, const uint8_t *values,
              const float *scales, int p, size_t n, size_t k, float *c, size_t c_len, size_t ldc,
              const float *bias, size_t bias_len, int act, float scale, int accumulate) {
    if (m == 0 || n == 0) return OR_OK;
    if (lda < k || ldc < n) return OR_ERR_SHAPE;
    if (a_len < (m - 1) * lda + k) return OR_ERR_SHAPE;
    if (c_len < (m - 1) * ldc + n) return OR_ERR_SHAPE;
    if (bias && bias_len < n) return OR_ERR_SHAPE;
    if (!or_fits(p, k) || or_value_bytes(p) == 0) return OR_ERR_ARG;
    size_t tile_rows = fused ? 8 : 6;
    size_t vb = or_value_bytes(p), blocks = div_ceil(k, Q8_BLOCK), panels = div_ceil(n, PANEL);
#pragma omp parallel
    {
        float *wide = (float *)malloc(KC * PANEL * sizeof(float));
        float *partial = (float *)calloc(m * PANEL, sizeof(float));
#pragma omp for schedule(static)
        for (size_t pp = 0; pp < panels; pp++) {
            size_t col = pp * PANEL, cols = n - col < PANEL ? n - col : PANEL;
            for (size_t k0 = 0; k0 < k; k0 += KC) {
                size_t kc = k - k0 < KC ? k - k0 : KC;
                const float *sc = NULL;
                if (p == P_INT8) sc = scales + pp * PANEL;
                if (p == P_Q8_0) sc = scales + (pp * blocks + k0 / Q8_BLOCK) * PANEL;
                or_widen(p, kc, values + (pp * k + k0) * PANEL * vb, sc, wide);
                for (size_t row = 0; row < m; row += tile_rows) {
                    size_t rows = m - row < tile_rows ? m - row : tile_rows;
                    or_tile(fused, kc, a + row * lda + k0, lda, rows, wide, PANEL, partial + row * PANEL, k0 > 0);
                }
            }
            for (size_t r = 0; r < m; r++)
                or_store(fused, partial + r * PANEL, c + r * ldc + col, cols, bias ? bias + col : NULL, act, scale,
                         accumulate);
        }
        free(wide);
        free(partial);
    }
    return OR_OK;
}

/* ---------------------------------------------------------------- integer oracle of the fast path
 *
 * Each activation row is scaled by a power of two 2^e chosen from the row's largest magnitude
 * so that v = rint(a * 2^e) fits |v| <= 32639, and v is split into two signed int8 digits,
 * v = 256 * hi + lo with lo in [-128, 127]. The product sums hi * q and lo * q exactly in i32,
 * and one shared dequantisation turns them into the f32 sum that the epilogue takes:
 *     S = 256 * acc_hi + acc_lo (exact, 64-bit);  u = (float)S * scale_n + 0;  sum = u * 2^-e.
 * A row holding a NaN or an infinity gives NaN sums (e = OR_EXP_NONFINITE).
 */
#define OR_EXP_NONFINITE INT32_MIN
#define DIGIT_MAX 32639.0f

/* The exponent E with x = m * 2^E, m in [0.5, 1), for a positive finite x, from its bits. */
static int32_t frexp_exponent(float x) {
    uint32_t b = to_bits(x);
    int32_t be = (int32_t)(b >> 23);
    if (be == 0) {
        uint32_t man = b & 0x7fffff;
        int32_t top = 31 - __builtin_clz(man);
        return top - 148;
    }
    return be - 126;
}

int32_t or_row_exponent(const float *a, size_t k) {
    float amax = 0.0f;
    for (size_t i = 0; i < k; i++) {
        if (!isfinite(a[i])) return OR_EXP_NONFINITE;
        amax = fmaxf(amax, fabsf(a[i]));
    }
    if (amax == 0.0f) return 0;
    int32_t e = 15 - frexp_exponent(amax);
    if (ldexpf(amax, e) > DIGIT_MAX) e -= 1;
    return e;
}

/* The accuracy guard's flag of one row (telmo_amd's fast path; no reference counterpart): with e
 * the row exponent, x = ldexp(a, e), v = rint(x) (the two digits' value) and d = rint(256 (x - v))
 * (the next eight bits), the row is flagged when 256 sum d^2 > sum v^2, summed as exact integers.
 * Rows holding a NaN or an infinity are not flagged. A flagged row's outputs are the fused
 * reference's (or_matmul). */
int or_guard_flag(const float *a, size_t k) {
    const int32_t e = or_row_exponent(a, k);
    if (e == OR_EXP_NONFINITE) return 0;
    int64_t vv = 0, dd = 0;
    for (size_t i = 0; i < k; i++) {
        const float x = ldexpf(a[i], e), v = rintf(x);
        const int64_t d = (int64_t)rintf((x - v) * 256.0f), iv = (int64_t)v;
        vv += iv * iv;
        dd += d * d;
    }
    return 256 * dd > vv;
}

/* Digits of rows a[m][lda] into hi/lo [m][k] and exponents [m]. */
void or_quantize_rows(const float *a, size_t lda, size_t m, size_t k, int8_t *hi, int8_t *lo, int32_t *ex) {
    for (size_t r = 0; r < m; r++) {
        const float *row = a + r * lda;
        int32_t e = or_row_exponent(row, k);
        ex[r] = e;
        for (size_t i = 0; i < k; i++) {
            int32_t v = e == OR_EXP_NONFINITE ? 0 : (int32_t)rintf(ldexpf(row[i], e));
            int32_t l = ((v + 128) & 255) - 128;
            hi[r * k + i] = (int8_t)((v - l) >> 8);
            lo[r * k + i] = (int8_t)l;
        }
    }
}

/* acc[m][n] = sum_i digits[m][i] * q[n][i], exactly, for both digit planes. `q` is [n][k]. */
void or_int_products(const int8_t *hi, const int8_t *lo, size_t m, size_t k, const int8_t *q, size_t n,
                     int32_t *acc_hi, int32_t *acc_lo) {
    for (size_t r = 0; r < m; r++)
        for (size_t o = 0; o < n; o++) {
            int64_t sh = 0, sl = 0;
            for (size_t i = 0; i < k; i++) {
                sh += (int64_t)hi[r * k + i] * q[o * k + i];
                sl += (int64_t)lo[r * k + i] * q[o * k + i];
            }
            acc_hi[r * n + o] = (int32_t)sh;
            acc_lo[r * n + o] = (int32_t)sl;
        }
}

float or_dequant(int32_t acc_hi, int32_t acc_lo, int32_t e, float scale) {
    if (e == OR_EXP_NONFINITE) return NAN;
    int64_t s = (int64_t)acc_hi * 256 + acc_lo;
    float u = (float)s * scale + 0.0f;
    return ldexpf(u, -e);
}

/* The whole fast path for int8 weights in the panel layout: same arguments and checks as
 * or_matmul, with the fused epilogue. k is at most 65536, so |acc| < 2^30. */
int or_matmul_fast(const float *a, size_t a_len, size_t lda, size_t m, const uint8_t *values, const float *scales,
                   size_t n, size_t k, float *c, size_t c_len, size_t ldc, const float *bias, size_t bias_len,
                   int act, float scale, int accumulate) {
    if (m == 0 || n == 0) return OR_OK;
    if (lda < k || ldc < n) return OR_ERR_SHAPE;
    if (a_len < (m - 1) * lda + k) return OR_ERR_SHAPE;
    if (c_len < (m - 1) * ldc + n) return OR_ERR_SHAPE;
    if (bias && bias_len < n) return OR_ERR_SHAPE;
    if (k > 65536) return OR_ERR_ARG;
    size_t kk = k ? k : 1, panels = div_ceil(n, PANEL);
    int8_t *hi = (int8_t *)malloc(m * kk), *lo = (int8_t *)malloc(m * kk);
    int32_t *ex = (int32_t *)malloc(m * sizeof(int32_t));
    int8_t *qt = (int8_t *)malloc(panels * PANEL * kk);
    or_quantize_rows(a, lda, m, k, hi, lo, ex);
    for (size_t o = 0; o < panels * PANEL; o++)
        for (size_t i = 0; i < k; i++) qt[o * kk + i] = (int8_t)values[((o / PANEL) * k + i) * PANEL + o % PANEL];
#pragma omp parallel for schedule(dynamic, 1)
    for (size_t r = 0; r < m; r++) {
        float sums[PANEL];
        for (size_t o0 = 0; o0 < n; o0 += PANEL) {
            size_t cols = n - o0 < PANEL ? n - o0 : PANEL;
            for (size_t j = 0; j < cols; j++) {
                const int8_t *q = qt + (o0 + j) * kk, *h = hi + r * kk, *l = lo + r * kk;
                int32_t sh = 0, sl = 0;
                for (size_t i = 0; i < k; i++) {
                    sh += (int32_t)h[i] * q[i];
                    sl += (int32_t)l[i] * q[i];
                }
                sums[j] = or_dequant(sh, sl, ex[r], scales[o0 + j]);
            }
            or_store(1, sums, c + r * ldc + o0, cols, bias ? bias + o0 : NULL, act, scale, accumulate);
        }
    }
    free(hi);
    free(lo);
    free(ex);
    free(qt);
    return OR_OK;
}

/* The fast path for Q8_0 weights (no counterpart in the reference, whose sums are all f32): per
 * 32-input block b of output o, T_b = 256 sum(hi q) + sum(lo q) exactly (|T_b| < 2^31), then
 * F = fmaf(d[o][b], (float)T_b, F) over the blocks in order from +0, and the row's 2^-e. NaN
 * for rows holding a NaN or infinity. The epilogue is the fused one. */
int or_matmul_fast_q8(const float *a, size_t a_len, size_t lda, size_t m, const uint8_t *values, const float *scales,
                      size_t n, size_t k, float *c, size_t c_len, size_t ldc, const float *bias, size_t bias_len,
                      int act, float scale, int accumulate) {
    if (m == 0 || n == 0) return OR_OK;
    if (lda < k || ldc < n) return OR_ERR_SHAPE;
    if (a_len < (m - 1) * lda + k) return OR_ERR_SHAPE;
    if (c_len < (m - 1) * ldc + n) return OR_ERR_SHAPE;
    if (bias && bias_len < n) return OR_ERR_SHAPE;
    if (k > 65536 || k % Q8_BLOCK) return OR_ERR_ARG;
    size_t kk = k ? k : 1, panels = div_ceil(n, PANEL), blocks = k / Q8_BLOCK;
    int8_t *hi = (int8_t *)malloc(m * kk), *lo = (int8_t *)malloc(m * kk);
    int32_t *ex = (int32_t *)malloc(m * sizeof(int32_t));
    int8_t *qt = (int8_t *)malloc(panels * PANEL * kk);
    or_quantize_rows(a, lda, m, k, hi, lo, ex);
    for (size_t o = 0; o < panels * PANEL; o++)
        for (size_t i = 0; i < k; i++) qt[o * kk + i] = (int8_t)values[((o / PANEL) * k + i) * PANEL + o % PANEL];
#pragma omp parallel for schedule(dynamic, 1)
    for (size_t r = 0; r < m; r++) {
        float sums[PANEL];
        for (size_t o0 = 0; o0 < n; o0 += PANEL) {
            size_t cols = n - o0 < PANEL ? n - o0 : PANEL;
            for (size_t j = 0; j < cols; j++) {
                const size_t o = o0 + j, p = o / PANEL;
                const int8_t *q = qt + o * kk, *h = hi + r * kk, *l = lo + r * kk;
                float f = 0.0f;
                for (size_t b = 0; b < blocks; b++) {
                    int32_t sh = 0, sl = 0;
                    for (size_t i = b * Q8_BLOCK; i < (b + 1) * Q8_BLOCK; i++) {
                        sh += (int32_t)h[i] * q[i];
                        sl += (int32_t)l[i] * q[i];
                    }
                    const int32_t t = sh * 256 + sl;
                    f = fmaf(scales[(p * blocks + b) * PANEL + o % PANEL], (float)t, f);
                }
                sums[j] = ex[r] == OR_EXP_NONFINITE ? NAN : ldexpf(f, -ex[r]);
            }
            or_store(1, sums, c + r * ldc + o0, cols, bias ? bias + o0 : NULL, act, scale, accumulate);
        }
    }
    free(hi);
    free(lo);
    free(ex);
    free(qt);
    return OR_OK;
}

/* ---- the TDT decoder ----------------------------------------------------------------------- */

/* c = a w^T + bias for m rows by the fast path's integer oracle (int8 or Q8_0 weights). */
static void tdt_linear(int p, const float *a, size_t m, size_t k, const uint8_t *values, const float *scales,
                       size_t n, const float *bias, float *c) {
    if (p == P_Q8_0)
        or_matmul_fast_q8(a, m * k, k, m, values, scales, n, k, c, m * n, n, bias, n, ACT_NONE, 1.0f, 0);
    else
        or_matmul_fast(a, m * k, k, m, values, scales, n, k, c, m * n, n, bias, n, ACT_NONE, 1.0f, 0);
}

static float tdt_sigmoid(float x) { return 1.0f / (1.0f + expf(-x)); }

/* The first largest of n values (a NaN is never larger). */
static size_t tdt_argmax(const float *v, size_t n) {
    size_t best = 0;
    for (size_t i = 0; i < n; i++)
        if (v[i] > v[best]) best = i;
    return best;
}

/* predict_rows: states are rows x layers x [h, c] (h floats each), preds rows x h. lstm_v / lstm_s /
 * lstm_b hold `layers` matrices 4h x 2h in the panel layout, their scales and biases. */
void or_tdt_predict(int p, size_t h, size_t layers, const float *emb, const uint8_t *const *lstm_v,
                    const float *const *lstm_s, const float *const *lstm_b, const uint8_t *proj_v,
                    const float *proj_s, const float *proj_b, const int32_t *tokens, size_t rows, float *states,
                    float *preds) {
    const size_t width = layers * 2 * h;
    float *input = calloc(rows * 2 * h, sizeof(float)), *gates = calloc(rows * 4 * h, sizeof(float));
    float *last = calloc(rows * h, sizeof(float));
    for (size_t r = 0; r < rows; r++) memcpy(input + r * 2 * h, emb + (size_t)tokens[r] * h, h * sizeof(float));
    for (size_t l = 0; l < layers; l++) {
        for (size_t r = 0; r < rows; r++)
            memcpy(input + r * 2 * h + h, states + r * width + l * 2 * h, h * sizeof(float));
        tdt_linear(p, input, rows, 2 * h, lstm_v[l], lstm_s[l], 4 * h, lstm_b[l], gates);
        for (size_t r = 0; r < rows; r++) {
            float *hs = states + r * width + l * 2 * h, *cs = hs + h;
            const float *g = gates + r * 4 * h;
            for (size_t j = 0; j < h; j++) {
                const float i = tdt_sigmoid(g[j]), f = tdt_sigmoid(g[h + j]), gg = tanhf(g[2 * h + j]),
                            o = tdt_sigmoid(g[3 * h + j]);
                cs[j] = f * cs[j] + i * gg;
                hs[j] = o * tanhf(cs[j]);
            }
            memcpy(input + r * 2 * h, hs, h * sizeof(float));
        }
    }
    for (size_t r = 0; r < rows; r++) memcpy(last + r * h, input + r * 2 * h, h * sizeof(float));
    tdt_linear(p, last, rows, h, proj_v, proj_s, h, proj_b, preds);
    free(input);
    free(gates);
    free(last);
}

/* decode_inner from frame *t with *on_frame tokens on it: tokens get (id, frame, duration) triples,
 * at most cap of them; returns the number emitted. enc holds frames rows of h floats (stride lde);
 * the joint is (vocab + ndur) x h; the blank is vocab - 1. */
size_t or_tdt_decode(int p, size_t h, size_t layers, size_t vocab, const int32_t *durations, size_t ndur,
                     size_t max_symbols, const uint8_t *joint_v, const float *joint_s, const float *joint_b,
                     const float *emb, const uint8_t *const *lstm_v, const float *const *lstm_s,
                     const float *const *lstm_b, const uint8_t *proj_v, const float *proj_s, const float *proj_b,
                     const float *enc, size_t lde, size_t frames, float *state, float *pred, size_t *t_io,
                     size_t *on_frame_io, int32_t *tokens, size_t cap) {
    const size_t outputs = vocab + ndur, blank = vocab - 1;
    float *z = calloc(h, sizeof(float)), *logits = calloc(outputs, sizeof(float));
    size_t t = *t_io, on_frame = *on_frame_io, count = 0;
    while (t < frames) {
        for (size_t i = 0; i < h; i++) z[i] = fmaxf(enc[t * lde + i] + pred[i], 0.0f);
        tdt_linear(p, z, 1, h, joint_v, joint_s, outputs, joint_b, logits);
        const size_t token = tdt_argmax(logits, vocab);
        const size_t duration = (size_t)durations[tdt_argmax(logits + vocab, ndur)];
        if (token == blank) {
            t += duration > 1 ? duration : 1;
            on_frame = 0;
            continue;
        }
        if (count < cap) {
            tokens[3 * count] = (int32_t)token;
            tokens[3 * count + 1] = (int32_t)t;
            tokens[3 * count + 2] = (int32_t)duration;
        }
        count++;
        const int32_t tok = (int32_t)token;
        or_tdt_predict(p, h, layers, emb, lstm_v, lstm_s, lstm_b, proj_v, proj_s, proj_b, &tok, 1, state, pred);
        if (duration > 0) {
            t += duration;
            on_frame = 0;
        } else {
            on_frame += 1;
            if (on_frame >= max_symbols) {
                t += 1;
                on_frame = 0;
            }
        }
    }
    *t_io = t;
    *on_frame_io = on_frame;
    free(z);
    free(logits);
    return count;
}
