// telmo's panel layout on the host (src/quant.rs): sizes, the int8 / Q8_0 quantisers and
// encode / decode of row-major f32 rows. No device is needed; the uploader takes the bytes this
// writes, as it takes the values of a TELMOPAK pack.
#include <cmath>
#include <cstring>
#include <vector>

#include "../../include/telmo_hip.h"

namespace {

constexpr size_t PANEL = 16, Q8_BLOCK = 32;

size_t div_ceil(size_t a, size_t b) { return (a + b - 1) / b; }

size_t value_bytes(uint32_t p) {
    switch (p) {
    case TG_F32: return 4;
    case TG_F16: case TG_BF16: return 2;
    case TG_INT8: case TG_Q8_0: return 1;
    default: return 0;
    }
}

uint32_t bits_of(float f) {
    uint32_t b;
    std::memcpy(&b, &f, 4);
    return b;
}

float float_of(uint32_t b) {
    float f;
    std::memcpy(&f, &b, 4);
    return f;
}

// f32 to IEEE half, rounding to nearest even (src/quant.rs:91-127), worked out on the value
// rather than its bits: a finite |x| with binary exponent E (x = f 2^E, 0.5 <= f < 1) sits on the
// half grid of step 2^(E - 11), or 2^-24 below the normal range; rint (nearest, ties to even in the
// default rounding mode) of |x| / step is exact in double, and the count m of steps gives the bits
// directly: subnormals are m itself, normals (E + 14) << 10 plus m - 1024 (the biased exponent is
// E + 14 = q + 25), where m = 2048 (a carry) lands on the next exponent's first value, and up to
// infinity. Infinity keeps its sign; a
// NaN keeps the top ten bits of its payload with the quiet bit set, as the reference writes it.
uint16_t to_half(float x) {
    const uint32_t b = bits_of(x);
    const uint16_t sign = (uint16_t)((b >> 16) & 0x8000);
    if (std::isnan(x)) return sign | 0x7e00 | (uint16_t)((b & 0x7fffff) >> 13);
    if (std::isinf(x)) return sign | 0x7c00;
    const double v = std::fabs((double)x);
    if (v == 0.0) return sign;
    int E;
    (void)std::frexp(v, &E);
    const int q = E - 11 > -24 ? E - 11 : -24;  // the grid step's exponent
    const double m = std::nearbyint(std::ldexp(v, -q));
    if (q == -24 && m < 1024.0) return sign | (uint16_t)m;  // a subnormal (or zero) half
    const double bits = (double)((q + 25) << 10) + (m - 1024.0);
    return bits >= 0x7c00 ? (uint16_t)(sign | 0x7c00) : (uint16_t)(sign | (uint16_t)bits);
}

// IEEE half to f32, exactly: m 2^-24 below the normal range, (1024 + m) 2^(e - 25) above it; a
// NaN becomes the quiet f32 NaN with the payload shifted into place.
float from_half(uint16_t h) {
    const uint32_t sign = (uint32_t)(h & 0x8000) << 16, e = (h >> 10) & 0x1f, m = h & 0x3ff;
    if (e == 0x1f) return float_of(sign | 0x7f800000u | (m ? 0x400000u | (m << 13) : 0u));
    const double mag = e == 0 ? std::ldexp((double)m, -24) : std::ldexp((double)(1024 + m), (int)e - 25);
    const float v = (float)mag;
    return sign ? -v : v;
}

// f32 to bfloat16, nearest even (src/quant.rs:149-156): as for the half, the value is rounded to
// the grid of 8 significant bits (step 2^(E - 8), or 2^-133 below the normal range) in double, and
// the result, an f32 (infinity when it rounds past the largest one), keeps its top 16 bits. A NaN
// gets the quiet bit.
uint16_t to_bf16(float x) {
    const uint32_t b = bits_of(x);
    if (std::isnan(x)) return (uint16_t)((b >> 16) | 0x40);
    const double v = (double)x;
    if (v == 0.0 || std::isinf(x)) return (uint16_t)(b >> 16);
    int E;
    (void)std::frexp(v, &E);
    const int q = E - 8 > -133 ? E - 8 : -133;
    const double r = std::ldexp(std::nearbyint(std::ldexp(v, -q)), q);
    const float f = std::fabs(r) >= 0x1p128 ? (r > 0 ? INFINITY : -INFINITY) : (float)r;
    return (uint16_t)(bits_of(f) >> 16);
}

// Rust's saturating `as i8` of an already rounded value.
int8_t saturate_i8(float v) {
    if (std::isnan(v)) return 0;
    if (v >= 127.0f) return 127;
    if (v <= -128.0f) return -128;
    return (int8_t)v;
}

float amax(const float *x, size_t len) {
    float m = 0.0f;
    for (size_t i = 0; i < len; i++) m = std::fmax(m, std::fabs(x[i]));
    return m;
}

// src/quant.rs:189-198: d = amax / 127 unrounded, q = clamp(round(v / d), -127, 127).
float quantize_int8(const float *x, size_t len, int8_t *q) {
    const float d = amax(x, len) / 127.0f, id = d != 0.0f ? 1.0f / d : 0.0f;
    for (size_t i = 0; i < len; i++) {
        float v = std::round(x[i] * id);
        if (!std::isnan(v)) v = std::fmin(std::fmax(v, -127.0f), 127.0f);
        q[i] = saturate_i8(v);
    }
    return d;
}

// src/quant.rs:176-187: per block of 32, scale stored f16-rounded, values from the unrounded one.
float quantize_q8_0(const float *x, size_t len, int8_t *q) {
    const float d = amax(x, len) / 127.0f, id = d != 0.0f ? 1.0f / d : 0.0f;
    for (size_t i = 0; i < len; i++) q[i] = saturate_i8(std::round(x[i] * id));
    return from_half(to_half(d));
}

}  // namespace

extern "C" {

size_t tg_panel_bytes(uint32_t precision, size_t n, size_t k) {
    return div_ceil(n, PANEL) * k * PANEL * value_bytes(precision);
}

size_t tg_scale_count(uint32_t precision, size_t n, size_t k) {
    const size_t panels = div_ceil(n, PANEL);
    if (precision == TG_INT8) return panels * PANEL;
    if (precision == TG_Q8_0) return panels * div_ceil(k, Q8_BLOCK) * PANEL;
    return 0;
}

int tg_fits(uint32_t precision, size_t k) { return precision != TG_Q8_0 || k % Q8_BLOCK == 0; }

void tg_random(float *out, size_t len, uint64_t seed) {
    if (!out) return;
    uint64_t s = seed * 0x9E3779B97F4A7C15ull | 1u;
    for (size_t i = 0; i < len; i++) {
        s ^= s << 13;
        s ^= s >> 7;
        s ^= s << 17;
        out[i] = (float)(s >> 40) * (1.0f / 16777216.0f) * 2.0f - 1.0f;
    }
}

int tg_encode(const float *w, size_t n, size_t k, uint32_t precision, uint8_t *values, size_t values_len,
              float *scales, size_t n_scales) {
    if (value_bytes(precision) == 0 || !tg_fits(precision, k)) return TG_ERR_ARG;
    if (values_len != tg_panel_bytes(precision, n, k) || n_scales != tg_scale_count(precision, n, k))
        return TG_ERR_ARG;
    if ((n * k && !w) || (values_len && !values) || (n_scales && !scales)) return TG_ERR_NULL;
    const size_t vb = value_bytes(precision), blocks = div_ceil(k, Q8_BLOCK);
    if (values_len) std::memset(values, 0, values_len);
    for (size_t i = 0; i < n_scales; i++) scales[i] = 0.0f;
    std::vector<int8_t> q(k ? k : 1);
    for (size_t o = 0; o < n; o++) {
        const size_t p = o / PANEL, j = o % PANEL;
        const float *row = w + o * k;
        if (precision == TG_INT8) scales[p * PANEL + j] = quantize_int8(row, k, q.data());
        if (precision == TG_Q8_0)
            for (size_t b = 0; b < blocks; b++)
                scales[(p * blocks + b) * PANEL + j] = quantize_q8_0(row + b * Q8_BLOCK, Q8_BLOCK, q.data() + b * Q8_BLOCK);
        uint8_t *panel = values + p * k * PANEL * vb;
        for (size_t i = 0; i < k; i++) {
            uint8_t *at = panel + (i * PANEL + j) * vb;
            switch (precision) {
            case TG_F32: std::memcpy(at, &row[i], 4); break;
            case TG_F16: { const uint16_t h = to_half(row[i]); std::memcpy(at, &h, 2); break; }
            case TG_BF16: { const uint16_t h = to_bf16(row[i]); std::memcpy(at, &h, 2); break; }
            default: at[0] = (uint8_t)q[i]; break;
            }
        }
    }
    return TG_OK;
}

int tg_decode(const uint8_t *values, size_t values_len, const float *scales, size_t n_scales, uint32_t precision,
              size_t n, size_t k, float *out) {
    if (value_bytes(precision) == 0 || !tg_fits(precision, k)) return TG_ERR_ARG;
    if (values_len != tg_panel_bytes(precision, n, k) || n_scales != tg_scale_count(precision, n, k))
        return TG_ERR_ARG;
    if ((values_len && !values) || (n_scales && !scales) || (n * k && !out)) return TG_ERR_NULL;
    const size_t vb = value_bytes(precision), blocks = div_ceil(k, Q8_BLOCK);
    for (size_t o = 0; o < n; o++) {
        const size_t p = o / PANEL, j = o % PANEL;
        for (size_t i = 0; i < k; i++) {
            const uint8_t *b = values + ((p * k + i) * PANEL + j) * vb;
            float v;
            switch (precision) {
            case TG_F32: std::memcpy(&v, b, 4); break;
            case TG_F16: { uint16_t h; std::memcpy(&h, b, 2); v = from_half(h); break; }
            case TG_BF16: { uint16_t h; std::memcpy(&h, b, 2); v = float_of((uint32_t)h << 16); break; }
            case TG_INT8: v = (float)(int8_t)b[0] * scales[p * PANEL + j]; break;
            default: v = (float)(int8_t)b[0] * scales[(p * blocks + i / Q8_BLOCK) * PANEL + j]; break;
            }
            out[o * k + i] = v;
        }
    }
    return TG_OK;
}

}  // extern "C"
