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

// Round to nearest even into IEEE half (src/quant.rs:91-127).
uint16_t to_half(float x) {
    const uint32_t b = bits_of(x);
    const uint16_t sign = (uint16_t)((b >> 16) & 0x8000);
    const int32_t exp = (int32_t)((b >> 23) & 0xff);
    const uint32_t man = b & 0x7fffff;
    if (exp == 0xff) return sign | 0x7c00 | (man ? (uint16_t)(0x200 | (man >> 13)) : 0);
    const int32_t e = exp - 112;
    if (e >= 0x1f) return sign | 0x7c00;
    if (e <= 0) {
        const uint32_t shift = (uint32_t)(126 - exp);
        if (shift > 24) return sign;
        const uint32_t full = man | 0x800000, half = 1u << (shift - 1);
        uint32_t m = full >> shift;
        const uint32_t rem = full & ((1u << shift) - 1);
        if (rem > half || (rem == half && (m & 1))) m++;
        return sign | (uint16_t)m;
    }
    uint32_t h = ((uint32_t)e << 10) | (man >> 13);
    const uint32_t rem = man & 0x1fff;
    if (rem > 0x1000 || (rem == 0x1000 && (h & 1))) h++;
    return sign | (uint16_t)h;
}

float from_half(uint16_t h) {
    const uint32_t sign = (uint32_t)(h & 0x8000) << 16, exp = (h >> 10) & 0x1f, man = h & 0x3ff;
    if (exp == 0) {
        if (man == 0) return float_of(sign);
        const float v = (float)man * (1.0f / 16777216.0f);
        return sign ? -v : v;
    }
    if (exp == 0x1f) return float_of(sign | 0x7f800000u | (man ? 0x400000u | (man << 13) : 0u));
    return float_of(sign | ((exp + 112) << 23) | (man << 13));
}

uint16_t to_bf16(float x) {
    const uint32_t b = bits_of(x);
    if (std::isnan(x)) return (uint16_t)((b >> 16) | 0x40);
    return (uint16_t)((b + 0x7fff + ((b >> 16) & 1)) >> 16);
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
