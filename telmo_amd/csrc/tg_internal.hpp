// Shared definitions of the MI355X int8-weight matrix product: device layouts, the dequantisation
// and epilogue arithmetic every kernel shares, and the launchers each kernel file provides.
//
// Everything here is compiled with -ffp-contract=off: a product followed by a sum is two
// roundings unless written as __builtin_fmaf, so results match the reference bit for bit where
// the arithmetic is the same.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <cstddef>

namespace tg {

// Outputs per weight panel (src/kernels/mod.rs:29) and inputs per Q8_0 block (src/quant.rs:17).
constexpr int PANEL = 16;
constexpr int Q8_BLOCK = 32;
// Inputs per MFMA k-block of the device layout.
constexpr int KBLK = 64;
// Largest |v| of a 15-bit activation split into two signed int8 digits v = 256 hi + lo.
constexpr float DIGIT_MAX = 32639.0f;
// Exponent marking a row that holds a NaN or an infinity: its sums are NaN.
constexpr int32_t EXP_NONFINITE = INT32_MIN;
// Longest k the integer path takes: |sum of hi * q| < 2^14 * k stays below 2^31.
constexpr size_t MAX_K_INT = 65536;

enum Precision : uint32_t { F32 = 0, F16 = 1, BF16 = 2, INT8 = 3, Q8_0 = 4 };
enum Act : uint32_t { ACT_NONE = 0, ACT_RELU = 1, ACT_SILU = 2 };

__host__ __device__ inline size_t div_ceil(size_t a, size_t b) { return (a + b - 1) / b; }

// Device copy of a weight matrix.
//   f32 / f16 / bf16: telmo's panel layout unchanged: value (o, i) at ((o/16 * k + i) * 16 + o%16).
//   int8 / Q8_0: the "MFMA layout": per panel p and k-block t of 64 inputs, 1024 bytes in lane
//     order, lane l = 16 g + j holding the 16 inputs 64 t + 16 g + [0, 16) of output 16 p + j,
//     at p * panel_stride + t * blk_stride. Inputs past k are zero. One 16-byte load per lane is
//     then the operand of an i8 MFMA (16x16x64) for both the GEMM and the dot4 GEMV.
//   scales: unchanged ([panels * 16] for int8, [panels * blocks * 16] for Q8_0).
struct DeviceWeights {
    size_t n, k;
    uint32_t precision;
    size_t panels;   // ceil(n / 16)
    size_t kb;       // ceil(k / 64): k-blocks of the MFMA layout
    uint8_t *values; // device
    float *scales;   // device, or null
    size_t values_bytes, n_scales;
    size_t panel_stride, blk_stride;  // bytes between panels and between k-blocks (MFMA layout)
};

// Quantised activations ("QA"), fragment-major: for each block of 16 rows R, k-block t and digit d
// (hi = 0, lo = 1), 1 KB at ((R * kb + t) * 2 + d) * 1024 in MFMA lane order: lane g * 16 + r holds
// the 16 digits of inputs 64 t + 16 g + [0, 16) of row 16 R + r. Digits of inputs past k are zero;
// rows past m in the last block are never read into a stored result.
inline size_t qa_bytes(size_t m, size_t k) { return div_ceil(m, 16) * div_ceil(k, KBLK) * 2048; }
__host__ __device__ inline size_t qa_offset(size_t row, size_t t, int d, size_t kb) {
    return (((row / 16) * kb + t) * 2 + d) * 1024 + (row % 16) * 16;
}

// ---------------------------------------------------------------------------- device arithmetic

// e^x in the steps of the reference's SIMD exp (src/kernels/avx512.rs:279-304): clamp, n =
// rint(x log2 e), a two-part reduction, a degree-6 fused polynomial, times 2^n from the exponent
// bits. x86 max/min return their second operand when either is NaN; fmaxf/fminf of (x, c) return
// c for a NaN x as well.
__device__ __forceinline__ float exp_simd(float x) {
    x = fminf(fmaxf(x, -87.33654f), 88.37626f);
    float n = __builtin_rintf(x * 1.44269504088896340736f);
    float r = __builtin_fmaf(-n, 0.6933594f, x);
    r = __builtin_fmaf(-n, -2.1219444e-4f, r);
    float p = 1.9875691e-4f;
    p = __builtin_fmaf(p, r, 1.3982e-3f);
    p = __builtin_fmaf(p, r, 8.333452e-3f);
    p = __builtin_fmaf(p, r, 4.1665796e-2f);
    p = __builtin_fmaf(p, r, 0.16666665f);
    p = __builtin_fmaf(p, r, 0.5f);
    p = __builtin_fmaf(p, r * r, r);
    p = p + 1.0f;
    float pow2n = __uint_as_float((uint32_t)((int32_t)n + 127) << 23);
    return p * pow2n;
}

// The epilogue of one output (src/kernels/avx512.rs:313-343): bias, activation, scale, then
// accumulate onto the old value. ReLU is x86 MAXPS(v, 0): v if v > 0, else 0. The bias value b and
// the old output are used only when has_bias / accumulate are set.
__device__ __forceinline__ float epilogue_vals(float v, bool has_bias, float b, uint32_t act, float scale,
                                               bool accumulate, float old) {
    if (has_bias) v = v + b;
    if (act == ACT_RELU) {
        v = v > 0.0f ? v : 0.0f;
    } else if (act == ACT_SILU) {
        v = v / (1.0f + exp_simd(0.0f - v));
    }
    v = v * scale;
    if (accumulate) v = old + v;
    return v;
}

// epilogue_vals with the activation fixed at compile time (ACT <= ACT_SILU; ACT = ACT_ANY reads act)
// and the bias and accumulation taken by selects rather than branches, so that an unrolled
// epilogue over many outputs has no branch per output. The same operations in the same order.
constexpr uint32_t ACT_ANY = 3;
template <uint32_t ACT>
__device__ __forceinline__ float epilogue_sel(float v, bool has_bias, float b, uint32_t act, float scale,
                                              bool accumulate, float old) {
    const float vb = v + b;
    v = has_bias ? vb : v;
    const uint32_t a = ACT == ACT_ANY ? act : ACT;
    if (a == ACT_RELU) {
        v = v > 0.0f ? v : 0.0f;
    } else if (a == ACT_SILU) {
        v = v / (1.0f + exp_simd(0.0f - v));
    }
    v = v * scale;
    const float va = old + v;
    return accumulate ? va : v;
}

__device__ __forceinline__ float epilogue(float v, const float *bias, size_t col, uint32_t act, float scale,
                                          bool accumulate, const float *cptr) {
    return epilogue_vals(v, bias != nullptr, bias ? bias[col] : 0.0f, act, scale, accumulate,
                         accumulate ? *cptr : 0.0f);
}

// The f32 sum of the integer path: S = 256 acc_hi + acc_lo exactly, one rounding to f32, times
// the output's scale, then the exact power-of-two unscaling of the row. "+ 0" makes an exact
// zero +0 whatever the scale's sign, as the reference's sums start at +0.
__device__ __forceinline__ float dequant(int32_t acc_hi, int32_t acc_lo, int32_t e, float scale) {
    if (e == EXP_NONFINITE) return __builtin_nanf("");
    // 256 hi + lo is exact in f64 (|S| < 2^39), so the conversion to f32 is the one rounding of S.
    const double s = __builtin_fma((double)acc_hi, 256.0, (double)acc_lo);
    const float u = (float)s * scale + 0.0f;
    return __builtin_ldexpf(u, -e);
}

// dequant for sums with |acc_hi| < 2^22 (dequant_fits): S = 256 hi + lo then fits an int32 (|lo| <
// 2^30 for k <= 65536), and its conversion to f32 is the same single rounding, with no f64
// arithmetic. GEMM epilogues take this path when every sum of the wavefront fits (a wave-uniform
// vote), which is all but certain for the sizes here: |hi| <= 127 * 127 * k.
__device__ __forceinline__ bool dequant_fits(int32_t acc_hi) { return (uint32_t)(acc_hi + (1 << 22)) < (1u << 23); }
__device__ __forceinline__ float dequant_i32(int32_t acc_hi, int32_t acc_lo, int32_t e, float scale) {
    if (e == EXP_NONFINITE) return __builtin_nanf("");
    const float u = (float)(acc_hi * 256 + acc_lo) * scale + 0.0f;
    return __builtin_ldexpf(u, -e);
}

// The row exponent e: the largest with max|a| * 2^e <= DIGIT_MAX, from the bits of amax
// (positive, finite) so that subnormals are handled exactly.
__device__ __forceinline__ int32_t row_exponent_of(float amax) {
    if (amax == 0.0f) return 0;
    uint32_t b = __float_as_uint(amax);
    int32_t be = (int32_t)(b >> 23);
    int32_t E = be == 0 ? (31 - __builtin_clz(b & 0x7fffff)) - 148 : be - 126;
    int32_t e = 15 - E;
    if (__builtin_ldexpf(amax, e) > DIGIT_MAX) e -= 1;
    return e;
}

// The two digits of one activation under exponent e: v = rint(a 2^e) = 256 hi + lo.
__device__ __forceinline__ void digits_of(float a, int32_t e, int8_t &hi, int8_t &lo) {
    int32_t v = e == EXP_NONFINITE ? 0 : (int32_t)__builtin_rintf(__builtin_ldexpf(a, e));
    int32_t l = ((v + 128) & 255) - 128;
    hi = (int8_t)((v - l) >> 8);
    lo = (int8_t)l;
}

// The digits of four consecutive inputs packed as (hi dword, lo dword): the same digits as
// digits_of, since lo = v mod 256 (as a signed byte) is the low byte of v, and
// hi = (v - lo) / 256 = (v + 128) >> 8 is byte 1 of v + 128 (|v| <= 32639).
__device__ __forceinline__ void digits4(float x0, float x1, float x2, float x3, int32_t e, uint32_t &hi,
                                        uint32_t &lo) {
    const bool ok = e != EXP_NONFINITE;
    const uint32_t v0 = ok ? (uint32_t)(int32_t)__builtin_rintf(__builtin_ldexpf(x0, e)) : 0u;
    const uint32_t v1 = ok ? (uint32_t)(int32_t)__builtin_rintf(__builtin_ldexpf(x1, e)) : 0u;
    const uint32_t v2 = ok ? (uint32_t)(int32_t)__builtin_rintf(__builtin_ldexpf(x2, e)) : 0u;
    const uint32_t v3 = ok ? (uint32_t)(int32_t)__builtin_rintf(__builtin_ldexpf(x3, e)) : 0u;
    // v_perm_b32(s0, s1, sel): byte i of the result is byte sel_i of s0:s1 (0-3 from s1, 4-7 from
    // s0), 0x0c gives zero.
    const uint32_t lo01 = __builtin_amdgcn_perm(v1, v0, 0x0c0c0400u);
    const uint32_t lo23 = __builtin_amdgcn_perm(v3, v2, 0x0c0c0400u);
    lo = __builtin_amdgcn_perm(lo23, lo01, 0x05040100u);
    const uint32_t hi01 = __builtin_amdgcn_perm(v1 + 128u, v0 + 128u, 0x0c0c0501u);
    const uint32_t hi23 = __builtin_amdgcn_perm(v3 + 128u, v2 + 128u, 0x0c0c0501u);
    hi = __builtin_amdgcn_perm(hi23, hi01, 0x05040100u);
}

// The guard's two sums over one input (RowGuard): v^2 and d^2 of x = a 2^e, v = rint(x),
// d = rint(256 (x - v)). x - v is exact (|x - v| <= 1/2 and both are f32 near each other), and so is
// the scaling by 256, so d is an integer in [-128, 128].
__device__ __forceinline__ void guard_terms(float a, int32_t e, double &vv, int32_t &dd) {
    const float x = __builtin_ldexpf(a, e);
    const float v = __builtin_rintf(x);
    const int32_t d = (int32_t)__builtin_rintf((x - v) * 256.0f);
    vv += (double)v * (double)v;
    dd += d * d;
}
// The flag of a row from its two sums (RowGuard).
__device__ __forceinline__ int32_t guard_flag(int32_t e, double vv, int32_t dd) {
    return e != EXP_NONFINITE && 256.0 * (double)dd > vv ? 1 : 0;
}

// ---------------------------------------------------------------------------- launchers

struct EpiArgs {
    const float *bias;  // device or null
    uint32_t act;
    float scale;
    int accumulate;
};

// Re-lays int8 / Q8_0 panel values (device, telmo's layout) into w's MFMA layout.
hipError_t launch_repack_i8(const uint8_t *src, const DeviceWeights &w, hipStream_t s);

// The map the row quantiser applies to each input before quantising it: the activation, then the
// scale (the order of epilogue_vals without bias and accumulation). The identity by default.
struct RowAct {
    uint32_t act = ACT_NONE;
    float scale = 1.0f;
    __device__ __forceinline__ float operator()(float v) const {
        return epilogue_vals(v, false, 0.0f, act, scale, false, 0.0f);
    }
};

// The accuracy guard of a product's quantised rows. Under its exponent e a row's inputs become
// x = a 2^e, v = rint(x) (the two digits' value) and d = rint(256 (x - v)) (the next eight bits);
// the row is flagged when 256 sum d^2 > sum v^2, that is when the relative size of what the two
// digits drop, rho = |x - v| / |x| ~ sqrt(sum d^2 / 65536) / sqrt(sum v^2), exceeds 2^-12. Both
// sums are exact integers (sum v^2 < 2^53 in f64, sum d^2 < 2^31), so the flag does not depend on
// the order of the sums. The fast path's row-normwise error measures 0.7 to 2.1 rho, so an unflagged
// row stays within about 5e-4 of the reference; N(0, 1) rows have rho near 3.5e-5. Rows with a NaN
// or an infinity are not flagged (their outputs are NaN, as without the guard).
struct RowGuard {
    int32_t *flags = nullptr;  // per row, 1 when flagged; null: no guard
    const float *c = nullptr;  // the product's output rows before it runs, kept for flagged rows
    size_t ldc = 0;            // when the epilogue accumulates: c[r ldc + j] -> save[r n + j], j < n
    size_t n = 0;
    float *save = nullptr;  // null when the epilogue does not accumulate
};

// Per-row digits and exponents of f(a[m][lda]) (k inputs) into qa (fragment-major) / exps, and
// the guard's flags (and saved output rows) when g.flags is set.
hipError_t launch_quantize_rows(const float *a, size_t lda, size_t m, size_t k, uint8_t *qa, int32_t *exps,
                                hipStream_t s, RowAct f = RowAct{}, const RowGuard &g = RowGuard{});

// out[r][j] = x[r][j] * sigmoid(x[r][half + j]).
hipError_t launch_glu(const float *x, size_t ldx, size_t m, size_t half, float *out, size_t ldo, hipStream_t s);
// softmax of m rows of n values in place (the reference's AVX-512 order).
hipError_t launch_softmax(float *x, size_t ldx, size_t m, size_t n, hipStream_t s);
// out[b (frames / 2) + r] = (x[b frames + 2 r] + x[b frames + 2 r + 1]) / 2 over n values per row.
hipError_t launch_average_pairs(const float *x, size_t ldx, size_t frames, size_t batch, size_t n, float *out,
                                size_t ldo, hipStream_t s);

// LayerNorm of m rows of n values (the reference's AVX-512 summation order).
hipError_t launch_dwconv1d(const float *x, size_t ldx, size_t frames, size_t batch, size_t channels, const float *w,
                           size_t kernel, const float *bias, size_t t0, size_t stride, size_t rows, int silu,
                           float *out, size_t ldo, hipStream_t s);
// The depthwise convolution of whole sequences (t0 = 0, stride 1, rows = frames) with its output
// rows quantised (qa, exps as launch_quantize_rows writes them for k = channels); out may be null.
// channels <= 2048 and 1 <= kernel <= 32 (dwconv_quant_fits).
bool dwconv_quant_fits(size_t channels, size_t kernel);
hipError_t launch_dwconv_quant(const float *x, size_t ldx, size_t frames, size_t batch, size_t channels,
                               const float *w, size_t kernel, const float *bias, int silu, float *out, size_t ldo,
                               uint8_t *qa, int32_t *exps, hipStream_t s);
hipError_t launch_layer_norm(const float *x, size_t ldx, size_t m, size_t n, const float *gamma, const float *beta,
                             float eps, float *out, size_t ldo, hipStream_t s);
// LayerNorm then the two-digit quantisation of its outputs (qa, exps); out (may be null, may be x)
// also gets the f32 outputs.
hipError_t launch_layer_norm_quant(const float *x, size_t ldx, size_t m, size_t n, const float *gamma,
                                   const float *beta, float eps, float *out, size_t ldo, uint8_t *qa, int32_t *exps,
                                   hipStream_t s);
// A layer boundary's two LayerNorms: out = LayerNorm(x; gamma, beta, eps) (out may be x), then the
// digits (qa, exps) of LayerNorm(out; gamma2, beta2, eps2), bit-identical to launch_layer_norm and
// then launch_layer_norm_quant of its outputs; one launch where the row kernel takes the rows.
hipError_t launch_layer_norm_pair(const float *x, size_t ldx, size_t m, size_t n, const float *gamma,
                                  const float *beta, float eps, float *out, size_t ldo, const float *gamma2,
                                  const float *beta2, float eps2, uint8_t *qa, int32_t *exps, hipStream_t s);

// The two-digit int8 MFMA GEMM over quantised rows (int8 and Q8_0 weights).
hipError_t launch_gemm_i8(const uint8_t *qa, const int32_t *exps, size_t m, const DeviceWeights &w, float *c,
                          size_t ldc, const EpiArgs &epi, hipStream_t s);
// The same GEMM (int8 or Q8_0 weights) with the GLU of its two output halves in the epilogue:
// out[r, j] = g[r, j] / (1 + exp(0 - g[r, n / 2 + j])), g the product through epi (no
// accumulation). n must be a multiple of 64 (gemm_glu_fits); out is m x n / 2, row stride ldo.
bool gemm_glu_fits(size_t n);
hipError_t launch_gemm_i8_glu(const uint8_t *qa, const int32_t *exps, size_t m, const DeviceWeights &w, float *out,
                              size_t ldo, const EpiArgs &epi, hipStream_t s);

// The FFN hidden rows' quantisation in two launches, bit-identical to the product into f32 rows
// followed by the row quantiser: the GEMM writes its outputs y = epi(sum) into h (row stride ldh)
// and, per row and workgroup column, the largest |y| as unsigned bits (all ones for a NaN or an
// infinity) into tmax[row * strips + column], strips = gemm_qout_strips(m, w); then the streaming
// quantiser turns h into the digit layout and row exponents, each row's exponent from its maxima.
// int8 weights, fast mode, no accumulation (epi.accumulate must be 0); m >= 1.
int gemm_qout_strips(size_t m, const DeviceWeights &w);
hipError_t launch_gemm_i8_qout(const uint8_t *qa, const int32_t *exps, size_t m, const DeviceWeights &w,
                               const EpiArgs &epi, float *h, size_t ldh, uint32_t *tmax, hipStream_t s);
// h: ldh a multiple of 64 and at least n rounded up to 64, 16-byte aligned.
hipError_t launch_quantize_known(const float *h, size_t ldh, size_t m, size_t n, const uint32_t *tmax, int strips,
                                 uint8_t *qa, int32_t *exps, hipStream_t s);

// The decode GEMVs (quantise the rows themselves; int8 and Q8_0 weights): the MFMA GEMV for
// m <= 16 rows of k <= 1984 inputs (m * ceil(k / 256) <= 64; 16-byte aligned rows, k % 4 == 0),
// else, for int8 only, the dot4 GEMV for m <= 8 rows whose digits fit 64 KB of LDS.
constexpr size_t GEMV_MAX_ROWS = 16;
bool gemv_fits(size_t m, size_t k, const float *a, size_t lda, uint32_t precision);
hipError_t launch_gemv_i8(const float *a, size_t lda, size_t m, const DeviceWeights &w, float *c, size_t ldc,
                          const EpiArgs &epi, hipStream_t s);

// The exact kernel: the reference's fused sums in input order, any precision.
hipError_t launch_exact(const float *a, size_t lda, size_t m, const DeviceWeights &w, float *c, size_t ldc,
                        const EpiArgs &epi, hipStream_t s);
// The guard's fix-up: the exact kernel's outputs for the rows flagged in flags[m] only, the epilogue
// accumulating onto save[r n + j] (the rows as they were before the product) when it accumulates.
hipError_t launch_exact_rows(const float *a, size_t lda, size_t m, const DeviceWeights &w, float *c, size_t ldc,
                             const EpiArgs &epi, const int32_t *flags, const float *save, hipStream_t s);
// A row-major f32 right-hand side [k, ldb], the exact kernel's sums (kernels_exact.hip).
hipError_t launch_rowmajor(const float *a, size_t lda, size_t m, size_t k, const float *b, size_t ldb, size_t n,
                           float *c, size_t ldc, const EpiArgs &epi, hipStream_t s);

// The greedy TDT decode (kernels_tdt.hip). The control block lives in device memory; the host
// writes it before a decode and reads it between batches of steps.
constexpr int TDT_ROWS = 16;            // most frames the joint scores per step; rows of a prediction
constexpr int TDT_MAX_LAYERS = 4;       // LSTM layers of the prediction network
constexpr int TDT_MAX_DURATIONS = 64;
// The control values the joint of a step saw, for the kernel that decides the step.
struct TdtSnap {
    int32_t valid, t, rows, on_frame, ntok, active, cur;
};
struct TdtCtl {
    int32_t t, on_frame, ntok;  // the frame, tokens on it so far, tokens emitted
    int32_t active;             // a token went to the prediction network this step
    int32_t done;               // the frames are used up and no prediction waits
    int32_t cur;                // the state buffer holding the current LSTM state (0: the caller's)
    int32_t rows;               // frames the next joint scores (1 .. TDT_ROWS)
    TdtSnap snap;
    // The resident decode's position: steps made and predictions run (the tags of its hand-over
    // words), and whether a wait passed its deadline.
    uint32_t step, preds;
    int32_t err;
};
struct TdtTokens {
    int32_t tok[TDT_ROWS];
};
// lstm[] and lstm_b[] are the interleaved copies (output 4 u + q is gate q of unit u).
struct TdtNet {
    size_t h, vocab, ndur, layers, blank, max_symbols;
    const DeviceWeights *joint, *lstm[TDT_MAX_LAYERS], *proj;
    const float *joint_b, *lstm_b[TDT_MAX_LAYERS], *proj_b, *emb;  // device
    const int32_t *durations;                                       // device, ndur
};
size_t tdt_max_rows(const DeviceWeights &lstm);
size_t tdt_partials_bytes();
size_t tdt_extras_bytes();
hipError_t launch_tdt_interleave(const DeviceWeights &src, const float *bias, const DeviceWeights &dst,
                                 float *bias_dst, size_t h, hipStream_t s);
hipError_t launch_tdt_predict(TdtCtl *ctl, const TdtTokens &toks, size_t m, const TdtNet &net, float *sa, float *sb,
                              float *preds, hipStream_t s);
hipError_t launch_tdt_step(TdtCtl *ctl, const TdtNet &net, const float *enc, size_t lde, int frames, float *sa,
                           float *sb, float *pred, void *partials, float *extras, int32_t *tokens, int cap,
                           hipStream_t s);

// The resident decode: one cooperative launch makes many steps with the network's matrices held in
// LDS, the workgroups handing each other values through tagged words.
constexpr size_t TDT_MAX_H = 992;
struct TdtPlan {
    int grid = 0;              // workgroups
    int JP = 0, GJ = 0;        // joint panels per workgroup, workgroups holding them
    int LP = 0, GL = 0;        // LSTM panels (of every layer) per workgroup, workgroups holding them
    int PP = 0, GP = 0;        // projection panels per workgroup, workgroups (the first GP)
    int qoff = 0;              // the first joint / LSTM workgroup
    size_t lds = 0;            // dynamic LDS bytes per workgroup
    bool q8 = false;           // Q8_0 matrices (their block scales in LDS too), else int8
    bool multi = false;        // the multi-stream decode fits (int8)
    size_t mlds = 0;           // its dynamic LDS bytes per workgroup
};
// Streams of one multi-stream decode launch, and what it reads and writes of each.
constexpr size_t TDT_MAX_STREAMS = 8;
struct TdtStream {
    const float *enc;
    size_t lde;
    int frames;
    float *state, *pred;
    int32_t *tokens;  // device, 3 int32 per token
    int cap;
};
// Whether the multi-stream decode takes this network (after tdt_resident_plan); sets plan.multi.
bool tdt_multi_plan(const TdtNet &net, TdtPlan &plan);
size_t tdt_multi_words(const TdtNet &net);  // 8-byte hand-over words for TDT_MAX_STREAMS streams
hipError_t launch_tdt_multi_init(const TdtNet &net, uint64_t *words, size_t m, const TdtStream *streams,
                                 const uint32_t *preds, hipStream_t s);
// Up to steps steps of m streams from their positions in ctl[0 .. m) (written by the host).
hipError_t launch_tdt_multi(TdtCtl *ctl, const TdtNet &net, const TdtPlan &plan, uint64_t *words, size_t m,
                            const TdtStream *streams, int steps, uint64_t wait_ticks, hipStream_t s);
// Whether the resident decode takes this network on the current device; fills plan and sets the
// kernel's LDS limit. Needs every matrix int8, or every one Q8_0, vocab < 65535, a cooperative
// launch and the panels in LDS.
bool tdt_resident_plan(const TdtNet &net, TdtPlan &plan);
size_t tdt_resident_words(const TdtNet &net);  // 8-byte hand-over words
// Writes the hand-over words for a decode from state and pred (tags 0; the other buffers none).
hipError_t launch_tdt_resident_init(const TdtNet &net, uint64_t *words, const float *state, const float *pred,
                                    hipStream_t s);
// Up to steps steps from the position in ctl (written by the host), which the launch updates.
hipError_t launch_tdt_resident(TdtCtl *ctl, const TdtNet &net, const TdtPlan &plan, uint64_t *words,
                               const float *enc, size_t lde, int frames, float *state, float *pred, int32_t *tokens,
                               int cap, int steps, uint64_t wait_ticks, hipStream_t s);

}  // namespace tg
