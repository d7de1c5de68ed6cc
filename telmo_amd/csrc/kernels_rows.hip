// Row kernels of the int8 path: the one-time re-layout of int8 / Q8_0 weight panels into the
// MFMA layout, the per-row two-digit quantisation of f32 activations, and the GLU and LayerNorm
// row kernels of the Conformer glue. All of them are HBM-bound: coalesced loads, no MFMA.
#include "tg_internal.hpp"

namespace tg {

// One workgroup of 64 lanes per (panel, k-block): the 64 input rows of 16 outputs (1 KB,
// contiguous in telmo's layout) go through LDS, and each lane writes the 16 inputs of one
// output that its MFMA operand needs, 16 contiguous bytes.
__global__ __launch_bounds__(64) void repack_i8_kernel(const uint8_t *__restrict__ src, uint8_t *__restrict__ dst,
                                                       size_t k, size_t kb, size_t panel_stride, size_t blk_stride) {
    __shared__ uint8_t tile[KBLK][PANEL + 4];
    const size_t blk = blockIdx.x;  // p * kb + t
    const size_t p = blk / kb, t = blk % kb;
    const int l = threadIdx.x;
    const size_t kk = t * KBLK + l;
    uint32_t v[4] = {0, 0, 0, 0};
    if (kk < k) {
        const uint32_t *s = reinterpret_cast<const uint32_t *>(src + (p * k + kk) * PANEL);
        for (int i = 0; i < 4; i++) v[i] = s[i];
    }
    for (int i = 0; i < 4; i++)
        for (int b = 0; b < 4; b++) tile[l][4 * i + b] = (uint8_t)(v[i] >> (8 * b));
    __syncthreads();
    const int g = l >> 4, j = l & 15;
    uint32_t o[4];
    for (int i = 0; i < 4; i++) {
        o[i] = 0;
        for (int b = 0; b < 4; b++) o[i] |= (uint32_t)tile[16 * g + 4 * i + b][j] << (8 * b);
    }
    uint4 out = make_uint4(o[0], o[1], o[2], o[3]);
    *reinterpret_cast<uint4 *>(dst + p * panel_stride + t * blk_stride + l * 16) = out;
}

hipError_t launch_repack_i8(const uint8_t *src, const DeviceWeights &w, hipStream_t s) {
    if (w.panels == 0 || w.kb == 0) return hipSuccess;
    hipLaunchKernelGGL(repack_i8_kernel, dim3((unsigned)(w.panels * w.kb)), dim3(64), 0, s, src, w.values, w.k, w.kb,
                       w.panel_stride, w.blk_stride);
    return hipGetLastError();
}

__device__ __forceinline__ float wave_max(float v) {
    for (int off = 32; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, 64));
    return v;
}

__device__ __forceinline__ int wave_or(int v) {
    for (int off = 32; off > 0; off >>= 1) v |= __shfl_xor(v, off, 64);
    return v;
}

// One wavefront per row: the largest magnitude (and any NaN or infinity) over the row's k
// inputs, the row exponent, then the digits of each input into the fragment-major QA.
__device__ __forceinline__ double wave_sum_f64(double v) {
    for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
    return v;
}

__device__ __forceinline__ int32_t wave_sum_i32(int32_t v) {
    for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
    return v;
}

// The guard's flag of a row (RowGuard) from the two sums of every input; with a save buffer, a
// flagged row's outputs as they are before the product are copied there by the workgroup's
// `threads` threads (thread t copies columns t, t + threads, ...).
__device__ __forceinline__ void guard_store(const RowGuard &g, size_t row, int32_t flag, int t, int threads) {
    if (t == 0) g.flags[row] = flag;
    if (flag && g.save) {
        const float *cr = g.c + row * g.ldc;
        float *sr = g.save + row * g.n;
        for (size_t j = t; j < g.n; j += threads) sr[j] = cr[j];
    }
}

__device__ __forceinline__ int32_t quantize_row_wave(const float *__restrict__ ar, size_t k, size_t kb,
                                                     uint8_t *__restrict__ qa, size_t row, int lane,
                                                     const RowAct &f, int32_t *flag = nullptr) {
    float amax = 0.0f;
    int bad = 0;
    for (size_t i = lane; i < k; i += 64) {
        float x = f(ar[i]);
        bad |= !__builtin_isfinite(x);
        amax = fmaxf(amax, fabsf(x));
    }
    amax = wave_max(amax);
    bad = wave_or(bad);
    const int32_t e = bad ? EXP_NONFINITE : row_exponent_of(amax);
    double vv = 0.0;
    int32_t dd = 0;
    for (size_t t = 0; t < kb; t++) {
        const size_t i = t * KBLK + lane;
        int8_t hi = 0, lo = 0;
        if (i < k) {
            const float x = f(ar[i]);
            digits_of(x, e, hi, lo);
            if (flag && e != EXP_NONFINITE) guard_terms(x, e, vv, dd);
        }
        const size_t at = qa_offset(row, t, 0, kb) + (lane >> 4) * 256 + (lane & 15);
        qa[at] = (uint8_t)hi;
        qa[at + 1024] = (uint8_t)lo;
    }
    if (flag) *flag = guard_flag(e, wave_sum_f64(vv), wave_sum_i32(dd));
    return e;
}

__global__ __launch_bounds__(256) void quantize_rows_kernel(const float *__restrict__ a, size_t lda, size_t m,
                                                            size_t k, size_t kb, uint8_t *__restrict__ qa,
                                                            int32_t *__restrict__ exps, RowAct f, RowGuard g) {
    const int lane = threadIdx.x & 63;
    const size_t row = (size_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= m) return;
    int32_t flag = 0;
    int32_t e = quantize_row_wave(a + row * lda, k, kb, qa, row, lane, f, g.flags ? &flag : nullptr);
    if (lane == 0) exps[row] = e;
    if (g.flags) guard_store(g, row, flag, lane, 64);
}

// One workgroup per row, the row held in registers: thread t owns the 4-input chunks t + 256 j
// (j < J), loaded as one float4 when the rows are 16-byte aligned. A block reduction gives the
// row's exponent; each thread then writes the 4 hi and 4 lo digits of each chunk as two dwords
// of the fragment-major QA. Chunks from k up to the 64-input padding are written as zeros.
//
// Rows go to workgroups so that the 16 rows of a QA row block run on one XCD: workgroup L runs on
// XCD L % 8 and takes row 16 (x bpx + i / 16) + i % 16 with x = L % 8, i = L / 8, bpx = row blocks
// per XCD. The row block's lines are then filled in one L2 instead of written back in pieces by
// several. Workgroups past the last row exit at once.
//
// MODE: 0 the identity; otherwise f = RowAct{act, scale} with act ACT_NONE (1), ACT_RELU (2) or
// ACT_SILU (3) fixed at compile time and applied to every value of a chunk with no branch (the
// chunk's values past k are zeros, which every f maps to a zero digit); a runtime act inside the
// unrolled chunks cost a branch per value.
//
// GUARD: the row's flag of the accuracy guard (RowGuard) from the inputs held in registers, after
// the digits are stored, and a flagged row's old outputs saved.
template <int J, int MODE, bool GUARD>
__global__ __launch_bounds__(256) void quantize_rows_regs_kernel(const float *__restrict__ a, size_t lda, int k,
                                                                 int kb, uint8_t *__restrict__ qa,
                                                                 int32_t *__restrict__ exps, int vec, size_t m,
                                                                 size_t bpx, float scale, RowGuard g) {
    __shared__ float s_max[4];
    __shared__ int s_bad[4];
    __shared__ double s_vv[4];
    __shared__ int32_t s_dd[4];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const size_t x = blockIdx.x % 8, i = blockIdx.x / 8;
    const size_t row = (x * bpx + i / 16) * 16 + i % 16;
    if (row >= m) return;
    const float *ar = a + row * lda;
    float4 v[J];
    float amax = 0.0f;
    int bad = 0;
#pragma unroll
    for (int j = 0; j < J; j++) {
        const int k0 = 4 * (tid + 256 * j);
        if (vec && k0 + 3 < k) {
            v[j] = *reinterpret_cast<const float4 *>(ar + k0);
        } else {
            v[j].x = k0 < k ? ar[k0] : 0.0f;
            v[j].y = k0 + 1 < k ? ar[k0 + 1] : 0.0f;
            v[j].z = k0 + 2 < k ? ar[k0 + 2] : 0.0f;
            v[j].w = k0 + 3 < k ? ar[k0 + 3] : 0.0f;
        }
        if constexpr (MODE != 0) {
            constexpr uint32_t A = MODE == 1 ? ACT_NONE : MODE == 2 ? ACT_RELU : ACT_SILU;
            v[j].x = epilogue_sel<A>(v[j].x, false, 0.0f, A, scale, false, 0.0f);
            v[j].y = epilogue_sel<A>(v[j].y, false, 0.0f, A, scale, false, 0.0f);
            v[j].z = epilogue_sel<A>(v[j].z, false, 0.0f, A, scale, false, 0.0f);
            v[j].w = epilogue_sel<A>(v[j].w, false, 0.0f, A, scale, false, 0.0f);
        }
        bad |= !__builtin_isfinite(v[j].x) | !__builtin_isfinite(v[j].y) | !__builtin_isfinite(v[j].z) |
               !__builtin_isfinite(v[j].w);
        amax = fmaxf(amax, fmaxf(fmaxf(fabsf(v[j].x), fabsf(v[j].y)), fmaxf(fabsf(v[j].z), fabsf(v[j].w))));
    }
    amax = wave_max(amax);
    bad = wave_or(bad);
    if (lane == 0) {
        s_max[wave] = amax;
        s_bad[wave] = bad;
    }
    __syncthreads();
    amax = fmaxf(fmaxf(s_max[0], s_max[1]), fmaxf(s_max[2], s_max[3]));
    bad = s_bad[0] | s_bad[1] | s_bad[2] | s_bad[3];
    const int32_t e = bad ? EXP_NONFINITE : row_exponent_of(amax);
    if (tid == 0) exps[row] = e;
    const int chunks = kb * 16;
#pragma unroll
    for (int j = 0; j < J; j++) {
        const int c = tid + 256 * j;
        if (c < chunks) {
            uint32_t hi, lo;
            digits4(v[j].x, v[j].y, v[j].z, v[j].w, e, hi, lo);
            // chunk c: k-block c / 16, 16-input group (c % 16) / 4, byte (c % 4) * 4 of its 16
            const size_t at = qa_offset(row, c >> 4, 0, kb) + ((c & 15) >> 2) * 256 + (c & 3) * 4;
            *reinterpret_cast<uint32_t *>(qa + at) = hi;
            *reinterpret_cast<uint32_t *>(qa + at + 1024) = lo;
        }
    }
    if constexpr (GUARD) {
        // Chunks past k hold zeros, whose v and d are zero.
        double vv = 0.0;
        int32_t dd = 0;
        if (e != EXP_NONFINITE) {
#pragma unroll
            for (int j = 0; j < J; j++) {
                guard_terms(v[j].x, e, vv, dd);
                guard_terms(v[j].y, e, vv, dd);
                guard_terms(v[j].z, e, vv, dd);
                guard_terms(v[j].w, e, vv, dd);
            }
        }
        vv = wave_sum_f64(vv);
        dd = wave_sum_i32(dd);
        if (lane == 0) {
            s_vv[wave] = vv;
            s_dd[wave] = dd;
        }
        __syncthreads();
        const int32_t flag = guard_flag(e, ((s_vv[0] + s_vv[1]) + s_vv[2]) + s_vv[3], s_dd[0] + s_dd[1] + s_dd[2] + s_dd[3]);
        guard_store(g, row, flag, tid, 256);
    }
}

template <int J>
void launch_regs(const float *a, size_t lda, size_t m, size_t k, size_t kb, uint8_t *qa, int32_t *exps, int vec,
                 const RowAct &f, const RowGuard &g, hipStream_t s) {
    const size_t bpx = div_ceil(div_ceil(m, (size_t)16), (size_t)8);
    const int mode = f.act == ACT_NONE ? (f.scale == 1.0f ? 0 : 1) : f.act == ACT_RELU ? 2 : 3;
    auto kernel = &quantize_rows_regs_kernel<J, 0, false>;
    if (g.flags) kernel = &quantize_rows_regs_kernel<J, 0, true>;  // the product entry points: no activation
    else if (mode == 1) kernel = &quantize_rows_regs_kernel<J, 1, false>;
    else if (mode == 2) kernel = &quantize_rows_regs_kernel<J, 2, false>;
    else if (mode == 3) kernel = &quantize_rows_regs_kernel<J, 3, false>;
    hipLaunchKernelGGL(kernel, dim3((unsigned)(8 * bpx * 16)), dim3(256), 0, s, a, lda, (int)k, (int)kb, qa, exps,
                       vec, m, bpx, f.scale, g);
}

hipError_t launch_quantize_rows(const float *a, size_t lda, size_t m, size_t k, uint8_t *qa, int32_t *exps,
                                hipStream_t s, RowAct f, const RowGuard &g) {
    if (g.flags && (f.act != ACT_NONE || f.scale != 1.0f)) return hipErrorInvalidValue;
    if (m == 0) return hipSuccess;
    const size_t kb = div_ceil(k, KBLK);
    // 16-byte loads need every row 16-byte aligned.
    const int vec = (reinterpret_cast<uintptr_t>(a) % 16 == 0) && (lda % 4 == 0);
    const size_t j = div_ceil(kb * 16, 256);  // 4-input chunks per thread
    if (j <= 1) launch_regs<1>(a, lda, m, k, kb, qa, exps, vec, f, g, s);
    else if (j <= 2) launch_regs<2>(a, lda, m, k, kb, qa, exps, vec, f, g, s);
    else if (j <= 4) launch_regs<4>(a, lda, m, k, kb, qa, exps, vec, f, g, s);
    else if (j <= 8) launch_regs<8>(a, lda, m, k, kb, qa, exps, vec, f, g, s);
    else if (j <= 16) launch_regs<16>(a, lda, m, k, kb, qa, exps, vec, f, g, s);
    else
        hipLaunchKernelGGL(quantize_rows_kernel, dim3((unsigned)div_ceil(m, 4)), dim3(256), 0, s, a, lda, m, k, kb,
                           qa, exps, f, g);
    return hipGetLastError();
}

// The row quantiser for rows whose largest magnitudes are known already: h holds m rows of n f32
// values (row stride ldh, a multiple of 64, 16-byte aligned rows; values past n are ignored), and
// tmax the largest |value| of each row over strips column ranges as unsigned bits, all ones for a
// range holding a NaN or an infinity (tmax[row * strips + s], as gemm_lds_kernel<..., QOUT = 1>
// leaves them). Each workgroup takes one 16-row block R and k-blocks QK_CH y .. QK_CH y + QK_CH - 1.
// Thread (r = tid / 16, c = tid % 16) folds row r's maxima c, c + 16, ... over its 16 lanes into the
// row exponent, the one quantize_rows_regs_kernel computes from the values, then writes the digits
// of inputs 64 t + 4 c + [0, 4) as one hi and one lo dword at operand lane 16 (c / 4) + r, bytes
// 4 (c % 4), so that each k-block's 2 KB of digits of the block's 16 rows goes out as one
// contiguous run, and every input is read once with a 16-byte load. Inputs past n and rows past m
// get zero digits.
constexpr int QK_CH = 4;

__global__ __launch_bounds__(256) void quantize_known_kernel(const float *__restrict__ h, size_t ldh, size_t m, int n,
                                                             int kb, const uint32_t *__restrict__ tmax, int strips,
                                                             uint8_t *__restrict__ qa, int32_t *__restrict__ exps,
                                                             size_t bpx, int ny) {
    const int tid = threadIdx.x, r = tid >> 4, c = tid & 15;
    // Workgroup L runs on XCD L % 8; XCD x takes 16-row blocks x bpx .. x bpx + bpx - 1 (ny workgroups
    // a block), the rows the product's tiles leave in that XCD's L2.
    const size_t xg = blockIdx.x % 8, gi = blockIdx.x / 8;
    const size_t R = xg * bpx + gi / ny, row = R * 16 + r;
    if (R * 16 >= m) return;  // uniform
    const int t0 = (int)(gi % ny) * QK_CH;
    const bool valid = row < m;
    const float *hr = h + (valid ? row : 0) * ldh;
    float4 v[QK_CH];
#pragma unroll
    for (int j = 0; j < QK_CH; j++) {
        const int i0 = (t0 + j) * KBLK + 4 * c;
        v[j] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        if (valid && t0 + j < kb) {
            const float4 x = *reinterpret_cast<const float4 *>(hr + i0);
            v[j].x = i0 < n ? x.x : 0.0f;
            v[j].y = i0 + 1 < n ? x.y : 0.0f;
            v[j].z = i0 + 2 < n ? x.z : 0.0f;
            v[j].w = i0 + 3 < n ? x.w : 0.0f;
        }
    }
    // The row's strip maxima: the first 128 strips' loads all issued before any is used, so they cost
    // one memory round trip.
    uint32_t mx = 0u;
    if (valid) {
        const uint32_t *tr = tmax + row * (size_t)strips;
        uint32_t sm[8];
#pragma unroll
        for (int u = 0; u < 8; u++) sm[u] = c + 16 * u < strips ? tr[c + 16 * u] : 0u;
#pragma unroll
        for (int u = 0; u < 8; u++) mx = max(mx, sm[u]);
        for (int st = c + 128; st < strips; st += 16) mx = max(mx, tr[st]);
    }
#pragma unroll
    for (int off = 8; off > 0; off >>= 1) mx = max(mx, (uint32_t)__shfl_xor((int)mx, off, 16));
    const int32_t e = !valid ? 0 : (mx >= 0x7f800000u ? EXP_NONFINITE : row_exponent_of(__uint_as_float(mx)));
    if (valid && t0 == 0 && c == 0) exps[row] = e;
#pragma unroll
    for (int j = 0; j < QK_CH; j++) {
        const int t = t0 + j;
        if (t >= kb) break;
        uint32_t hi = 0u, lo = 0u;
        if (valid) digits4(v[j].x, v[j].y, v[j].z, v[j].w, e, hi, lo);
        uint8_t *blk = qa + ((R * kb + t) * 2) * 1024 + (16 * (c >> 2) + r) * 16 + 4 * (c & 3);
        *reinterpret_cast<uint32_t *>(blk) = hi;
        *reinterpret_cast<uint32_t *>(blk + 1024) = lo;
    }
}

hipError_t launch_quantize_known(const float *h, size_t ldh, size_t m, size_t n, const uint32_t *tmax, int strips,
                                 uint8_t *qa, int32_t *exps, hipStream_t s) {
    if (m == 0 || n == 0) return hipSuccess;
    const size_t kb = div_ceil(n, KBLK);
    if (ldh % KBLK != 0 || ldh < kb * KBLK || reinterpret_cast<uintptr_t>(h) % 16 != 0) return hipErrorInvalidValue;
    const size_t bpx = div_ceil(div_ceil(m, (size_t)16), (size_t)8), ny = div_ceil(kb, (size_t)QK_CH);
    hipLaunchKernelGGL(quantize_known_kernel, dim3((unsigned)(8 * bpx * ny)), dim3(256), 0, s, h, ldh, m, (int)n,
                       (int)kb, tmax, strips, qa, exps, bpx, (int)ny);
    return hipGetLastError();
}

// out = a * sigmoid(b) as the reference's SIMD glu computes it: a / (1 + exp(0 - b))
// (src/kernels/avx512.rs:410-430).
__global__ __launch_bounds__(256) void glu_kernel(const float *__restrict__ x, size_t ldx, size_t m, size_t half,
                                                  float *__restrict__ out, size_t ldo) {
    const size_t total = m * half;
    for (size_t idx = (size_t)blockIdx.x * 256 + threadIdx.x; idx < total; idx += (size_t)gridDim.x * 256) {
        const size_t r = idx / half, j = idx % half;
        const float av = x[r * ldx + j], bv = x[r * ldx + half + j];
        out[r * ldo + j] = av / (1.0f + exp_simd(0.0f - bv));
    }
}

hipError_t launch_glu(const float *x, size_t ldx, size_t m, size_t half, float *out, size_t ldo, hipStream_t s) {
    size_t total = m * half;
    if (total == 0) return hipSuccess;
    size_t blocks = div_ceil(total, 256);
    if (blocks > 65536) blocks = 65536;
    hipLaunchKernelGGL(glu_kernel, dim3((unsigned)blocks), dim3(256), 0, s, x, ldx, m, half, out, ldo);
    return hipGetLastError();
}

// softmax of each row in place as the reference's AVX-512 kernel computes it
// (src/kernels/avx512.rs:382-407): the row maximum; e = exp(x - max) with the SIMD exp, stored;
// sixteen partial sums, partial j adding e[j], e[j + 16], ... in order from +0, folded by halves
// (j + 8, j + 4, j + 2, j + 1); inv = 1 / sum; x = e * inv. One workgroup per row. The maximum of
// a row without NaN is the same in any order, so the workgroup reduces it at once; a row holding a
// NaN takes the reference's lane order (x86 MAXPS per lane from -inf, then the halving fold with
// the lower lane first). The sums are the serial part: the row goes through LDS in chunks of
// SM_CH values, transposed so that lane j of wavefront 0 reads its partial's inputs contiguously,
// and lanes 0..15 continue their sixteen chains chunk after chunk. Every thread reads back only
// the e values it stored itself.
constexpr int SM_CH = 4096, SM_LD = SM_CH / 16 + 4;

__device__ __forceinline__ float x86_maxf(float a, float b) { return a > b ? a : b; }

__global__ __launch_bounds__(256) void softmax_kernel(float *__restrict__ x, size_t ldx, size_t m, int n) {
    __shared__ float eT[16 * SM_LD];
    __shared__ float red[4];
    __shared__ int nan_s[4];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    for (size_t row = blockIdx.x; row < m; row += gridDim.x) {
        float *p = x + row * ldx;
        float mx = -INFINITY;
        int nan = 0;
        for (int i = tid; i < n; i += 256) {
            const float v = p[i];
            nan |= v != v;
            mx = v > mx ? v : mx;
        }
        for (int o = 32; o >= 1; o >>= 1) {
            const float y = __shfl_xor(mx, o);
            mx = y > mx ? y : mx;
            nan |= __shfl_xor(nan, o);
        }
        if (lane == 0) {
            red[wave] = mx;
            nan_s[wave] = nan;
        }
        __syncthreads();
        mx = x86_maxf(x86_maxf(red[0], red[1]), x86_maxf(red[2], red[3]));
        if (nan_s[0] | nan_s[1] | nan_s[2] | nan_s[3]) {
            // The reference's lane order: partial j folds x[j], x[j + 16], ... into -inf.
            float pm = -INFINITY;
            if (wave == 0 && lane < 16)
                for (int i = lane; i < n; i += 16) pm = x86_maxf(pm, p[i]);
            for (int o = 8; o >= 1; o >>= 1) {
                const float y = __shfl_down(pm, o, 16);
                pm = x86_maxf(pm, y);  // lanes j < o: lower lane j first, upper lane j + o second
            }
            if (tid == 0) red[0] = pm;
            __syncthreads();
            mx = red[0];
        }
        float part = 0.0f;
        for (int c0 = 0; c0 < n; c0 += SM_CH) {
            const int len = min(SM_CH, n - c0);
            __syncthreads();  // the previous chunk's sums are done with eT
            for (int i = tid; i < len; i += 256) {
                const float e = exp_simd(p[c0 + i] - mx);
                p[c0 + i] = e;
                eT[(i & 15) * SM_LD + (i >> 4)] = e;
            }
            __syncthreads();
            if (wave == 0 && lane < 16) {
                const float *col = eT + lane * SM_LD;
                const int cnt = (len - lane + 15) >> 4;  // inputs j + 16 t < len of this partial
                for (int t = 0; t < cnt; t++) part = part + col[t];
            }
        }
        if (wave == 0) {
            float s = part;
            s = s + __shfl_xor(s, 8, 16);
            s = s + __shfl_xor(s, 4, 16);
            s = s + __shfl_xor(s, 2, 16);
            s = s + __shfl_xor(s, 1, 16);
            if (lane == 0) red[0] = 1.0f / s;
        }
        __syncthreads();
        const float inv = red[0];
        for (int i = tid; i < n; i += 256) p[i] = p[i] * inv;
        __syncthreads();  // red is rewritten by the next row
    }
}

// The same softmax with the row held in registers (n <= 256 J): thread t holds inputs t + 256 j,
// read from memory once. The maximum as above (a row holding a NaN takes the reference's lane order
// from memory, which still holds the inputs); e = exp(x - max) kept in registers; for the sums each
// chunk of SM_CH values is staged in LDS transposed as above, and lane j of wavefront 0 reads its
// partial's inputs sixteen bytes at a time, 32 values ahead of its additions (the same additions in
// the same order: a read per addition made the chains wait on LDS 1024 times per row); the outputs
// e * inv are written once. Granite's self-conditioning softmax (750 rows of 16384) took 117 us
// with the kernel above. FULL: n == 256 J, no input past the row's end.
template <int J, bool FULL>
__global__ __launch_bounds__(256) void softmax_regs_kernel(float *__restrict__ x, size_t ldx, size_t m, int n) {
    __shared__ __attribute__((aligned(16))) float eT[16 * SM_LD];
    __shared__ float red[4];
    __shared__ int nan_s[4];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    for (size_t row = blockIdx.x; row < m; row += gridDim.x) {
        float *p = x + row * ldx;
        float v[J];
        float mx = -INFINITY;
        int nan = 0;
#pragma unroll
        for (int j = 0; j < J; j++) {
            const int i = tid + 256 * j;
            v[j] = FULL || i < n ? p[i] : -INFINITY;
            nan |= v[j] != v[j];
            mx = v[j] > mx ? v[j] : mx;
        }
        for (int o = 32; o >= 1; o >>= 1) {
            const float y = __shfl_xor(mx, o);
            mx = y > mx ? y : mx;
            nan |= __shfl_xor(nan, o);
        }
        if (lane == 0) {
            red[wave] = mx;
            nan_s[wave] = nan;
        }
        __syncthreads();
        mx = x86_maxf(x86_maxf(red[0], red[1]), x86_maxf(red[2], red[3]));
        if (nan_s[0] | nan_s[1] | nan_s[2] | nan_s[3]) {
            float pm = -INFINITY;
            if (wave == 0 && lane < 16)
                for (int i = lane; i < n; i += 16) pm = x86_maxf(pm, p[i]);
            for (int o = 8; o >= 1; o >>= 1) {
                const float y = __shfl_down(pm, o, 16);
                pm = x86_maxf(pm, y);
            }
            __syncthreads();  // every thread has read red before it is rewritten
            if (tid == 0) red[0] = pm;
            __syncthreads();
            mx = red[0];
        }
#pragma unroll
        for (int j = 0; j < J; j++)
            if (FULL || tid + 256 * j < n) v[j] = exp_simd(v[j] - mx);
        float part = 0.0f;
#pragma unroll
        for (int c = 0; c < (J + 15) / 16; c++) {
            const int c0 = c * SM_CH;
            if (c0 >= n) break;  // uniform
            const int len = min(SM_CH, n - c0);
            __syncthreads();  // the previous chunk's sums (and every read of red) are done
#pragma unroll
            for (int jj = 0; jj < 16; jj++) {
                const int il = tid + 256 * jj;  // input c0 + il is v[16 c + jj]
                if (16 * c + jj < J && (FULL || il < len)) eT[(il & 15) * SM_LD + (il >> 4)] = v[16 * c + jj];
            }
            __syncthreads();
            if (wave == 0 && lane < 16) {
                const float *col = eT + lane * SM_LD;
                const int cnt = (len - lane + 15) >> 4;  // inputs j + 16 t < len of this partial
                int t = 0;
                for (; t + 32 <= cnt; t += 32) {
                    float4 q[8];
#pragma unroll
                    for (int u = 0; u < 8; u++) q[u] = reinterpret_cast<const float4 *>(col + t)[u];
#pragma unroll
                    for (int u = 0; u < 8; u++) {
                        part = part + q[u].x;
                        part = part + q[u].y;
                        part = part + q[u].z;
                        part = part + q[u].w;
                    }
                }
                for (; t < cnt; t++) part = part + col[t];
            }
        }
        if (wave == 0) {
            float s = part;
            s = s + __shfl_xor(s, 8, 16);
            s = s + __shfl_xor(s, 4, 16);
            s = s + __shfl_xor(s, 2, 16);
            s = s + __shfl_xor(s, 1, 16);
            if (lane == 0) red[0] = 1.0f / s;
        }
        __syncthreads();
        const float inv = red[0];
#pragma unroll
        for (int j = 0; j < J; j++) {
            const int i = tid + 256 * j;
            if (FULL || i < n) p[i] = v[j] * inv;
        }
        __syncthreads();  // red is rewritten by the next row
    }
}

hipError_t launch_softmax(float *x, size_t ldx, size_t m, size_t n, hipStream_t s) {
    if (m == 0 || n == 0) return hipSuccess;
    const size_t blocks = m < 65536 ? m : 65536;
    const dim3 g((unsigned)blocks), b(256);
    if (n <= 1024) hipLaunchKernelGGL((softmax_regs_kernel<4, false>), g, b, 0, s, x, ldx, m, (int)n);
    else if (n <= 4096) hipLaunchKernelGGL((softmax_regs_kernel<16, false>), g, b, 0, s, x, ldx, m, (int)n);
    else if (n <= 8192) hipLaunchKernelGGL((softmax_regs_kernel<32, false>), g, b, 0, s, x, ldx, m, (int)n);
    else if (n == 16384) hipLaunchKernelGGL((softmax_regs_kernel<64, true>), g, b, 0, s, x, ldx, m, (int)n);
    else if (n < 16384) hipLaunchKernelGGL((softmax_regs_kernel<64, false>), g, b, 0, s, x, ldx, m, (int)n);
    else hipLaunchKernelGGL(softmax_kernel, g, b, 0, s, x, ldx, m, (int)n);
    return hipGetLastError();
}

// Granite's strided-block pooling (src/granite.rs:918-931): output row r of sequence b is
// (x[b frames + 2 r] + x[b frames + 2 r + 1]) / 2, a rounded sum then an exact halving, for
// r < frames / 2 (a last odd frame dropped).
__global__ __launch_bounds__(256) void average_pairs_kernel(const float *__restrict__ x, size_t ldx, size_t frames,
                                                            size_t rows, size_t total, size_t n,
                                                            float *__restrict__ out, size_t ldo) {
    const size_t cells = total * n;
    for (size_t idx = (size_t)blockIdx.x * 256 + threadIdx.x; idx < cells; idx += (size_t)gridDim.x * 256) {
        const size_t r = idx / n, c = idx - r * n;
        const size_t b = r / rows, src = b * frames + 2 * (r - b * rows);
        out[r * ldo + c] = (x[src * ldx + c] + x[(src + 1) * ldx + c]) / 2.0f;
    }
}

hipError_t launch_average_pairs(const float *x, size_t ldx, size_t frames, size_t batch, size_t n, float *out,
                                size_t ldo, hipStream_t s) {
    const size_t rows = frames / 2, total = rows * batch;
    if (total == 0 || n == 0) return hipSuccess;
    size_t blocks = div_ceil(total * n, 256);
    if (blocks > 65536) blocks = 65536;
    hipLaunchKernelGGL(average_pairs_kernel, dim3((unsigned)blocks), dim3(256), 0, s, x, ldx, frames, rows, total, n,
                       out, ldo);
    return hipGetLastError();
}

// LayerNorm of rows of n values as the reference's AVX-512 kernel computes it
// (src/kernels/avx512.rs:346-380): sixteen partial sums, partial j adding inputs j, j + 16, ... in
// order, folded by halves (j + 8, j + 4, j + 2, j + 1) into the row sum; mean = sum / n; the same
// for fma(d, d, q) with d = x - mean; rstd = 1 / sqrt(q / n + eps); out = fma((x - mean) rstd,
// gamma, beta). Sixteen lanes per row hold the sixteen partials, so a wavefront takes four rows.
// out may be x (each input is read before its own output is written).
__global__ __launch_bounds__(256) void layer_norm_kernel(const float *x, size_t ldx, size_t m, int n,
                                                         const float *__restrict__ gamma,
                                                         const float *__restrict__ beta, float eps, float *out,
                                                         size_t ldo) {
    const int j = threadIdx.x & 15;
    const size_t row = (size_t)blockIdx.x * 16 + (threadIdx.x >> 4);
    const bool valid = row < m;
    const float *xr = x + (valid ? row : 0) * ldx;
    float s = 0.0f;
    if (valid)
        for (int i = j; i < n; i += 16) s = s + xr[i];
    s = s + __shfl_xor(s, 8, 16);
    s = s + __shfl_xor(s, 4, 16);
    s = s + __shfl_xor(s, 2, 16);
    s = s + __shfl_xor(s, 1, 16);
    const float mean = s / (float)n;
    float q = 0.0f;
    if (valid)
        for (int i = j; i < n; i += 16) {
            const float d = xr[i] - mean;
            q = __builtin_fmaf(d, d, q);
        }
    q = q + __shfl_xor(q, 8, 16);
    q = q + __shfl_xor(q, 4, 16);
    q = q + __shfl_xor(q, 2, 16);
    q = q + __shfl_xor(q, 1, 16);
    const float rstd = 1.0f / __builtin_sqrtf(q / (float)n + eps);
    if (valid) {
        float *orow = out + row * ldo;
        for (int i = j; i < n; i += 16) {
            const float d = (xr[i] - mean) * rstd;
            orow[i] = __builtin_fmaf(d, gamma[i], beta[i]);
        }
    }
}

// The same arithmetic with the rows staged in LDS: R rows of n values (n <= LN_LDS_MAX, rows
// LN_PAD floats apart so the four rows of a wavefront's partial sums fall in different banks) are
// read once with 16-byte loads when every row is 16-byte aligned, the sixteen partials of each row
// are summed from LDS in the order above, and the outputs go out in 16-byte runs when out's rows
// are aligned. Every input of the block is read before any output is written, so out may be x.
constexpr int LN_PAD = 16, LN_LDS_MAX = 16384 - LN_PAD;  // one padded row fits 64 KB
constexpr int LN4_MAX = 1024, LN4_ROW = LN4_MAX + 16;  // layer_norm4_kernel's rows

__global__ __launch_bounds__(256) void layer_norm_lds_kernel(const float *x, size_t ldx, size_t m, int n, int R,
                                                             const float *__restrict__ gamma,
                                                             const float *__restrict__ beta, float eps, float *out,
                                                             size_t ldo) {
    extern __shared__ __attribute__((aligned(16))) float rows_s[];
    __shared__ float stat[16][2];
    const int tid = threadIdx.x, stride = n + LN_PAD;
    const size_t row0 = (size_t)blockIdx.x * R;
    const int nr = (int)min((size_t)R, m - row0);
    const bool vin = ((reinterpret_cast<uintptr_t>(x) | ldx * sizeof(float)) % 16 == 0) && n % 4 == 0;
    if (vin) {
        const int q = n / 4;
        for (int c = tid; c < nr * q; c += 256) {
            const int r = c / q, i = 4 * (c - r * q);
            *reinterpret_cast<float4 *>(rows_s + r * stride + i) =
                *reinterpret_cast<const float4 *>(x + (row0 + r) * ldx + i);
        }
    } else {
        for (int c = tid; c < nr * n; c += 256) {
            const int r = c / n, i = c - r * n;
            rows_s[r * stride + i] = x[(row0 + r) * ldx + i];
        }
    }
    __syncthreads();
    const int j = tid & 15, r = tid >> 4;
    if (r < nr) {
        const float *xr = rows_s + r * stride;
        float s = 0.0f;
        for (int i = j; i < n; i += 16) s = s + xr[i];
        s = s + __shfl_xor(s, 8, 16);
        s = s + __shfl_xor(s, 4, 16);
        s = s + __shfl_xor(s, 2, 16);
        s = s + __shfl_xor(s, 1, 16);
        const float mean = s / (float)n;
        float q = 0.0f;
        for (int i = j; i < n; i += 16) {
            const float d = xr[i] - mean;
            q = __builtin_fmaf(d, d, q);
        }
        q = q + __shfl_xor(q, 8, 16);
        q = q + __shfl_xor(q, 4, 16);
        q = q + __shfl_xor(q, 2, 16);
        q = q + __shfl_xor(q, 1, 16);
        if (j == 0) {
            stat[r][0] = mean;
            stat[r][1] = 1.0f / __builtin_sqrtf(q / (float)n + eps);
        }
    }
    __syncthreads();
    const bool vout = ((reinterpret_cast<uintptr_t>(out) | ldo * sizeof(float)) % 16 == 0) && n % 4 == 0 &&
                      (reinterpret_cast<uintptr_t>(gamma) | reinterpret_cast<uintptr_t>(beta)) % 16 == 0;
    if (vout) {
        const int q = n / 4;
        for (int c = tid; c < nr * q; c += 256) {
            const int rr = c / q, i = 4 * (c - rr * q);
            const float mean = stat[rr][0], rstd = stat[rr][1];
            const float4 v = *reinterpret_cast<const float4 *>(rows_s + rr * stride + i);
            const float4 g = *reinterpret_cast<const float4 *>(gamma + i);
            const float4 b = *reinterpret_cast<const float4 *>(beta + i);
            float4 o;
            o.x = __builtin_fmaf((v.x - mean) * rstd, g.x, b.x);
            o.y = __builtin_fmaf((v.y - mean) * rstd, g.y, b.y);
            o.z = __builtin_fmaf((v.z - mean) * rstd, g.z, b.z);
            o.w = __builtin_fmaf((v.w - mean) * rstd, g.w, b.w);
            *reinterpret_cast<float4 *>(out + (row0 + rr) * ldo + i) = o;
        }
    } else {
        for (int c = tid; c < nr * n; c += 256) {
            const int rr = c / n, i = c - rr * n;
            const float d = (rows_s[rr * stride + i] - stat[rr][0]) * stat[rr][1];
            out[(row0 + rr) * ldo + i] = __builtin_fmaf(d, gamma[i], beta[i]);
        }
    }
}

bool layer_norm_row_fits(const float *x, size_t ldx, size_t m, size_t n, const float *gamma, const float *beta,
                          const float *out, size_t ldo);
hipError_t launch_layer_norm4(const float *x, size_t ldx, size_t m, size_t n, const float *gamma, const float *beta,
                              float eps, float *out, size_t ldo, uint8_t *qa, int32_t *exps, hipStream_t s);
hipError_t launch_layer_norm_row(const float *x, size_t ldx, size_t m, size_t n, const float *gamma,
                                  const float *beta, float eps, float *out, size_t ldo, uint8_t *qa, int32_t *exps,
                                  hipStream_t s, const float *gamma2 = nullptr, const float *beta2 = nullptr,
                                  float eps2 = 0.0f);

hipError_t launch_layer_norm(const float *x, size_t ldx, size_t m, size_t n, const float *gamma, const float *beta,
                             float eps, float *out, size_t ldo, hipStream_t s) {
    if (m == 0 || n == 0) return hipSuccess;
    if (layer_norm_row_fits(x, ldx, m, n, gamma, beta, out, ldo))
        return launch_layer_norm_row(x, ldx, m, n, gamma, beta, eps, out, ldo, nullptr, nullptr, s);
    if (n <= (size_t)LN4_MAX) return launch_layer_norm4(x, ldx, m, n, gamma, beta, eps, out, ldo, nullptr, nullptr, s);
    if (n <= (size_t)LN_LDS_MAX) {
        // Up to sixteen rows and 64 KB of LDS per block.
        const int R = (int)min((size_t)16, (size_t)16384 / (n + LN_PAD));
        const size_t lds = (size_t)R * (n + LN_PAD) * sizeof(float);
        hipLaunchKernelGGL(layer_norm_lds_kernel, dim3((unsigned)div_ceil(m, (size_t)R)), dim3(256), lds, s, x, ldx, m,
                           (int)n, R, gamma, beta, eps, out, ldo);
        return hipGetLastError();
    }
    hipLaunchKernelGGL(layer_norm_kernel, dim3((unsigned)div_ceil(m, (size_t)16)), dim3(256), 0, s, x, ldx, m, (int)n,
                       gamma, beta, eps, out, ldo);
    return hipGetLastError();
}

// LayerNorm of one 16-row block (one row block of the quantised layout) followed by the two-digit
// quantisation of its outputs: the bits layer_norm_kernel writes, then those quantize_rows_regs_kernel
// makes of them, in one launch. Pass 1 is layer_norm_kernel's: thread (r = tid / 16, j = tid % 16)
// sums partial j of row r, the row's mean and rstd go to LDS. Pass 2 walks the runs of 16 inputs
// the GEMM's A operand reads: run rho (rho = tid, tid + 256, ...) is k-block t = rho / 64 and operand
// lane L = rho % 64, i.e. inputs 64 t + 16 (L / 16) + [0, 16) of row L % 16, so the 16 threads with
// tid % 16 == r hold all of row r. Each computes its outputs (writing them to out when given) and
// their largest magnitude; the row's largest gives its exponent, and pass 3 computes the outputs
// again and writes each run's 16 hi and 16 lo digits as one 16-byte store each, lane L of the run's
// 1 KB operand blocks. The inputs are read from memory once and from the caches after that. Digits
// of rows past m and of inputs past n are zero. out may be x: every read of an input precedes the
// write of its output in the same thread, and pass 1 ends at a barrier before any write.
__global__ __launch_bounds__(256) void layer_norm_quant_kernel(const float *x, size_t ldx, size_t m, int n,
                                                               const float *__restrict__ gamma,
                                                               const float *__restrict__ beta, float eps, float *out,
                                                               size_t ldo, uint8_t *__restrict__ qa,
                                                               int32_t *__restrict__ exps, int kb, int vec) {
    __shared__ float stat[16][2];
    __shared__ float part_max[4][16];
    __shared__ int part_bad[4][16];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const size_t R = blockIdx.x, row0 = R * 16;
    {
        const int j = tid & 15, r = tid >> 4;
        const size_t row = row0 + r;
        const bool valid = row < m;
        const float *xr = x + (valid ? row : 0) * ldx;
        float s = 0.0f;
        if (valid)
            for (int i = j; i < n; i += 16) s = s + xr[i];
        s = s + __shfl_xor(s, 8, 16);
        s = s + __shfl_xor(s, 4, 16);
        s = s + __shfl_xor(s, 2, 16);
        s = s + __shfl_xor(s, 1, 16);
        const float mean = s / (float)n;
        float q = 0.0f;
        if (valid)
            for (int i = j; i < n; i += 16) {
                const float d = xr[i] - mean;
                q = __builtin_fmaf(d, d, q);
            }
        q = q + __shfl_xor(q, 8, 16);
        q = q + __shfl_xor(q, 4, 16);
        q = q + __shfl_xor(q, 2, 16);
        q = q + __shfl_xor(q, 1, 16);
        if (j == 0) {
            stat[r][0] = mean;
            stat[r][1] = 1.0f / __builtin_sqrtf(q / (float)n + eps);
        }
    }
    __syncthreads();
    const int r = tid & 15, runs = kb * 64;
    const size_t row = row0 + r;
    const bool valid = row < m;
    const float mean = stat[r][0], rstd = stat[r][1];
    const float *xr = x + (valid ? row : 0) * ldx;
    // The outputs of run rho (zero past n) into y.
    auto outputs = [&](int rho, float (&y)[16]) {
        const int i0 = 64 * (rho >> 6) + 16 * ((rho & 63) >> 4);
        if (vec && i0 + 16 <= n) {
#pragma unroll
            for (int c = 0; c < 16; c += 4) {
                const float4 v = *reinterpret_cast<const float4 *>(xr + i0 + c);
                const float4 g = *reinterpret_cast<const float4 *>(gamma + i0 + c);
                const float4 b = *reinterpret_cast<const float4 *>(beta + i0 + c);
                y[c] = __builtin_fmaf((v.x - mean) * rstd, g.x, b.x);
                y[c + 1] = __builtin_fmaf((v.y - mean) * rstd, g.y, b.y);
                y[c + 2] = __builtin_fmaf((v.z - mean) * rstd, g.z, b.z);
                y[c + 3] = __builtin_fmaf((v.w - mean) * rstd, g.w, b.w);
            }
        } else {
#pragma unroll
            for (int c = 0; c < 16; c++) {
                const int i = i0 + c;
                y[c] = i < n ? __builtin_fmaf((xr[i] - mean) * rstd, gamma[i], beta[i]) : 0.0f;
            }
        }
        return i0;
    };
    float amax = 0.0f;
    int bad = 0;
    if (valid) {
        for (int rho = tid; rho < runs; rho += 256) {
            float y[16];
            const int i0 = outputs(rho, y);
#pragma unroll
            for (int c = 0; c < 16; c++) {
                bad |= !__builtin_isfinite(y[c]);
                amax = fmaxf(amax, fabsf(y[c]));
            }
            if (out) {
                float *orow = out + row * ldo;
                if (vec && i0 + 16 <= n && ((reinterpret_cast<uintptr_t>(out) | ldo * sizeof(float)) % 16 == 0)) {
#pragma unroll
                    for (int c = 0; c < 16; c += 4)
                        *reinterpret_cast<float4 *>(orow + i0 + c) = make_float4(y[c], y[c + 1], y[c + 2], y[c + 3]);
                } else {
#pragma unroll
                    for (int c = 0; c < 16; c++)
                        if (i0 + c < n) orow[i0 + c] = y[c];
                }
            }
        }
    }
    // The row's threads: tid % 16 == r, four in each wavefront.
    amax = fmaxf(amax, __shfl_xor(amax, 16, 64));
    amax = fmaxf(amax, __shfl_xor(amax, 32, 64));
    bad |= __shfl_xor(bad, 16, 64);
    bad |= __shfl_xor(bad, 32, 64);
    if (lane < 16) {
        part_max[wave][lane] = amax;
        part_bad[wave][lane] = bad;
    }
    __syncthreads();
    amax = fmaxf(fmaxf(part_max[0][r], part_max[1][r]), fmaxf(part_max[2][r], part_max[3][r]));
    bad = part_bad[0][r] | part_bad[1][r] | part_bad[2][r] | part_bad[3][r];
    const int32_t e = bad ? EXP_NONFINITE : row_exponent_of(amax);
    if (valid && tid < 16) exps[row] = e;
    for (int rho = tid; rho < runs; rho += 256) {
        uint4 hi = make_uint4(0, 0, 0, 0), lo = make_uint4(0, 0, 0, 0);
        if (valid) {
            float y[16];
            outputs(rho, y);
            digits4(y[0], y[1], y[2], y[3], e, hi.x, lo.x);
            digits4(y[4], y[5], y[6], y[7], e, hi.y, lo.y);
            digits4(y[8], y[9], y[10], y[11], e, hi.z, lo.z);
            digits4(y[12], y[13], y[14], y[15], e, hi.w, lo.w);
        }
        uint8_t *blk = qa + ((R * kb + (rho >> 6)) * 2) * 1024 + (rho & 63) * 16;
        *reinterpret_cast<uint4 *>(blk) = hi;
        *reinterpret_cast<uint4 *>(blk + 1024) = lo;
    }
}

// LayerNorm of rows of n <= 1024 values, four rows per single-wavefront workgroup, with its outputs
// written as f32 (out) and/or quantised (qa, exps). The arithmetic is layer_norm_kernel's:
//  pass 1: lane (r = lane / 16, j = lane % 16) loads inputs j, j + 16, ... of row r into registers,
//          all loads in flight at once, and sums partial j from them in order; the same registers
//          give the squared deviations; 16-lane folds as the reference's (j + 8, + 4, + 2, + 1);
//  the rows go to LDS (rows ROW_LDS floats apart, so the 64 lanes' stores hit 64 banks);
//  pass 2: lane (c = lane / 4, r = lane % 4) takes runs c, c + 16, ... of 16 inputs of row r, the
//          runs the GEMM's A operand reads (run rho: k-block rho / 4, operand lane group rho % 4),
//          computes their outputs, writes them to out, and the row's largest magnitude (over the 16
//          lanes holding row r) gives its exponent; each run's 16 hi and 16 lo digits go out as one
//          16-byte store each. Rows past m write zero digits; out may be x (a lane reads a run of x
//          before writing it, and pass 1 of the wavefront precedes every write).
__global__ __launch_bounds__(64) void layer_norm4_kernel(const float *x, size_t ldx, size_t m, int n,
                                                         const float *__restrict__ gamma,
                                                         const float *__restrict__ beta, float eps, float *out,
                                                         size_t ldo, uint8_t *__restrict__ qa,
                                                         int32_t *__restrict__ exps, int kb, int vec, size_t bpx) {
    __shared__ __attribute__((aligned(16))) float rows_s[4 * LN4_ROW];
    __shared__ float stat[4][2];
    const int lane = threadIdx.x;
    // Workgroup L runs on XCD L % 8; XCD x takes 16-row blocks x bpx .. x bpx + bpx - 1, four
    // workgroups a block, the rows a product's tiles leave in that XCD's L2.
    const size_t xg = blockIdx.x % 8, gi = blockIdx.x / 8;
    const size_t row0 = (xg * bpx + gi / 4) * 16 + (gi % 4) * 4;
    if (row0 >= (qa ? (m + 15) / 16 * 16 : m)) return;  // uniform
    {
        const int r = lane >> 4, j = lane & 15;
        const size_t row = row0 + r;
        const bool valid = row < m;
        const float *xr = x + (valid ? row : 0) * ldx;
        // Every lane loads 64 values from valid addresses (indices past n read element 0, rows past
        // m read row 0), so the loads are one straight run in flight together; the sums below take
        // only the indices below n.
        float v[LN4_MAX / 16];
#pragma unroll
        for (int i = 0; i < LN4_MAX / 16; i++) v[i] = xr[j + 16 * i < n ? j + 16 * i : 0];
        float s = 0.0f;
#pragma unroll
        for (int i = 0; i < LN4_MAX / 16; i++)
            if (j + 16 * i < n) s = s + v[i];
        s = s + __shfl_xor(s, 8, 16);
        s = s + __shfl_xor(s, 4, 16);
        s = s + __shfl_xor(s, 2, 16);
        s = s + __shfl_xor(s, 1, 16);
        const float mean = s / (float)n;
        float q = 0.0f;
#pragma unroll
        for (int i = 0; i < LN4_MAX / 16; i++)
            if (j + 16 * i < n) {
                const float d = v[i] - mean;
                q = __builtin_fmaf(d, d, q);
            }
        q = q + __shfl_xor(q, 8, 16);
        q = q + __shfl_xor(q, 4, 16);
        q = q + __shfl_xor(q, 2, 16);
        q = q + __shfl_xor(q, 1, 16);
        if (j == 0) {
            stat[r][0] = mean;
            stat[r][1] = 1.0f / __builtin_sqrtf(q / (float)n + eps);
        }
#pragma unroll
        for (int i = 0; i < LN4_MAX / 16; i++) rows_s[r * LN4_ROW + j + 16 * i] = v[i];
    }
    __syncthreads();
    if (!qa) {
        // f32 outputs only: lane (r = lane / 16, j = lane % 16) writes the float4s j, j + 16, ... of
        // row r, so a row's 16 lanes store 256 contiguous bytes per instruction.
        const int r = lane >> 4, j = lane & 15;
        const size_t row = row0 + r;
        if (row >= m) return;
        const float mean = stat[r][0], rstd = stat[r][1];
        const float *src = rows_s + r * LN4_ROW;
        float *orow = out + row * ldo;
        const bool v4 = vec && n % 4 == 0 && ((reinterpret_cast<uintptr_t>(out) | ldo * sizeof(float)) % 16 == 0);
        if (v4) {
            for (int i0 = 4 * j; i0 < n; i0 += 64) {
                const float4 xv = *reinterpret_cast<const float4 *>(src + i0);
                const float4 g = *reinterpret_cast<const float4 *>(gamma + i0);
                const float4 b = *reinterpret_cast<const float4 *>(beta + i0);
                float4 o;
                o.x = __builtin_fmaf((xv.x - mean) * rstd, g.x, b.x);
                o.y = __builtin_fmaf((xv.y - mean) * rstd, g.y, b.y);
                o.z = __builtin_fmaf((xv.z - mean) * rstd, g.z, b.z);
                o.w = __builtin_fmaf((xv.w - mean) * rstd, g.w, b.w);
                *reinterpret_cast<float4 *>(orow + i0) = o;
            }
        } else {
            for (int i = j; i < n; i += 16) orow[i] = __builtin_fmaf((src[i] - mean) * rstd, gamma[i], beta[i]);
        }
        return;
    }
    const int c = lane >> 2, r = lane & 3;
    const size_t row = row0 + r;
    const bool valid = row < m;
    const float mean = stat[r][0], rstd = stat[r][1];
    const int runs = (n + 15) / 16;  // runs holding inputs; runs up to kb * 4 hold zero digits
    float y[LN4_MAX / 256][16];
    float amax = 0.0f;
    int bad = 0;
#pragma unroll
    for (int u = 0; u < LN4_MAX / 256; u++) {
        const int rho = c + 16 * u, i0 = 16 * rho;
#pragma unroll
        for (int e = 0; e < 16; e++) y[u][e] = 0.0f;
        if (!valid || rho >= runs) continue;
        const float *src = rows_s + r * LN4_ROW + i0;
        if (vec && i0 + 16 <= n) {
#pragma unroll
            for (int e = 0; e < 16; e += 4) {
                const float4 xv = *reinterpret_cast<const float4 *>(src + e);
                const float4 g = *reinterpret_cast<const float4 *>(gamma + i0 + e);
                const float4 b = *reinterpret_cast<const float4 *>(beta + i0 + e);
                y[u][e] = __builtin_fmaf((xv.x - mean) * rstd, g.x, b.x);
                y[u][e + 1] = __builtin_fmaf((xv.y - mean) * rstd, g.y, b.y);
                y[u][e + 2] = __builtin_fmaf((xv.z - mean) * rstd, g.z, b.z);
                y[u][e + 3] = __builtin_fmaf((xv.w - mean) * rstd, g.w, b.w);
            }
        } else {
#pragma unroll
            for (int e = 0; e < 16; e++)
                if (i0 + e < n) y[u][e] = __builtin_fmaf((src[e] - mean) * rstd, gamma[i0 + e], beta[i0 + e]);
        }
#pragma unroll
        for (int e = 0; e < 16; e++) {
            bad |= !__builtin_isfinite(y[u][e]);
            amax = fmaxf(amax, fabsf(y[u][e]));
        }
        if (out) {
            float *orow = out + row * ldo + i0;
            if (vec && i0 + 16 <= n && ((reinterpret_cast<uintptr_t>(out) | ldo * sizeof(float)) % 16 == 0)) {
#pragma unroll
                for (int e = 0; e < 16; e += 4)
                    *reinterpret_cast<float4 *>(orow + e) = make_float4(y[u][e], y[u][e + 1], y[u][e + 2], y[u][e + 3]);
            } else {
#pragma unroll
                for (int e = 0; e < 16; e++)
                    if (i0 + e < n) orow[e] = y[u][e];
            }
        }
    }
    // Row r's lanes are those with lane % 4 == r.
#pragma unroll
    for (int off = 4; off < 64; off <<= 1) {
        amax = fmaxf(amax, __shfl_xor(amax, off, 64));
        bad |= __shfl_xor(bad, off, 64);
    }
    const int32_t e = bad ? EXP_NONFINITE : row_exponent_of(amax);
    if (valid && c == 0) exps[row] = e;
    const size_t R = row / 16;
#pragma unroll
    for (int u = 0; u < LN4_MAX / 256; u++) {
        const int rho = c + 16 * u;
        if (rho >= kb * 4) continue;
        uint4 hi = make_uint4(0, 0, 0, 0), lo = make_uint4(0, 0, 0, 0);
        if (valid) {
            digits4(y[u][0], y[u][1], y[u][2], y[u][3], e, hi.x, lo.x);
            digits4(y[u][4], y[u][5], y[u][6], y[u][7], e, hi.y, lo.y);
            digits4(y[u][8], y[u][9], y[u][10], y[u][11], e, hi.z, lo.z);
            digits4(y[u][12], y[u][13], y[u][14], y[u][15], e, hi.w, lo.w);
        }
        uint8_t *blk = qa + ((R * kb + (rho >> 2)) * 2) * 1024 + (16 * (rho & 3) + row % 16) * 16;
        *reinterpret_cast<uint4 *>(blk) = hi;
        *reinterpret_cast<uint4 *>(blk + 1024) = lo;
    }
}

hipError_t launch_layer_norm4(const float *x, size_t ldx, size_t m, size_t n, const float *gamma, const float *beta,
                              float eps, float *out, size_t ldo, uint8_t *qa, int32_t *exps, hipStream_t s) {
    const size_t kb = div_ceil(n, KBLK);
    const int vec = ((reinterpret_cast<uintptr_t>(x) | ldx * sizeof(float) | reinterpret_cast<uintptr_t>(gamma) |
                      reinterpret_cast<uintptr_t>(beta)) % 16 == 0);
    // Workgroups of four rows, four a 16-row block (whose rows past m still get their zero digits),
    // bpx blocks per XCD.
    const size_t bpx = div_ceil(div_ceil(m, (size_t)16), (size_t)8);
    hipLaunchKernelGGL(layer_norm4_kernel, dim3((unsigned)(8 * bpx * 4)), dim3(64), 0, s, x, ldx, m, (int)n, gamma,
                       beta, eps, out, ldo, qa, exps, (int)kb, vec, bpx);
    return hipGetLastError();
}

constexpr int LNQ_MAX = 1024;

// LayerNorm of a row of n <= 1024 values (n % 4 == 0, rows and gamma, beta 16-byte aligned) per
// workgroup of 256 threads, with its outputs written as f32 (out) and/or quantised (qa, exps). The
// arithmetic is layer_norm_kernel's:
//  1. thread t loads inputs 4 t + [0, 4) (zeros past n) with one 16-byte load, keeps them in
//     registers and copies them to LDS; gamma and beta are loaded with them;
//  2. lanes p < 16 of wavefront 0 run the row's two chains in the reference's order: lane p adds
//     inputs p, p + 16, ... in order (the zeros past n leave a sum unchanged, as it starts at +0 and
//     cannot become -0), then the squared deviations the same, a masked deviation of 0 past n; both
//     fold as the reference's (p + 8, + 4, + 2, + 1); mean and rstd go to LDS;
//  3. after one barrier every thread writes its four outputs (16-byte stores to out) and, with the
//     row maximum reduced over the workgroup, their digits: chunk t is k-block t / 16, operand lane
//     16 ((t % 16) / 4) + row % 16, bytes 4 (t % 4) + [0, 4).
// Rows are spread over the XCDs in 16-row blocks as quantize_rows_regs_kernel spreads them; rows past
// m up to the end of the last 16-row block get zero digits when qa is given. out may be x: a thread
// reads its inputs before it writes their outputs, and no thread writes another's inputs.
//
// PAIR: two LayerNorms of the row in one launch, as a stack's layer boundary runs them (a layer's
// last LayerNorm in place, then the next layer's first with its digits): the first (gamma, beta,
// eps) goes to out as above; its outputs, exactly as stored, are then copied to LDS and run through
// the same chains for the second (gamma2, beta2, eps2), whose outputs give the digits. The bits of
// the two launches, with the row read from memory once.

// Lanes p < 16 of wavefront 0: the row's mean and 1 / sqrt(var + eps) (step 2 above) into stat.
template <bool FULL>
__device__ __forceinline__ void row_stats(const float *row_s, int n, float eps, float *stat, int p) {
    const float *xr = row_s + p;
    float s = 0.0f;
#pragma unroll
    for (int q0 = 0; q0 < LNQ_MAX / 16; q0 += 16) {
#pragma unroll
        for (int q = q0; q < q0 + 16; q++) s = s + xr[16 * q];
    }
    s = s + __shfl_xor(s, 8, 16);
    s = s + __shfl_xor(s, 4, 16);
    s = s + __shfl_xor(s, 2, 16);
    s = s + __shfl_xor(s, 1, 16);
    const float mean = s / (float)n;
    float sq = 0.0f;
#pragma unroll
    for (int q0 = 0; q0 < LNQ_MAX / 16; q0 += 16) {
#pragma unroll
        for (int q = q0; q < q0 + 16; q++) {
            const float d = FULL || p + 16 * q < n ? xr[16 * q] - mean : 0.0f;
            sq = __builtin_fmaf(d, d, sq);
        }
    }
    sq = sq + __shfl_xor(sq, 8, 16);
    sq = sq + __shfl_xor(sq, 4, 16);
    sq = sq + __shfl_xor(sq, 2, 16);
    sq = sq + __shfl_xor(sq, 1, 16);
    if (p == 0) {
        stat[0] = mean;
        stat[1] = 1.0f / __builtin_sqrtf(sq / (float)n + eps);
    }
}

__device__ __forceinline__ float4 ln_out(const float4 &v, float mean, float rstd, const float4 &g, const float4 &b) {
    return float4{__builtin_fmaf((v.x - mean) * rstd, g.x, b.x), __builtin_fmaf((v.y - mean) * rstd, g.y, b.y),
                  __builtin_fmaf((v.z - mean) * rstd, g.z, b.z), __builtin_fmaf((v.w - mean) * rstd, g.w, b.w)};
}

template <bool FULL, bool PAIR>  // FULL: n == LNQ_MAX, no masking in the chains
__global__ __launch_bounds__(256) void layer_norm_row_kernel(const float *x, size_t ldx, size_t m, int n,
                                                             const float *__restrict__ gamma,
                                                             const float *__restrict__ beta, float eps, float *out,
                                                             size_t ldo, uint8_t *__restrict__ qa,
                                                             int32_t *__restrict__ exps, int kb, size_t bpx,
                                                             const float *__restrict__ gamma2,
                                                             const float *__restrict__ beta2, float eps2) {
    __shared__ __attribute__((aligned(16))) float row_s[LNQ_MAX];
    __shared__ float stat[2];
    __shared__ float s_max[4];
    __shared__ int s_bad[4];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const size_t xg = blockIdx.x % 8, i = blockIdx.x / 8;
    const size_t row = (xg * bpx + i / 16) * 16 + i % 16;
    const bool valid = row < m;
    if (!valid && (!qa || row >= (m + 15) / 16 * 16)) return;  // uniform over the workgroup
    const float4 zero = {0.0f, 0.0f, 0.0f, 0.0f};
    const bool in = valid && (FULL || 4 * tid < n);
    float4 v = zero, g = zero, b = zero, g2 = zero, b2 = zero;
    if (in) {
        v = reinterpret_cast<const float4 *>(x + row * ldx)[tid];
        g = reinterpret_cast<const float4 *>(gamma)[tid];
        b = reinterpret_cast<const float4 *>(beta)[tid];
        if constexpr (PAIR) {
            g2 = reinterpret_cast<const float4 *>(gamma2)[tid];
            b2 = reinterpret_cast<const float4 *>(beta2)[tid];
        }
    }
    reinterpret_cast<float4 *>(row_s)[tid] = v;
    __syncthreads();
    if (tid < 16) row_stats<FULL>(row_s, n, eps, stat, tid);
    __syncthreads();
    float4 y = zero;
    if (in) {
        y = ln_out(v, stat[0], stat[1], g, b);
        if (out) reinterpret_cast<float4 *>(out + row * ldo)[tid] = y;
    }
    if constexpr (PAIR) {
        // Every thread has read stat and the chains have read row_s (the barrier above) before the
        // second row and its statistics overwrite them.
        reinterpret_cast<float4 *>(row_s)[tid] = y;
        __syncthreads();
        if (tid < 16) row_stats<FULL>(row_s, n, eps2, stat, tid);
        __syncthreads();
        if (in) y = ln_out(y, stat[0], stat[1], g2, b2);
    }
    if (!qa) return;  // uniform
    float amax = fmaxf(fmaxf(fabsf(y.x), fabsf(y.y)), fmaxf(fabsf(y.z), fabsf(y.w)));
    int bad = !__builtin_isfinite(y.x) | !__builtin_isfinite(y.y) | !__builtin_isfinite(y.z) | !__builtin_isfinite(y.w);
    amax = wave_max(amax);
    bad = wave_or(bad);
    if (lane == 0) {
        s_max[wave] = amax;
        s_bad[wave] = bad;
    }
    __syncthreads();
    amax = fmaxf(fmaxf(s_max[0], s_max[1]), fmaxf(s_max[2], s_max[3]));
    bad = s_bad[0] | s_bad[1] | s_bad[2] | s_bad[3];
    const int32_t e = !valid ? 0 : (bad ? EXP_NONFINITE : row_exponent_of(amax));
    if (valid && tid == 0) exps[row] = e;
    if (tid < kb * 16) {
        uint32_t hi = 0, lo = 0;
        if (valid) digits4(y.x, y.y, y.z, y.w, e, hi, lo);
        const size_t at = qa_offset(row, tid >> 4, 0, kb) + ((tid & 15) >> 2) * 256 + (tid & 3) * 4;
        *reinterpret_cast<uint32_t *>(qa + at) = hi;
        *reinterpret_cast<uint32_t *>(qa + at + 1024) = lo;
    }
}

// Whether layer_norm_row_kernel takes these rows: fewer than LNQ_ROWS_MAX of them (beyond, the
// single-wavefront layer_norm4_kernel fills the chip and costs fewer instructions per row), n <= 1024
// and a multiple of 4, x, gamma, beta (and out when given) 16-byte aligned with row strides of
// whole 16-byte units.
constexpr size_t LNQ_ROWS_MAX = 2048;

bool layer_norm_row_fits(const float *x, size_t ldx, size_t m, size_t n, const float *gamma, const float *beta,
                          const float *out, size_t ldo) {
    uintptr_t al = reinterpret_cast<uintptr_t>(x) | ldx * sizeof(float) | reinterpret_cast<uintptr_t>(gamma) |
                   reinterpret_cast<uintptr_t>(beta);
    if (out) al |= reinterpret_cast<uintptr_t>(out) | ldo * sizeof(float);
    return m < LNQ_ROWS_MAX && n > 0 && n <= (size_t)LNQ_MAX && n % 4 == 0 && al % 16 == 0;
}

// gamma2 non-null: the PAIR instance (out must then be given).
hipError_t launch_layer_norm_row(const float *x, size_t ldx, size_t m, size_t n, const float *gamma,
                                  const float *beta, float eps, float *out, size_t ldo, uint8_t *qa, int32_t *exps,
                                  hipStream_t s, const float *gamma2, const float *beta2, float eps2) {
    const size_t kb = div_ceil(n, KBLK);
    // One workgroup per row of each 16-row block, bpx blocks per XCD.
    const size_t bpx = div_ceil(div_ceil(m, (size_t)16), (size_t)8);
    const unsigned groups = (unsigned)(8 * bpx * 16);
    const bool full = n == (size_t)LNQ_MAX;
    auto kernel = full ? &layer_norm_row_kernel<true, false> : &layer_norm_row_kernel<false, false>;
    if (gamma2) kernel = full ? &layer_norm_row_kernel<true, true> : &layer_norm_row_kernel<false, true>;
    hipLaunchKernelGGL(kernel, dim3(groups), dim3(256), 0, s, x, ldx, m, (int)n, gamma, beta, eps, out, ldo, qa, exps,
                       (int)kb, bpx, gamma2, beta2, eps2);
    return hipGetLastError();
}

hipError_t launch_layer_norm_quant(const float *x, size_t ldx, size_t m, size_t n, const float *gamma,
                                   const float *beta, float eps, float *out, size_t ldo, uint8_t *qa, int32_t *exps,
                                   hipStream_t s) {
    if (m == 0 || n == 0) return hipSuccess;
    if (layer_norm_row_fits(x, ldx, m, n, gamma, beta, out, ldo))
        return launch_layer_norm_row(x, ldx, m, n, gamma, beta, eps, out, ldo, qa, exps, s);
    if (n <= (size_t)LN4_MAX) return launch_layer_norm4(x, ldx, m, n, gamma, beta, eps, out, ldo, qa, exps, s);
    const size_t kb = div_ceil(n, KBLK);
    const int vec = ((reinterpret_cast<uintptr_t>(x) | ldx * sizeof(float) | reinterpret_cast<uintptr_t>(gamma) |
                      reinterpret_cast<uintptr_t>(beta)) % 16 == 0);
    hipLaunchKernelGGL(layer_norm_quant_kernel, dim3((unsigned)div_ceil(m, (size_t)16)), dim3(256), 0, s, x, ldx, m,
                       (int)n, gamma, beta, eps, out, ldo, qa, exps, (int)kb, vec);
    return hipGetLastError();
}

hipError_t launch_layer_norm_pair(const float *x, size_t ldx, size_t m, size_t n, const float *gamma,
                                  const float *beta, float eps, float *out, size_t ldo, const float *gamma2,
                                  const float *beta2, float eps2, uint8_t *qa, int32_t *exps, hipStream_t s) {
    if (m == 0 || n == 0) return hipSuccess;
    if (layer_norm_row_fits(x, ldx, m, n, gamma, beta, out, ldo) &&
        (reinterpret_cast<uintptr_t>(gamma2) | reinterpret_cast<uintptr_t>(beta2)) % 16 == 0)
        return launch_layer_norm_row(x, ldx, m, n, gamma, beta, eps, out, ldo, qa, exps, s, gamma2, beta2, eps2);
    // Elsewhere the two launches, the second reading the first's outputs.
    const hipError_t e = launch_layer_norm(x, ldx, m, n, gamma, beta, eps, out, ldo, s);
    if (e != hipSuccess) return e;
    return launch_layer_norm_quant(out, ldo, m, n, gamma2, beta2, eps2, nullptr, 0, qa, exps, s);
}

// Depthwise 1-D convolution with "same" zero padding, one output row per frame
// t = t0 + r * stride, as the reference's dwconv1d_frame computes it (src/kernels/scalar.rs:164-187):
// out[c] = bias[c], then for each tap j in order, out[c] = out[c] + w[j][c] * x[t + j - kernel/2][c]
// (a rounded product, then a rounded sum), taps outside [0, frames) skipped. With silu the row then
// goes through v / (1 + exp(0 - v)) as the caller's (k.silu)(row) does. Grid z walks a batch of
// equal-length sequences laid one after another (frames input rows, rows output rows each).
//
// Main kernel: a block owns 256 channels (one per lane) and R = 16 (8 for 32 taps at stride 2)
// consecutive output rows; kernel <= KMAX
// and the stride is STRIDE. Each lane loads the SPAN = (R - 1) * STRIDE + KMAX frames its rows reach
// and the KMAX tap weights into registers in one batch of independent loads (frames outside the
// input are clamped to an edge row, their taps skipped below; taps past kernel are never summed),
// then sums its R rows, taps in order, without touching memory. Blocks wholly inside the input
// (all but the first and last of a sequence) skip the edge tests. HBM reads each input row about
// SPAN / (R * STRIDE) times per 256-channel slice and writes each output once.
template <int R, int STRIDE, int KMAX>
__global__ __launch_bounds__(256) void dwconv1d_reg_kernel(const float *__restrict__ x, size_t ldx, int64_t frames,
                                                           size_t channels, const float *__restrict__ w, int kernel,
                                                           const float *__restrict__ bias, int64_t t0, size_t rows,
                                                           int silu, float *__restrict__ out, size_t ldo,
                                                           unsigned tiles, unsigned slices, unsigned total) {
    constexpr int SPAN = (R - 1) * STRIDE + KMAX;
    // Workgroup L runs on XCD L % 8. Each XCD takes a contiguous run of (sequence, row tile, channel
    // slice) work items, slices fastest, so the frames a tile shares with its neighbours are read
    // into one L2 at about the same time.
    const unsigned per = (total + 7) / 8, idx = (blockIdx.x % 8) * per + blockIdx.x / 8;
    if (idx >= total) return;
    const unsigned slice = idx % slices, tile = (idx / slices) % tiles, seq = idx / slices / tiles;
    const size_t c = (size_t)slice * 256 + threadIdx.x;
    const size_t cc = c < channels ? c : channels - 1;  // idle lanes load a valid column and store nothing
    x += (size_t)seq * (size_t)frames * ldx;
    out += (size_t)seq * rows * ldo;
    const size_t r0 = (size_t)tile * R;
    const int64_t first = t0 + (int64_t)r0 * STRIDE - kernel / 2;  // the frame of window slot 0
    float v[SPAN], wr[KMAX];
#pragma unroll
    for (int s = 0; s < SPAN; s++) {
        const int64_t f = first + s;
        const int64_t fc = f < 0 ? 0 : (f >= frames ? frames - 1 : f);
        v[s] = x[(size_t)fc * ldx + cc];
    }
#pragma unroll
    for (int j = 0; j < KMAX; j++) wr[j] = w[(size_t)(j < kernel ? j : kernel - 1) * channels + cc];
    const float b = bias[cc];
    float acc[R];
#pragma unroll
    for (int i = 0; i < R; i++) acc[i] = b;
    if (first >= 0 && first + (R - 1) * STRIDE + kernel <= frames) {
#pragma unroll
        for (int j = 0; j < KMAX; j++) {
            if (j < kernel) {
#pragma unroll
                for (int i = 0; i < R; i++) acc[i] = acc[i] + wr[j] * v[i * STRIDE + j];
            }
        }
    } else {
#pragma unroll
        for (int j = 0; j < KMAX; j++) {
            if (j < kernel) {
#pragma unroll
                for (int i = 0; i < R; i++) {
                    const float nv = acc[i] + wr[j] * v[i * STRIDE + j];
                    acc[i] = (uint64_t)(first + i * STRIDE + j) < (uint64_t)frames ? nv : acc[i];
                }
            }
        }
    }
    if (c >= channels) return;
#pragma unroll
    for (int i = 0; i < R; i++) {
        if (r0 + i >= rows) break;
        float o = acc[i];
        if (silu) o = o / (1.0f + exp_simd(0.0f - o));
        out[(r0 + i) * ldo + c] = o;
    }
}

// Fallback for kernels beyond 32 taps, strides beyond 2 and empty inputs or kernels: the same sums
// straight from global memory, DW_ROWS output rows per lane.
constexpr int DW_ROWS = 8;

__global__ __launch_bounds__(256) void dwconv1d_kernel(const float *__restrict__ x, size_t ldx, int64_t frames,
                                                       size_t channels, const float *__restrict__ w, int kernel,
                                                       const float *__restrict__ bias, int64_t t0, int64_t stride,
                                                       size_t rows, int silu, float *__restrict__ out, size_t ldo) {
    const size_t c = (size_t)blockIdx.y * 256 + threadIdx.x;
    if (c >= channels) return;
    x += (size_t)blockIdx.z * (size_t)frames * ldx;  // sequence z of the batch
    out += (size_t)blockIdx.z * rows * ldo;
    const size_t r0 = (size_t)blockIdx.x * DW_ROWS;
    const int64_t half = kernel / 2;
    const float b = bias[c];
    float acc[DW_ROWS];
#pragma unroll
    for (int i = 0; i < DW_ROWS; i++) acc[i] = b;
    for (int j = 0; j < kernel; j++) {
        const float wj = w[(size_t)j * channels + c];
#pragma unroll
        for (int i = 0; i < DW_ROWS; i++) {
            const int64_t src = t0 + (int64_t)(r0 + i) * stride + j - half;
            if (r0 + i < rows && src >= 0 && src < frames) acc[i] = acc[i] + wj * x[(size_t)src * ldx + c];
        }
    }
#pragma unroll
    for (int i = 0; i < DW_ROWS; i++) {
        if (r0 + i >= rows) break;
        float v = acc[i];
        if (silu) v = v / (1.0f + exp_simd(0.0f - v));
        out[(r0 + i) * ldo + c] = v;
    }
}

template <int R, int STRIDE, int KMAX>
void launch_dwconv_reg(const float *x, size_t ldx, size_t frames, size_t batch, size_t channels, const float *w,
                       size_t kernel, const float *bias, size_t t0, size_t rows, int silu, float *out, size_t ldo,
                       hipStream_t s) {
    // the host keeps tiles * slices * batch below 2^24 work items
    const unsigned tiles = (unsigned)div_ceil(rows, (size_t)R), slices = (unsigned)div_ceil(channels, (size_t)256);
    const unsigned total = tiles * slices * (unsigned)batch;
    hipLaunchKernelGGL((dwconv1d_reg_kernel<R, STRIDE, KMAX>), dim3(div_ceil(total, 8u) * 8), dim3(256), 0, s, x, ldx,
                       (int64_t)frames, channels, w, (int)kernel, bias, (int64_t)t0, rows, silu, out, ldo, tiles, slices,
                       total);
}

// The depthwise convolution of whole sequences (output row r of a sequence = frame r, stride 1) with
// its output rows quantised as the row quantiser would (tg_dwconv1d_quant_device): the same f32
// values as dwconv1d_reg_kernel, then the same exponents and digits as quantize_rows_regs_kernel.
// Workgroup b takes output rows R b .. R b + R - 1 of the stacked sequences (so its rows may hold the
// end of one sequence and the start of the next) over all channels, one channel per thread and
// slice of 1024: R = 16 (a whole QA row block) for large batches, R = 4 (a quarter of one, four
// times the workgroups) for short ones, where the per-row arithmetic and not the memory bounds the
// time. Each thread loads the SPAN input rows its R outputs reach (clamped to the input) and the
// taps into registers, sums taps in order from the bias (a tap whose input row lies outside its
// output row's sequence is skipped, not added as zero), applies the SiLU, and stages the row in LDS
// (row stride CWS floats, 16 bytes past a multiple of 256 so the digit pass reads without bank
// conflicts). The R row maxima and non-finite flags are reduced over the workgroup; then each
// thread packs the digits of 16 inputs of one row into a 16-byte hi and a 16-byte lo store (item
// (t, g, i): k-block t, 16-input group g, row i, rows fastest, so a wavefront's stores are runs of
// R x 16 contiguous bytes of the operand layout). Channels past the last and rows past the last get
// zero digits; their f32 values are not stored.
template <int R, int KMAX, int SL>
__global__ __launch_bounds__(1024) void dwconv_quant_kernel(const float *__restrict__ x, size_t ldx, int64_t frames,
                                                            int64_t total, int channels,
                                                            const float *__restrict__ w, int kernel,
                                                            const float *__restrict__ bias, int silu,
                                                            float *__restrict__ out, size_t ldo,
                                                            uint8_t *__restrict__ qa, int32_t *__restrict__ exps,
                                                            int kb, size_t bpx) {
    static_assert(16 % R == 0, "whole QA row blocks split evenly");
    constexpr int SPAN = R - 1 + KMAX, CWS = 1024 * SL + 4, WAVES = 16;
    __shared__ __attribute__((aligned(16))) float tile[R * CWS];
    __shared__ float s_max[WAVES][R];
    __shared__ int s_bad[WAVES];
    __shared__ int32_t s_e[R];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    // Workgroup L runs on XCD L % 8; each XCD takes a contiguous run of row groups.
    const size_t grp = (blockIdx.x % 8) * bpx + blockIdx.x / 8;
    const int64_t g0 = (int64_t)grp * R;
    if (g0 >= total) return;  // uniform over the workgroup
    const int half = kernel / 2;
    const int64_t first = g0 - half;  // the input row of window slot 0
    // The first row of each output row's sequence, as a window slot: lo[i] = start - first, in
    // [i + half + 1 - frames, i + half] (wave-uniform).
    int32_t lo[R];
    {
        int64_t s = (g0 / frames) * frames;
#pragma unroll
        for (int i = 0; i < R; i++) {
            while (g0 + i >= s + frames) s += frames;
            lo[i] = (int32_t)(s - first);
        }
    }
    // The whole window inside row 0's sequence: every row of the group is in it and every tap valid.
    const bool inner = lo[0] <= 0 && (R - 1) + (kernel - 1) < lo[0] + frames;
    float rmax[R];
#pragma unroll
    for (int i = 0; i < R; i++) rmax[i] = 0.0f;
    int rbad = 0;
#pragma unroll 1
    for (int sl = 0; sl < SL; sl++) {
        const int c = sl * 1024 + tid;
        const int cc = c < channels ? c : channels - 1;  // idle lanes load a valid column and store nothing
        float acc[R];
        {
            float v[SPAN], wr[KMAX];
#pragma unroll
            for (int s = 0; s < SPAN; s++) {
                const int64_t f = first + s;
                const int64_t fc = f < 0 ? 0 : (f >= total ? total - 1 : f);
                v[s] = x[(size_t)fc * ldx + cc];
            }
#pragma unroll
            for (int j = 0; j < KMAX; j++) wr[j] = w[(size_t)(j < kernel ? j : kernel - 1) * channels + cc];
            const float b = bias[cc];
#pragma unroll
            for (int i = 0; i < R; i++) acc[i] = b;
            if (inner) {
#pragma unroll
                for (int j = 0; j < KMAX; j++) {
                    if (j < kernel) {
#pragma unroll
                        for (int i = 0; i < R; i++) acc[i] = acc[i] + wr[j] * v[i + j];
                    }
                }
            } else {
#pragma unroll
                for (int j = 0; j < KMAX; j++) {
                    if (j < kernel) {
#pragma unroll
                        for (int i = 0; i < R; i++) {
                            const float nv = acc[i] + wr[j] * v[i + j];
                            acc[i] = (uint32_t)(i + j - lo[i]) < (uint32_t)frames ? nv : acc[i];
                        }
                    }
                }
            }
        }
#pragma unroll
        for (int i = 0; i < R; i++) {
            float o = acc[i];
            if (silu) o = o / (1.0f + exp_simd(0.0f - o));
            const bool ok = c < channels && g0 + i < total;
            tile[i * CWS + c] = ok ? o : 0.0f;
            if (ok) {
                if (out) out[(size_t)(g0 + i) * ldo + c] = o;
                rmax[i] = fmaxf(rmax[i], fabsf(o));
                rbad |= (!__builtin_isfinite(o)) << i;
            }
        }
    }
#pragma unroll
    for (int i = 0; i < R; i++) {
        const float m = wave_max(rmax[i]);
        if (lane == 0) s_max[wave][i] = m;
    }
    rbad = wave_or(rbad);
    if (lane == 0) s_bad[wave] = rbad;
    __syncthreads();
    if (tid < R) {
        float m = 0.0f;
        int b = 0;
#pragma unroll
        for (int q = 0; q < WAVES; q++) {
            m = fmaxf(m, s_max[q][tid]);
            b |= s_bad[q];
        }
        const bool valid = g0 + tid < total;
        const int32_t e = !valid ? 0 : (((b >> tid) & 1) ? EXP_NONFINITE : row_exponent_of(m));
        s_e[tid] = e;
        if (valid) exps[g0 + tid] = e;
    }
    __syncthreads();
    const size_t blk = (size_t)(g0 / 16);
    const int r0 = (int)(g0 % 16);
    for (int item = tid; item < 4 * R * kb; item += 1024) {
        const int i = item % R, g = (item / R) % 4, t = item / (4 * R);
        const float4 *src = reinterpret_cast<const float4 *>(tile + i * CWS + 64 * t + 16 * g);
        const int32_t e = s_e[i];
        uint32_t h[4], l[4];
#pragma unroll
        for (int q = 0; q < 4; q++) {
            const float4 a = src[q];
            digits4(a.x, a.y, a.z, a.w, e, h[q], l[q]);
        }
        uint8_t *dst = qa + ((blk * (size_t)kb + t) * 2) * 1024 + (16 * g + r0 + i) * 16;
        *reinterpret_cast<uint4 *>(dst) = make_uint4(h[0], h[1], h[2], h[3]);
        *reinterpret_cast<uint4 *>(dst + 1024) = make_uint4(l[0], l[1], l[2], l[3]);
    }
}

// The largest |o| of each of a lane's N rows (N a power of two up to 16) over the wavefront by
// recursive halving: at each step a lane keeps half of its rows, sends the other half to its
// partner and takes the partner's copy of the half it keeps (N - 1 + 6 - log2 N shuffles against
// 6 N for one reduction per row). On return m[0] of lane l is the wavefront's maximum of row
// sum_k b_(5-k) 2^(log2 N - 1 - k), b_i bit i of l (wave_max_row).
template <int N>
__device__ __forceinline__ void wave_max_rows(float (&m)[N], int lane) {
    static_assert(N >= 1 && N <= 16 && (N & (N - 1)) == 0, "a power of two up to 16");
#pragma unroll
    for (int h = N / 2, off = 32; h >= 1; h >>= 1, off >>= 1) {
        const bool up = lane & off;
#pragma unroll
        for (int k = 0; k < h; k++) {
            const float send = up ? m[k] : m[k + h];
            const float keep = up ? m[k + h] : m[k];
            m[k] = fmaxf(keep, __shfl_xor(send, off, 64));
        }
    }
    constexpr int LOG = N == 1 ? 0 : N == 2 ? 1 : N == 4 ? 2 : N == 8 ? 3 : 4;
#pragma unroll
    for (int off = 32 >> LOG; off >= 1; off >>= 1) m[0] = fmaxf(m[0], __shfl_xor(m[0], off, 64));
}

template <int N>
__device__ __forceinline__ int wave_max_row(int lane) {
    constexpr int LOG = N == 1 ? 0 : N == 2 ? 1 : N == 4 ? 2 : N == 8 ? 3 : 4;
    return (lane >> (6 - LOG)) & (N - 1);  // the top LOG bits of the lane, bit 5 the highest
}

// The taps of dwconv_quant_block_kernel for R output rows: acc[i] (starting at the bias) += w[j] *
// input slot i + j, for j in order. The input rows are read in batches of B, a batch's loads all
// issued before its first use, so the wavefront waits out the memory latency once per batch.
// FULL: every tap of every output lies inside the output's sequence and kernel = KMAX, so the taps
// are added unconditionally from the unclamped rows; otherwise rows are clamped to the input and a
// tap is skipped when its input row lies outside its output row's sequence or j >= kernel.
template <bool FULL, int R, int KMAX>
__device__ __forceinline__ void block_taps(float4 (&acc)[R], const float4 (&wr)[KMAX], const float *__restrict__ x,
                                           size_t ldx, int64_t first, int64_t total, int cc, int kernel,
                                           const int32_t (&lo)[R], int64_t frames) {
    constexpr int SPAN = R - 1 + KMAX, B = 8;
    const float *base = x + cc;
#pragma unroll
    for (int s0 = 0; s0 < SPAN; s0 += B) {
        float4 v[B];
#pragma unroll
        for (int u = 0; u < B; u++) {
            if (s0 + u < SPAN) {
                const int64_t f = first + s0 + u;
                const int64_t fc = FULL ? f : (f < 0 ? 0 : (f >= total ? total - 1 : f));
                v[u] = *reinterpret_cast<const float4 *>(base + (size_t)fc * ldx);
            }
        }
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int u = 0; u < B; u++) {
            const int sl = s0 + u;
            if (sl >= SPAN) break;
#pragma unroll
            for (int i = (sl - KMAX + 1 > 0 ? sl - KMAX + 1 : 0); i < (sl < R ? sl + 1 : R); i++) {
                const int j = sl - i;  // tap j of output i; taps of one output arrive in order
                if (FULL || (j < kernel && (uint32_t)(sl - lo[i]) < (uint32_t)frames)) {
                    acc[i].x = acc[i].x + wr[j].x * v[u].x;
                    acc[i].y = acc[i].y + wr[j].y * v[u].y;
                    acc[i].z = acc[i].z + wr[j].z * v[u].z;
                    acc[i].w = acc[i].w + wr[j].w * v[u].w;
                }
            }
        }
    }
}

// dwconv_quant_kernel for whole QA row blocks of 4 to 1024 channels (a multiple of 4) with 16-byte
// aligned rows, taps and bias, and kernel <= 9. Workgroup b takes output rows 16 b .. 16 b + 15:
// 16 / RT groups of W threads (W = 16 kb rounded up to whole wavefronts, kb the k-blocks of a
// row), thread j of group q taking channels 4 j .. 4 j + 3 of rows RT q .. RT q + RT - 1 (threads
// past the last channel hold zeros). The thread reads each of the RT + kernel - 1 input rows its
// outputs reach once (a 16-byte load) and adds it into the outputs it feeds, tap j of output i
// being input slot i + j, so every output still sums its taps in order from the bias (a tap
// outside its output row's sequence skipped); the outputs stay in registers (no LDS tile). After
// the SiLU, the row maxima and non-finite flags are reduced over the workgroup, each thread packs
// the digits of its four channels of each of its rows into LDS (rows 16 kb + 4 dwords apart: hi
// rows, then lo rows), and the workgroup copies the row block's QA bytes (kb x 2 KB, contiguous)
// out in 16-byte stores, consecutive lanes writing consecutive bytes. The same values, exponents
// and digits as dwconv_quant_kernel.
template <int RT, int KMAX>
__global__ __launch_bounds__(1024) void dwconv_quant_block_kernel(const float *__restrict__ x, size_t ldx,
                                                                  int64_t frames, int64_t total, int channels,
                                                                  const float *__restrict__ w, int kernel,
                                                                  const float *__restrict__ bias, int silu,
                                                                  float *__restrict__ out, size_t ldo,
                                                                  uint8_t *__restrict__ qa,
                                                                  int32_t *__restrict__ exps, int kb, size_t bpx) {
    constexpr int R = 16, G = R / RT;
    static_assert(R % RT == 0, "whole row groups");
    extern __shared__ __attribute__((aligned(16))) uint32_t stage[];  // [2][R][16 kb + 4]
    __shared__ float s_max[16][R];
    __shared__ int s_bad[16];
    __shared__ int32_t s_e[R];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int W = (int)(blockDim.x / G), wpg = W >> 6;  // threads and wavefronts per row group
    const int cq = tid % W, rq = tid / W;                // rq is wave-uniform
    const int rs = 16 * kb + 4;                          // staged row stride, dwords
    // Workgroup L runs on XCD L % 8; each XCD takes a contiguous run of row blocks.
    const size_t blk = (blockIdx.x % 8) * bpx + blockIdx.x / 8;
    const int64_t g0 = (int64_t)blk * R;
    if (g0 >= total) return;  // uniform over the workgroup
    const int64_t r0 = g0 + RT * rq;  // this thread's first output row
    const int half = kernel / 2;
    const int64_t first = r0 - half;  // the input row of window slot 0
    // The first row of each output row's sequence as a window slot (wave-uniform).
    int32_t lo[RT];
    {
        int64_t s = (r0 / frames) * frames;
#pragma unroll
        for (int i = 0; i < RT; i++) {
            while (r0 + i >= s + frames) s += frames;
            lo[i] = (int32_t)(s - first);
        }
    }
    const bool inner = lo[0] <= 0 && (RT - 1) + (kernel - 1) < lo[0] + frames;
    const int c = 4 * cq;
    const bool live = c < channels;
    const int cc = live ? c : channels - 4;  // idle lanes read valid channels and keep nothing
    float4 wr[KMAX];
#pragma unroll
    for (int j = 0; j < KMAX; j++)
        wr[j] = *reinterpret_cast<const float4 *>(w + (size_t)(j < kernel ? j : kernel - 1) * channels + cc);
    float4 acc[RT];
    {
        const float4 b = *reinterpret_cast<const float4 *>(bias + cc);
#pragma unroll
        for (int i = 0; i < RT; i++) acc[i] = b;
    }
    if (inner && kernel == KMAX)
        block_taps<true>(acc, wr, x, ldx, first, total, cc, kernel, lo, frames);
    else
        block_taps<false>(acc, wr, x, ldx, first, total, cc, kernel, lo, frames);
    float m[RT];
    int rbad = 0;
#pragma unroll
    for (int i = 0; i < RT; i++) {
        float4 o = acc[i];
        if (silu) {
            o.x = o.x / (1.0f + exp_simd(0.0f - o.x));
            o.y = o.y / (1.0f + exp_simd(0.0f - o.y));
            o.z = o.z / (1.0f + exp_simd(0.0f - o.z));
            o.w = o.w / (1.0f + exp_simd(0.0f - o.w));
        }
        const bool ok = live && r0 + i < total;
        if (ok && out) *reinterpret_cast<float4 *>(out + (size_t)(r0 + i) * ldo + c) = o;
        acc[i] = ok ? o : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        m[i] = fmaxf(fmaxf(fabsf(acc[i].x), fabsf(acc[i].y)), fmaxf(fabsf(acc[i].z), fabsf(acc[i].w)));
        const bool fin = __builtin_isfinite(acc[i].x) && __builtin_isfinite(acc[i].y) &&
                         __builtin_isfinite(acc[i].z) && __builtin_isfinite(acc[i].w);
        rbad |= (int)!fin << i;
    }
    wave_max_rows<RT>(m, lane);
    rbad = wave_or(rbad);
    {
        constexpr int LOG = RT == 1 ? 0 : RT == 2 ? 1 : RT == 4 ? 2 : RT == 8 ? 3 : 4;
        if ((lane & ((64 >> LOG) - 1)) == 0) s_max[wave][RT * rq + wave_max_row<RT>(lane)] = m[0];
    }
    if (lane == 0) s_bad[wave] = rbad;
    __syncthreads();
    if (tid < R) {
        // row tid: the wavefronts of its row group
        const int q0 = (tid / RT) * wpg;
        float mx = 0.0f;
        int b = 0;
        for (int q = q0; q < q0 + wpg; q++) {
            mx = fmaxf(mx, s_max[q][tid]);
            b |= s_bad[q];
        }
        const bool valid = g0 + tid < total;
        const int32_t e = !valid ? 0 : (((b >> (tid % RT)) & 1) ? EXP_NONFINITE : row_exponent_of(mx));
        s_e[tid] = e;
        if (valid) exps[g0 + tid] = e;
    }
    __syncthreads();
    if (cq < 16 * kb) {
#pragma unroll
        for (int i = 0; i < RT; i++) {
            const int row = RT * rq + i;
            uint32_t h, l;
            digits4(acc[i].x, acc[i].y, acc[i].z, acc[i].w, s_e[row], h, l);
            stage[row * rs + cq] = h;
            stage[(R + row) * rs + cq] = l;
        }
    }
    __syncthreads();
    // Chunk q of the row block's QA bytes (16 bytes at q * 16): k-block t = q / 128, digit
    // d = q / 64 % 2, 16-input group g = q / 16 % 4, row r = q % 16.
    uint8_t *dst = qa + (size_t)blk * kb * 2048;
    for (int q = tid; q < 128 * kb; q += blockDim.x) {
        const int r = q & 15, g = (q >> 4) & 3, d = (q >> 6) & 1, t = q >> 7;
        const uint4 v = *reinterpret_cast<const uint4 *>(stage + (d * R + r) * rs + 16 * t + 4 * g);
        *reinterpret_cast<uint4 *>(dst + (size_t)q * 16) = v;
    }
}

bool dwconv_quant_fits(size_t channels, size_t kernel) {
    return channels >= 1 && channels <= 2048 && kernel >= 1 && kernel <= 32;
}

// Rows below which the four-row workgroups take the call (fewer than two 16-row workgroups per CU).
constexpr size_t DQ_SMALL = 8192;
// Rows from which dwconv_quant_block_kernel takes the calls it fits, and from which it runs eight
// rows per thread (two workgroups per CU) rather than four (one). 1024 x 9 taps with SiLU, in us:
//   rows         750   1500   3000   7500   12000
//   row slices   8.5   12.3   17.7   36.4    58.6   (dwconv_quant_kernel)
//   4 per thread 10.1  10.7   11.7   22.5    33.3
//   8 per thread 11.1  12.6   13.7   21.5    30.7
constexpr size_t DQ_BLOCK_ROWS = 1024, DQ_RT8_ROWS = 6144;

hipError_t launch_dwconv_quant(const float *x, size_t ldx, size_t frames, size_t batch, size_t channels,
                               const float *w, size_t kernel, const float *bias, int silu, float *out, size_t ldo,
                               uint8_t *qa, int32_t *exps, hipStream_t s) {
    const size_t total = frames * batch;
    if (total == 0 || channels == 0) return hipSuccess;
    if (!dwconv_quant_fits(channels, kernel)) return hipErrorInvalidValue;
    const size_t kb = div_ceil(channels, (size_t)KBLK);
    const bool aligned = ((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(w) |
                           reinterpret_cast<uintptr_t>(bias) | reinterpret_cast<uintptr_t>(out)) % 16) == 0 &&
                         ldx % 4 == 0 && (!out || ldo % 4 == 0);
    if (total >= DQ_BLOCK_ROWS && kernel <= 9 && channels % 4 == 0 && channels <= 1024 && aligned) {
        const size_t bpx = div_ceil(div_ceil(total, (size_t)16), (size_t)8);
        const size_t lds = 2 * 16 * (16 * kb + 4) * sizeof(uint32_t);  // at most 33 KB
        const unsigned wg = (unsigned)div_ceil(16 * kb, (size_t)64) * 64;  // a row group, whole wavefronts
        if (total >= DQ_RT8_ROWS)
            hipLaunchKernelGGL((dwconv_quant_block_kernel<8, 9>), dim3((unsigned)(8 * bpx)), dim3(2 * wg), lds, s, x,
                               ldx, (int64_t)frames, (int64_t)total, (int)channels, w, (int)kernel, bias, silu, out,
                               ldo, qa, exps, (int)kb, bpx);
        else
            hipLaunchKernelGGL((dwconv_quant_block_kernel<4, 9>), dim3((unsigned)(8 * bpx)), dim3(4 * wg), lds, s, x,
                               ldx, (int64_t)frames, (int64_t)total, (int)channels, w, (int)kernel, bias, silu, out,
                               ldo, qa, exps, (int)kb, bpx);
        return hipGetLastError();
    }
    const size_t rows = total < DQ_SMALL ? 4 : 16;
    const size_t bpx = div_ceil(div_ceil(total, rows), (size_t)8);
    const dim3 grid((unsigned)(8 * bpx));
#define TG_DQ(R_, KM, SL_)                                                                                       \
    hipLaunchKernelGGL((dwconv_quant_kernel<R_, KM, SL_>), grid, dim3(1024), 0, s, x, ldx, (int64_t)frames,       \
                       (int64_t)total, (int)channels, w, (int)kernel, bias, silu, out, ldo, qa, exps, (int)kb, bpx)
#define TG_DQ_K(R_, SL_)                         \
    do {                                         \
        if (kernel <= 9) TG_DQ(R_, 9, SL_);      \
        else if (kernel <= 16) TG_DQ(R_, 16, SL_); \
        else TG_DQ(R_, 32, SL_);                 \
    } while (0)
    if (rows == 4) {
        if (channels <= 1024) TG_DQ_K(4, 1);
        else TG_DQ_K(4, 2);
    } else {
        if (channels <= 1024) TG_DQ_K(16, 1);
        else TG_DQ_K(16, 2);
    }
#undef TG_DQ_K
#undef TG_DQ
    return hipGetLastError();
}

hipError_t launch_dwconv1d(const float *x, size_t ldx, size_t frames, size_t batch, size_t channels, const float *w,
                           size_t kernel, const float *bias, size_t t0, size_t stride, size_t rows, int silu,
                           float *out, size_t ldo, hipStream_t s) {
    if (rows == 0 || channels == 0 || batch == 0) return hipSuccess;
    // the register window needs a frame to clamp to and at least one tap
    if (frames > 0 && kernel > 0 && (stride == 1 || stride == 2) && kernel <= 32) {
        if (stride == 1) {
            if (kernel <= 9)
                launch_dwconv_reg<16, 1, 9>(x, ldx, frames, batch, channels, w, kernel, bias, t0, rows, silu, out, ldo, s);
            else if (kernel <= 16)
                launch_dwconv_reg<16, 1, 16>(x, ldx, frames, batch, channels, w, kernel, bias, t0, rows, silu, out, ldo,
                                             s);
            else
                launch_dwconv_reg<16, 1, 32>(x, ldx, frames, batch, channels, w, kernel, bias, t0, rows, silu, out, ldo,
                                             s);
        } else {
            if (kernel <= 9)
                launch_dwconv_reg<16, 2, 9>(x, ldx, frames, batch, channels, w, kernel, bias, t0, rows, silu, out, ldo, s);
            else if (kernel <= 16)
                launch_dwconv_reg<16, 2, 16>(x, ldx, frames, batch, channels, w, kernel, bias, t0, rows, silu, out, ldo,
                                             s);
            else
                launch_dwconv_reg<8, 2, 32>(x, ldx, frames, batch, channels, w, kernel, bias, t0, rows, silu, out, ldo, s);
        }
        return hipGetLastError();
    }
    // row tiles along x, 256-channel slices along y, sequences along z (the host keeps y, z < 65536)
    const dim3 grid((unsigned)div_ceil(rows, (size_t)DW_ROWS), (unsigned)div_ceil(channels, (size_t)256),
                    (unsigned)batch);
    hipLaunchKernelGGL(dwconv1d_kernel, grid, dim3(256), 0, s, x, ldx, (int64_t)frames, channels, w, (int)kernel, bias,
                       (int64_t)t0, (int64_t)stride, rows, silu, out, ldo);
    return hipGetLastError();
}

}  // namespace tg
