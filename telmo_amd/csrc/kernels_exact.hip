// The exact kernel: the reference's fused arithmetic on the GPU, for validation and for callers
// that need bit-identity with telmo's SIMD CPU kernels.
//
// One lane per output sums acc = fmaf(a[r][i], widen(w)[o][i], acc) for i = 0..k-1 in order
// (src/kernels/avx512.rs:70-105 and 156-213: input-order fused sums), with widen as
// src/kernels/scalar.rs:54-107 (int8: one rounded product q * scale), then the shared epilogue,
// which uses the reference's SIMD exp. Any precision; weights in the device layout.
#include "tg_internal.hpp"

namespace tg {

namespace {

__device__ __forceinline__ float half_to_float(uint16_t h) {
    const uint32_t sign = (uint32_t)(h & 0x8000) << 16;
    const uint32_t exp = (h >> 10) & 0x1f, man = h & 0x3ff;
    if (exp == 0) {
        if (man == 0) return __uint_as_float(sign);
        const float v = (float)man * (1.0f / 16777216.0f);
        return sign ? -v : v;
    }
    if (exp == 0x1f) return __uint_as_float(sign | 0x7f800000u | (man ? 0x400000u | (man << 13) : 0u));
    return __uint_as_float(sign | ((exp + 112) << 23) | (man << 13));
}

__device__ __forceinline__ float widen_one(const uint8_t *__restrict__ wv, const float *__restrict__ scales,
                                           uint32_t prec, size_t k, size_t ps, size_t bs, size_t p, int j, size_t i) {
    switch (prec) {
    case F32: return reinterpret_cast<const float *>(wv)[(p * k + i) * PANEL + j];
    case F16: return half_to_float(reinterpret_cast<const uint16_t *>(wv)[(p * k + i) * PANEL + j]);
    case BF16: return __uint_as_float((uint32_t)reinterpret_cast<const uint16_t *>(wv)[(p * k + i) * PANEL + j] << 16);
    default: {
        const size_t t = i / KBLK, g = (i % KBLK) / 16, ii = i % 16;
        const int8_t q = (int8_t)wv[p * ps + t * bs + (g * 16 + j) * 16 + ii];
        const float s = prec == INT8 ? scales[p * PANEL + j]
                                     : scales[(p * div_ceil(k, Q8_BLOCK) + i / Q8_BLOCK) * PANEL + j];
        return (float)q * s;
    }
    }
}

__global__ __launch_bounds__(256) void exact_kernel(const float *__restrict__ a, size_t lda, int m, int k,
                                                    const uint8_t *__restrict__ wv, const float *__restrict__ scales,
                                                    uint32_t prec, int N, size_t ps, size_t bs, float *__restrict__ c,
                                                    size_t ldc, const float *__restrict__ bias, uint32_t act,
                                                    float escale, int accumulate) {
    const int col = blockIdx.x * 64 + (threadIdx.x & 63);
    const int row = blockIdx.y * 4 + (threadIdx.x >> 6);
    if (row >= m || col >= N) return;
    const size_t p = col / PANEL;
    const int j = col % PANEL;
    const float *ar = a + (size_t)row * lda;
    float acc = 0.0f;
    for (int i = 0; i < k; i++) acc = __builtin_fmaf(ar[i], widen_one(wv, scales, prec, k, ps, bs, p, j, i), acc);
    float *cp = c + (size_t)row * ldc + col;
    *cp = epilogue(acc, bias, (size_t)col, act, escale, accumulate != 0, cp);
}

// The accuracy guard's fix-up (RowGuard): the exact kernel's sums and epilogue for the flagged rows
// of a product the fast path has just written, over every output column. Workgroup (x, y) takes the
// 64 columns 64 x .. and the rows of chunk y; its wavefronts read the chunk's flags 64 at a time and
// take the flagged rows in turn (wavefront w the w-th, w + 4-th, ... of each group of 64). A flagged
// row's old outputs come from save (kept by the quantiser) when the epilogue accumulates.
__global__ __launch_bounds__(256) void exact_rows_kernel(const float *__restrict__ a, size_t lda, int m, int k,
                                                         const uint8_t *__restrict__ wv,
                                                         const float *__restrict__ scales, uint32_t prec, int N,
                                                         size_t ps, size_t bs, float *__restrict__ c, size_t ldc,
                                                         const float *__restrict__ bias, uint32_t act, float escale,
                                                         int accumulate, const int32_t *__restrict__ flags,
                                                         const float *__restrict__ save, int chunk) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int col = blockIdx.x * 64 + lane;
    const int r0 = blockIdx.y * chunk, r1 = min(m, r0 + chunk);
    const size_t p = (size_t)(col < N ? col : N - 1) / PANEL;
    const int j = (col < N ? col : N - 1) % PANEL;
    for (int base = r0; base < r1; base += 64) {
        const int f = base + lane < r1 ? flags[base + lane] : 0;
        uint64_t mask = __ballot(f != 0);
        for (int nth = 0; mask; nth++, mask &= mask - 1) {
            if ((nth & 3) != wave) continue;
            const int row = base + __builtin_ctzll(mask);
            if (col >= N) continue;
            const float *ar = a + (size_t)row * lda;
            float acc = 0.0f;
            for (int i = 0; i < k; i++)
                acc = __builtin_fmaf(ar[i], widen_one(wv, scales, prec, k, ps, bs, p, j, i), acc);
            const float old = accumulate ? save[(size_t)row * N + col] : 0.0f;
            c[(size_t)row * ldc + col] = epilogue_vals(acc, bias != nullptr, bias ? bias[col] : 0.0f, act, escale,
                                                       accumulate != 0, old);
        }
    }
}

// BView::row_major as the right-hand side (src/kernels/mod.rs:320-339): column col of input i is
// b[i ldb + col], read straight from the row-major f32 matrix, summed as the exact kernel sums.
__global__ __launch_bounds__(256) void rowmajor_kernel(const float *__restrict__ a, size_t lda, int m, int k,
                                                       const float *__restrict__ b, size_t ldb, int N,
                                                       float *__restrict__ c, size_t ldc, const float *__restrict__ bias,
                                                       uint32_t act, float escale, int accumulate) {
    const int col = blockIdx.x * 64 + (threadIdx.x & 63);
    const int row = blockIdx.y * 4 + (threadIdx.x >> 6);
    if (row >= m || col >= N) return;
    const float *ar = a + (size_t)row * lda;
    float acc = 0.0f;
    for (int i = 0; i < k; i++) acc = __builtin_fmaf(ar[i], b[(size_t)i * ldb + col], acc);
    float *cp = c + (size_t)row * ldc + col;
    *cp = epilogue(acc, bias, (size_t)col, act, escale, accumulate != 0, cp);
}

}  // namespace

hipError_t launch_rowmajor(const float *a, size_t lda, size_t m, size_t k, const float *b, size_t ldb, size_t n,
                           float *c, size_t ldc, const EpiArgs &epi, hipStream_t s) {
    if (m == 0 || n == 0) return hipSuccess;
    dim3 grid((unsigned)div_ceil(n, 64), (unsigned)div_ceil(m, 4));
    hipLaunchKernelGGL(rowmajor_kernel, grid, dim3(256), 0, s, a, lda, (int)m, (int)k, b, ldb, (int)n, c, ldc, epi.bias,
                       epi.act, epi.scale, epi.accumulate);
    return hipGetLastError();
}

hipError_t launch_exact(const float *a, size_t lda, size_t m, const DeviceWeights &w, float *c, size_t ldc,
                        const EpiArgs &epi, hipStream_t s) {
    if (m == 0 || w.n == 0) return hipSuccess;
    dim3 grid((unsigned)div_ceil(w.n, 64), (unsigned)div_ceil(m, 4));
    hipLaunchKernelGGL(exact_kernel, grid, dim3(256), 0, s, a, lda, (int)m, (int)w.k, w.values, w.scales,
                       w.precision, (int)w.n, w.panel_stride, w.blk_stride, c, ldc, epi.bias, epi.act, epi.scale,
                       epi.accumulate);
    return hipGetLastError();
}

hipError_t launch_exact_rows(const float *a, size_t lda, size_t m, const DeviceWeights &w, float *c, size_t ldc,
                             const EpiArgs &epi, const int32_t *flags, const float *save, hipStream_t s) {
    if (m == 0 || w.n == 0) return hipSuccess;
    // About 2048 workgroups: the column groups times row chunks of whole groups of 64 rows.
    const size_t cols = div_ceil(w.n, 64), groups = div_ceil(m, 64);
    size_t chunks = 2048 / cols;
    chunks = chunks < 1 ? 1 : (chunks > groups ? groups : chunks);
    const size_t chunk = div_ceil(groups, chunks) * 64;
    dim3 grid((unsigned)cols, (unsigned)div_ceil(m, chunk));
    hipLaunchKernelGGL(exact_rows_kernel, grid, dim3(256), 0, s, a, lda, (int)m, (int)w.k, w.values, w.scales,
                       w.precision, (int)w.n, w.panel_stride, w.blk_stride, c, ldc, epi.bias, epi.act, epi.scale,
                       epi.accumulate, flags, save, (int)chunk);
    return hipGetLastError();
}

}  // namespace tg
