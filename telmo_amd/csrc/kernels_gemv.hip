// The decode-step GEMVs (m = 1..16 rows) over int8 weights: HBM-bound streams of the weights.
//
// Both kernels split their rows into two int8 digits in LDS themselves (the same digits and
// exponents as the GEMM path, so a row gives bit-identical outputs on every path) and read the
// weights in the MFMA layout: per k-block of 64 inputs of a 16-output panel, lane l = 16 g + j
// loads 16 contiguous bytes (inputs 64 t + 16 g + [0, 16) of output j), 1 KB per wave, coalesced.
//
// gemv_mfma_kernel (m <= 16, k <= 1984, 16-byte aligned rows, k % 4 == 0; one int8 row takes its
// dot4 body, no MFMA): the digits sit in LDS as 16 x 64 MFMA A operands in lane
// order, so each 1 KB weight block costs one 16-byte LDS read per digit and two
// v_mfma_i32_16x16x64_i8, whatever m is. The rows are read once into registers ahead of the
// weights; workgroups stay resident and walk the panels, so the rows are digitised once per
// workgroup, and the next panel's weights, scales, bias and old outputs are requested before the
// current panel's epilogue.
//
// gemv_i8_kernel (m <= 8, other rows): one panel per wavefront, v_dot4_i32_i8 against each
// row's digits; the four input groups meet by lane exchanges (xor 16, xor 32).
#include "gemv_core.hpp"

namespace tg {

namespace {

constexpr int THREADS = 256;
constexpr size_t GEMV_LDS_BUDGET = 64 * 1024 - 256;  // the rest of 64 KB holds the exponents

__device__ __forceinline__ float wave_max(float v) {
    for (int off = 32; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, 64));
    return v;
}

__device__ __forceinline__ int wave_or(int v) {
    for (int off = 32; off > 0; off >>= 1) v |= __shfl_xor(v, off, 64);
    return v;
}

using gemv::v4f;
using gemv::v4i;

// One weight panel (16 outputs) per wavefront. The panel's first KBC k-blocks are requested
// before anything else, so their HBM latency overlaps the workgroup's quantisation of the rows
// into LDS; longer rows continue in chunks of KBC k-blocks.
template <int MR, int KBC>
__global__ __launch_bounds__(THREADS) void gemv_i8_kernel(const float *__restrict__ a, size_t lda, int k,
                                                          const uint8_t *__restrict__ wv,
                                                          const float *__restrict__ scales, int N, int P, int KB,
                                                          float *__restrict__ c, size_t ldc,
                                                          const float *__restrict__ bias, uint32_t act, float escale,
                                                          int accumulate, size_t panel_stride, size_t blk_stride) {
    extern __shared__ __attribute__((aligned(16))) uint8_t sqa[];  // MR rows x KB x 128 bytes
    __shared__ int32_t sexp[MR];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const size_t row_bytes = (size_t)KB * 128;
    const int p = blockIdx.x * (THREADS / 64) + wave;
    const uint8_t *wp = wv + (size_t)min(p, P - 1) * panel_stride + lane * 16;

    v4i wr[KBC];
    if (KB > 0) {
#pragma unroll
        for (int t = 0; t < KBC; t++) wr[t] = *reinterpret_cast<const v4i *>(wp + (size_t)min(t, KB - 1) * blk_stride);
    }

    // Digits of the rows, one wavefront per row.
    for (int r = wave; r < MR; r += THREADS / 64) {
        const float *ar = a + (size_t)r * lda;
        float amax = 0.0f;
        int bad = 0;
        for (int i = lane; i < k; i += 64) {
            const float x = ar[i];
            bad |= !__builtin_isfinite(x);
            amax = fmaxf(amax, fabsf(x));
        }
        amax = wave_max(amax);
        bad = wave_or(bad);
        const int32_t e = bad ? EXP_NONFINITE : row_exponent_of(amax);
        if (lane == 0) sexp[r] = e;
        uint8_t *q = sqa + r * row_bytes;
        for (int t = 0; t < KB; t++) {
            const int i = t * KBLK + lane;
            int8_t hi = 0, lo = 0;
            if (i < k) digits_of(ar[i], e, hi, lo);
            q[t * 128 + lane] = (uint8_t)hi;
            q[t * 128 + 64 + lane] = (uint8_t)lo;
        }
    }
    __syncthreads();

    const int g = lane >> 4, j = lane & 15;
    int acc[MR][2];
#pragma unroll
    for (int r = 0; r < MR; r++) acc[r][0] = acc[r][1] = 0;
    for (int c0 = 0; c0 < KB; c0 += KBC) {
        if (c0 > 0) {
#pragma unroll
            for (int t = 0; t < KBC; t++)
                wr[t] = *reinterpret_cast<const v4i *>(wp + (size_t)min(c0 + t, KB - 1) * blk_stride);
        }
#pragma unroll
        for (int t = 0; t < KBC; t++) {
            if (c0 + t < KB) {
#pragma unroll
                for (int r = 0; r < MR; r++) {
                    const uint8_t *ap = sqa + r * row_bytes + (c0 + t) * 128 + g * 16;
                    const v4i ahi = *reinterpret_cast<const v4i *>(ap);
                    const v4i alo = *reinterpret_cast<const v4i *>(ap + 64);
                    int h = acc[r][0], l = acc[r][1];
                    h = __builtin_amdgcn_sdot4(ahi.x, wr[t].x, h, false);
                    h = __builtin_amdgcn_sdot4(ahi.y, wr[t].y, h, false);
                    h = __builtin_amdgcn_sdot4(ahi.z, wr[t].z, h, false);
                    h = __builtin_amdgcn_sdot4(ahi.w, wr[t].w, h, false);
                    l = __builtin_amdgcn_sdot4(alo.x, wr[t].x, l, false);
                    l = __builtin_amdgcn_sdot4(alo.y, wr[t].y, l, false);
                    l = __builtin_amdgcn_sdot4(alo.z, wr[t].z, l, false);
                    l = __builtin_amdgcn_sdot4(alo.w, wr[t].w, l, false);
                    acc[r][0] = h;
                    acc[r][1] = l;
                }
            }
        }
    }
    // Sum over the four 16-input groups (lanes j, j + 16, j + 32, j + 48).
#pragma unroll
    for (int r = 0; r < MR; r++)
#pragma unroll
        for (int d = 0; d < 2; d++) {
            int v = acc[r][d];
            v += __shfl_xor(v, 16, 64);
            v += __shfl_xor(v, 32, 64);
            acc[r][d] = v;
        }
    const int col = p * PANEL + j;
    if (g == 0 && p < P && col < N) {
        const float sc = scales[col];
#pragma unroll
        for (int r = 0; r < MR; r++) {
            float *cp = c + (size_t)r * ldc + col;
            const float s = dequant(acc[r][0], acc[r][1], sexp[r], sc);
            *cp = epilogue(s, bias, (size_t)col, act, escale, accumulate != 0, cp);
        }
    }
}

template <int MR>
hipError_t launch_rows(const float *a, size_t lda, const DeviceWeights &w, float *c, size_t ldc, const EpiArgs &epi,
                       hipStream_t s) {
    const size_t blocks = div_ceil(w.panels, THREADS / 64);
    const size_t lds = (size_t)MR * w.kb * 128;
#define TG_GEMV(KBC)                                                                                     \
    hipLaunchKernelGGL((gemv_i8_kernel<MR, KBC>), dim3((unsigned)blocks), dim3(THREADS), lds, s, a, lda,  \
                       (int)w.k, w.values, w.scales, (int)w.n, (int)w.panels, (int)w.kb, c, ldc, epi.bias,  \
                       epi.act, epi.scale, epi.accumulate, w.panel_stride, w.blk_stride)
    if (w.kb <= 10) TG_GEMV(10);
    else TG_GEMV(20);
#undef TG_GEMV
    return hipGetLastError();
}


// Rows are read from a (row stride lda), outputs written to c: the GEMV of tg_matmul_device.
template <int WAVES, int KBC, int J, int Q8, int DOTR, int KS>
__global__ __launch_bounds__(WAVES * 64) void gemv_mfma_kernel(const float *__restrict__ a, size_t lda, int m, int k,
                                                               const uint8_t *__restrict__ wv,
                                                               const float *__restrict__ scales, int N, int P, int KB,
                                                               int NB, float *__restrict__ c, size_t ldc,
                                                               const float *__restrict__ bias, uint32_t act,
                                                               float escale, int accumulate, size_t panel_stride,
                                                               size_t blk_stride) {
    extern __shared__ __attribute__((aligned(16))) uint8_t sqa[];  // KB x (hi, lo) x 1 KB operands
    __shared__ uint32_t slot[WAVES * J];                           // max |x| bits per wavefront of chunks
    gemv::StoreC out{c, ldc};
    gemv::mfma_body<WAVES, KBC, J, Q8, gemv::RowsIn, gemv::StoreC, DOTR, KS>(gemv::RowsIn{a, lda}, out, m, k, wv,
                                                                          scales, N, P, KB, NB, c, ldc, bias, act,
                                                                          escale, accumulate, panel_stride,
                                                                          blk_stride, sqa, slot);
}

// A single decode row (m = 1, int8 weights) takes the dot4 variant of the body: the same row, panels
// and epilogue, with v_dot4_i32_i8 in place of the MFMA and the four input groups summed across the
// wavefront. From two rows on, the dot4 form is bound by its LDS operand reads and VALU work (each
// row adds two 16-byte LDS reads and eight v_dot4 per 1 KB of weights, where one MFMA pair serves
// up to 16 rows), so batches of streams take the MFMA.
bool gemv_dot_rows(size_t m) { return m == 1; }

constexpr int MFMA_MAX_KB = 31;       // digits within 62 KB of LDS
constexpr size_t MFMA_MAX_WAVE_ROWS = 64;  // m * ceil(KB / 4): chunk wavefronts, at most 16 per thread of 256
constexpr size_t MFMA_MAX_GRID = 1024;     // four resident workgroups per CU; more panels are walked

// The MFMA GEMV reads rows with 16-byte loads: rows 16-byte aligned, k a multiple of 4.
bool mfma_fits(size_t m, size_t k, const float *a, size_t lda) {
    const size_t kb = div_ceil(k, KBLK);
    return m >= 1 && m <= GEMV_MAX_ROWS && kb >= 1 && kb <= (size_t)MFMA_MAX_KB &&
           m * div_ceil(kb, (size_t)4) <= MFMA_MAX_WAVE_ROWS && reinterpret_cast<uintptr_t>(a) % 16 == 0 &&
           lda % 4 == 0 && k % 4 == 0;
}

template <int WAVES, int KBC, int J, int KS>
void launch_mfma_t(const float *a, size_t lda, size_t m, const DeviceWeights &w, float *c, size_t ldc,
                   const EpiArgs &epi, size_t blocks, bool dot, hipStream_t s) {
    void (*kernel)(const float *, size_t, int, int, const uint8_t *, const float *, int, int, int, int, float *,
                   size_t, const float *, uint32_t, float, int, size_t, size_t);
    if constexpr (KS > 1) kernel = dot ? gemv_mfma_kernel<WAVES, KBC, J, 0, 1, KS> : gemv_mfma_kernel<WAVES, KBC, J, 0, 0, KS>;
    else if (w.precision == Q8_0) kernel = gemv_mfma_kernel<WAVES, KBC, J, 1, 0, 1>;
    else kernel = dot ? gemv_mfma_kernel<WAVES, KBC, J, 0, 1, 1> : gemv_mfma_kernel<WAVES, KBC, J, 0, 0, 1>;
    hipLaunchKernelGGL(kernel, dim3((unsigned)blocks), dim3(WAVES * 64), w.kb * 2048, s, a, lda, (int)m, (int)w.k,
                       w.values, w.scales, (int)w.n, (int)w.panels, (int)w.kb, (int)(w.k / Q8_BLOCK), c, ldc, epi.bias,
                       epi.act, epi.scale, epi.accumulate, w.panel_stride, w.blk_stride);
}

template <int WAVES, int KBC, int KS>
void launch_mfma_j(size_t j, const float *a, size_t lda, size_t m, const DeviceWeights &w, float *c,
                   size_t ldc, const EpiArgs &epi, size_t blocks, bool dot, hipStream_t s) {
    if (j <= 1) launch_mfma_t<WAVES, KBC, 1, KS>(a, lda, m, w, c, ldc, epi, blocks, dot, s);
    else if (j <= 2) launch_mfma_t<WAVES, KBC, 2, KS>(a, lda, m, w, c, ldc, epi, blocks, dot, s);
    else if (j <= 3) launch_mfma_t<WAVES, KBC, 3, KS>(a, lda, m, w, c, ldc, epi, blocks, dot, s);
    else if (j <= 4) launch_mfma_t<WAVES, KBC, 4, KS>(a, lda, m, w, c, ldc, epi, blocks, dot, s);
    else if (j <= 6) launch_mfma_t<WAVES, KBC, 6, KS>(a, lda, m, w, c, ldc, epi, blocks, dot, s);
    else if (j <= 8) launch_mfma_t<WAVES, KBC, 8, KS>(a, lda, m, w, c, ldc, epi, blocks, dot, s);
    else if (j <= 12) launch_mfma_t<WAVES, KBC, 12, KS>(a, lda, m, w, c, ldc, epi, blocks, dot, s);
    else launch_mfma_t<WAVES, KBC, 16, KS>(a, lda, m, w, c, ldc, epi, blocks, dot, s);
}

hipError_t launch_mfma(const float *a, size_t lda, size_t m, const DeviceWeights &w, float *c, size_t ldc,
                       const EpiArgs &epi, hipStream_t s) {
    const size_t chunks = m * div_ceil(w.kb, (size_t)4) * 64;
    const bool dot = gemv_dot_rows(m) && w.precision == INT8;
    if (w.precision == INT8 && w.panels <= MFMA_MAX_GRID && m <= 8) {
        // Few panels: one workgroup of four wavefronts per panel, its k-blocks split four ways, so
        // that four times the SIMDs stream the weights and each walks a quarter of the row. (Past
        // eight rows, digitising the rows once per panel costs more than the split saves.)
        const size_t j = div_ceil(chunks, (size_t)256), kq = div_ceil(w.kb, (size_t)4);
        if (j > 16) return hipErrorInvalidValue;  // excluded by mfma_fits
        if (kq <= 3) launch_mfma_j<4, 3, 4>(j, a, lda, m, w, c, ldc, epi, w.panels, dot, s);
        else if (kq <= 5) launch_mfma_j<4, 5, 4>(j, a, lda, m, w, c, ldc, epi, w.panels, dot, s);
        else launch_mfma_j<4, 8, 4>(j, a, lda, m, w, c, ldc, epi, w.panels, dot, s);
        return hipGetLastError();
    }
    // Two-wave workgroups for short products, so they spread over more CUs.
    int waves = w.panels < 1024 ? 2 : 4;
    size_t j = div_ceil(chunks, (size_t)waves * 64);
    if (j > 16) {
        waves = 4;
        j = div_ceil(chunks, (size_t)256);
    }
    if (j > 16) return hipErrorInvalidValue;  // excluded by mfma_fits
    const size_t per_wave = div_ceil(w.panels, (size_t)waves * MFMA_MAX_GRID);
    const size_t blocks = div_ceil(w.panels, (size_t)waves * per_wave);
    if (waves == 2) {
        if (w.kb <= 10) launch_mfma_j<2, 10, 1>(j, a, lda, m, w, c, ldc, epi, blocks, dot, s);
        else launch_mfma_j<2, 16, 1>(j, a, lda, m, w, c, ldc, epi, blocks, dot, s);
    } else {
        if (w.kb <= 10) launch_mfma_j<4, 10, 1>(j, a, lda, m, w, c, ldc, epi, blocks, dot, s);
        else launch_mfma_j<4, 16, 1>(j, a, lda, m, w, c, ldc, epi, blocks, dot, s);
    }
    return hipGetLastError();
}

}  // namespace

bool gemv_fits(size_t m, size_t k, const float *a, size_t lda, uint32_t precision) {
    const size_t kb = div_ceil(k, KBLK);
    if (m == 0 || k == 0) return false;
    if (mfma_fits(m, k, a, lda)) return true;
    return precision == INT8 && m <= 8 && m * kb * 128 <= GEMV_LDS_BUDGET;  // the dot4 GEMV is int8 only
}

hipError_t launch_gemv_i8(const float *a, size_t lda, size_t m, const DeviceWeights &w, float *c, size_t ldc,
                          const EpiArgs &epi, hipStream_t s) {
    if (m == 0 || w.n == 0) return hipSuccess;
    if (mfma_fits(m, w.k, a, lda)) return launch_mfma(a, lda, m, w, c, ldc, epi, s);
    if (w.precision != INT8) return hipErrorInvalidValue;  // excluded by gemv_fits
    switch (m) {
    case 1: return launch_rows<1>(a, lda, w, c, ldc, epi, s);
    case 2: return launch_rows<2>(a, lda, w, c, ldc, epi, s);
    case 3: return launch_rows<3>(a, lda, w, c, ldc, epi, s);
    case 4: return launch_rows<4>(a, lda, w, c, ldc, epi, s);
    case 5: return launch_rows<5>(a, lda, w, c, ldc, epi, s);
    case 6: return launch_rows<6>(a, lda, w, c, ldc, epi, s);
    case 7: return launch_rows<7>(a, lda, w, c, ldc, epi, s);
    case 8: return launch_rows<8>(a, lda, w, c, ldc, epi, s);
    default: return hipErrorInvalidValue;
    }
}

}  // namespace tg
