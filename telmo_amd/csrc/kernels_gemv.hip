// The decode-step GEMV (m = 1..8 rows) over int8 weights: bandwidth-bound, no MFMA.
//
// Each workgroup first splits its m activation rows into two int8 digits in LDS (the same
// digits and exponents as the GEMM path, so a row gives bit-identical outputs on either path).
// Each wavefront then streams groups of 4 weight panels (64 outputs) in the MFMA layout: per
// k-block of 64 inputs, lane l = 16 g + j loads 16 contiguous bytes per panel (the inputs
// 64 t + 16 g + [0, 16) of output j), a fully coalesced 1 KB per panel per wave, and sums them
// against the digits with v_dot4_i32_i8 (4 products per lane-op, exact in i32). After the k loop a
// two-step reduce-scatter over g (lane xor 32, then xor 16) leaves lane (g, j) the full sums of
// output j of panel g, and the 64 lanes store 64 contiguous outputs per row.
#include "tg_internal.hpp"

namespace tg {

namespace {

constexpr int THREADS = 256;
constexpr size_t GEMV_LDS_BUDGET = 64 * 1024;

__device__ __forceinline__ float wave_max(float v) {
    for (int off = 32; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, 64));
    return v;
}

__device__ __forceinline__ int wave_or(int v) {
    for (int off = 32; off > 0; off >>= 1) v |= __shfl_xor(v, off, 64);
    return v;
}

template <int MR>
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
    const int groups = (P + 3) / 4;
    for (int grp = blockIdx.x * (THREADS / 64) + wave; grp < groups; grp += gridDim.x * (THREADS / 64)) {
        int acc[4][MR][2];
        for (int q = 0; q < 4; q++)
            for (int r = 0; r < MR; r++) acc[q][r][0] = acc[q][r][1] = 0;
        const uint8_t *wp[4];
        for (int q = 0; q < 4; q++) {
            const int p = min(grp * 4 + q, P - 1);
            wp[q] = wv + (size_t)p * panel_stride + lane * 16;
        }
        for (int t = 0; t < KB; t++) {
            uint4 w[4];
            for (int q = 0; q < 4; q++) w[q] = *reinterpret_cast<const uint4 *>(wp[q] + (size_t)t * blk_stride);
            for (int r = 0; r < MR; r++) {
                const uint8_t *ap = sqa + r * row_bytes + t * 128 + g * 16;
                const uint4 ahi = *reinterpret_cast<const uint4 *>(ap);
                const uint4 alo = *reinterpret_cast<const uint4 *>(ap + 64);
                for (int q = 0; q < 4; q++) {
                    int h = acc[q][r][0], l = acc[q][r][1];
                    h = __builtin_amdgcn_sdot4((int)ahi.x, (int)w[q].x, h, false);
                    h = __builtin_amdgcn_sdot4((int)ahi.y, (int)w[q].y, h, false);
                    h = __builtin_amdgcn_sdot4((int)ahi.z, (int)w[q].z, h, false);
                    h = __builtin_amdgcn_sdot4((int)ahi.w, (int)w[q].w, h, false);
                    l = __builtin_amdgcn_sdot4((int)alo.x, (int)w[q].x, l, false);
                    l = __builtin_amdgcn_sdot4((int)alo.y, (int)w[q].y, l, false);
                    l = __builtin_amdgcn_sdot4((int)alo.z, (int)w[q].z, l, false);
                    l = __builtin_amdgcn_sdot4((int)alo.w, (int)w[q].w, l, false);
                    acc[q][r][0] = h;
                    acc[q][r][1] = l;
                }
            }
        }
        // Reduce-scatter over g. Step 1 (xor 32): lanes with g < 2 keep panels 0, 1 and take the
        // partner's partial sums of them; lanes with g >= 2 keep panels 2, 3.
        const bool upper = (g & 2) != 0, odd = (g & 1) != 0;
        int half[2][MR][2];
        for (int i = 0; i < 2; i++)
            for (int r = 0; r < MR; r++)
                for (int d = 0; d < 2; d++) {
                    const int keep = upper ? acc[i + 2][r][d] : acc[i][r][d];
                    const int send = upper ? acc[i][r][d] : acc[i + 2][r][d];
                    half[i][r][d] = keep + __shfl_xor(send, 32, 64);
                }
        // Step 2 (xor 16): even g keeps the first of its two panels, odd g the second.
        int fin[MR][2];
        for (int r = 0; r < MR; r++)
            for (int d = 0; d < 2; d++) {
                const int keep = odd ? half[1][r][d] : half[0][r][d];
                const int send = odd ? half[0][r][d] : half[1][r][d];
                fin[r][d] = keep + __shfl_xor(send, 16, 64);
            }
        const int p = grp * 4 + g;
        const int col = p * PANEL + j;
        if (p < P && col < N) {
            const float sc = scales[col];
            for (int r = 0; r < MR; r++) {
                float *cp = c + (size_t)r * ldc + col;
                const float s = dequant(fin[r][0], fin[r][1], sexp[r], sc);
                *cp = epilogue(s, bias, (size_t)col, act, escale, accumulate != 0, cp);
            }
        }
    }
}

template <int MR>
hipError_t launch_rows(const float *a, size_t lda, const DeviceWeights &w, float *c, size_t ldc, const EpiArgs &epi,
                       hipStream_t s) {
    const size_t groups = div_ceil(w.panels, 4);
    size_t blocks = div_ceil(groups, THREADS / 64);
    if (blocks > 2048) blocks = 2048;
    const size_t lds = (size_t)MR * w.kb * 128;
    hipLaunchKernelGGL(gemv_i8_kernel<MR>, dim3((unsigned)blocks), dim3(THREADS), lds, s, a, lda, (int)w.k,
                       w.values, w.scales, (int)w.n, (int)w.panels, (int)w.kb, c, ldc, epi.bias, epi.act, epi.scale,
                       epi.accumulate, w.panel_stride, w.blk_stride);
    return hipGetLastError();
}

}  // namespace

bool gemv_fits(size_t m, size_t k) {
    return m >= 1 && m <= GEMV_MAX_ROWS && m * div_ceil(k, KBLK) * 128 <= GEMV_LDS_BUDGET;
}

hipError_t launch_gemv_i8(const float *a, size_t lda, size_t m, const DeviceWeights &w, float *c, size_t ldc,
                          const EpiArgs &epi, hipStream_t s) {
    if (m == 0 || w.n == 0) return hipSuccess;
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
