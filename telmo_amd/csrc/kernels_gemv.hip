// The decode-step GEMVs (m = 1..16 rows) over int8 weights: HBM-bound streams of the weights.
//
// Both kernels split their rows into two int8 digits in LDS themselves (the same digits and
// exponents as the GEMM path, so a row gives bit-identical outputs on every path) and read the
// weights in the MFMA layout: per k-block of 64 inputs of a 16-output panel, lane l = 16 g + j
// loads 16 contiguous bytes (inputs 64 t + 16 g + [0, 16) of output j), 1 KB per wave, coalesced.
//
// gemv_mfma_kernel (m <= 16, k <= 1984, 16-byte aligned rows, k % 4 == 0): the digits sit in LDS as 16 x 64 MFMA A operands in lane
// order, so each 1 KB weight block costs one 16-byte LDS read per digit and two
// v_mfma_i32_16x16x64_i8, whatever m is. The rows are read once into registers ahead of the
// weights; workgroups stay resident and walk the panels, so the rows are digitised once per
// workgroup, and the next panel's weights, scales, bias and old outputs are requested before the
// current panel's epilogue.
//
// gemv_i8_kernel (m <= 8, other rows): one panel per wavefront, v_dot4_i32_i8 against each
// row's digits; the four input groups meet by lane exchanges (xor 16, xor 32).
#include "tg_internal.hpp"

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

typedef int v4i __attribute__((ext_vector_type(4)));
typedef float v4f __attribute__((ext_vector_type(4)));

// Four zero inputs: what the MFMA GEMV loads for chunks past the end of a row. Never written; not
// const, so that it lives in global memory like the rows and the loads stay global loads.
__device__ __attribute__((aligned(16))) float ZERO_CHUNK[4] = {0.0f, 0.0f, 0.0f, 0.0f};

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


// The maximum over the 64 lanes (all active), returned to every lane. DPP moves within rows of
// 16 lanes (quad_perm [1,0,3,2], quad_perm [2,3,0,1], row_half_mirror, row_mirror) leave each row's
// maximum in all its lanes; the four rows meet through v_readlane. No LDS traffic.
__device__ __forceinline__ uint32_t wave_max_u(uint32_t v) {
    v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0xB1, 0xF, 0xF, false));
    v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x4E, 0xF, 0xF, false));
    v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x141, 0xF, 0xF, false));
    v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x140, 0xF, 0xF, false));
    const uint32_t r0 = (uint32_t)__builtin_amdgcn_readlane((int)v, 0);
    const uint32_t r1 = (uint32_t)__builtin_amdgcn_readlane((int)v, 16);
    const uint32_t r2 = (uint32_t)__builtin_amdgcn_readlane((int)v, 32);
    const uint32_t r3 = (uint32_t)__builtin_amdgcn_readlane((int)v, 48);
    return max(max(r0, r1), max(r2, r3));
}

// What one wavefront needs of panel p: its KBC first weight blocks, and for its lane's column the
// scale, the bias and the old outputs of its four rows (when accumulating).
template <int KBC>
__device__ __forceinline__ void fetch_panel(v4i (&wr)[KBC], float &sc, float &bv, float (&old)[4], int p, int lane,
                                            const uint8_t *wv, size_t panel_stride, size_t blk_stride, int KB,
                                            const float *scales, const float *bias, const float *c, size_t ldc,
                                            int N, int m, int accumulate) {
    const uint8_t *wp = wv + (size_t)p * panel_stride + lane * 16;
#pragma unroll
    for (int t = 0; t < KBC; t++) wr[t] = *reinterpret_cast<const v4i *>(wp + (size_t)min(t, KB - 1) * blk_stride);
    // Branch-free: loads that are not needed read a valid address and are discarded, so the
    // compiler's load counting stays exact and nothing here waits on earlier loads.
    const int col = p * PANEL + (lane & 15), orow = (lane >> 4) * 4;
    sc = scales[col];
    bv = *(bias ? bias + min(col, N - 1) : scales + col);
#pragma unroll
    for (int v = 0; v < 4; v++) {
        const bool need = accumulate && orow + v < m && col < N;
        old[v] = *(need ? c + (size_t)(orow + v) * ldc + col : c);
    }
}

// Q8_0 weights: for k-blocks c0 .. c0 + KBC - 1 of panel p, the two 8-byte operand halves of this
// lane (inputs 32 h + 8 g .. + 8 of output j, read from layout lane 16 (2 h + g / 2) + j at byte
// 8 (g % 2)) and the scales of the two 32-input blocks (zero past the last block).
template <int KBC>
__device__ __forceinline__ void load_q8(long (&wq)[KBC][2], float (&sq)[KBC][2], const uint8_t *wp, const float *sp,
                                        int c0, int KB, int NB, size_t blk_stride, int off0) {
#pragma unroll
    for (int t = 0; t < KBC; t++) {
        const int tt = min(c0 + t, KB - 1), b0 = 2 * tt, b1 = b0 + 1;
        wq[t][0] = *reinterpret_cast<const long *>(wp + (size_t)tt * blk_stride + off0);
        wq[t][1] = *reinterpret_cast<const long *>(wp + (size_t)tt * blk_stride + off0 + 512);
        sq[t][0] = sp[(size_t)b0 * PANEL];
        const float s1 = sp[(size_t)min(b1, NB - 1) * PANEL];
        sq[t][1] = b1 < NB ? s1 : 0.0f;
    }
}

// What one wavefront needs of Q8_0 panel p: its first KBC k-blocks' operand halves and block
// scales, and for its lane's column the bias and the old outputs (branch-free, as fetch_panel).
template <int KBC>
__device__ __forceinline__ void fetch_panel_q8(long (&wq)[KBC][2], float (&sq)[KBC][2], float &bv, float (&old)[4],
                                               int p, int lane, const uint8_t *wv, size_t panel_stride,
                                               size_t blk_stride, int KB, int NB, int off0, const float *scales,
                                               const float *bias, const float *c, size_t ldc, int N, int m,
                                               int accumulate) {
    const int col = p * PANEL + (lane & 15), orow = (lane >> 4) * 4;
    load_q8<KBC>(wq, sq, wv + (size_t)p * panel_stride, scales + (size_t)p * NB * PANEL + (lane & 15), 0, KB, NB,
                 blk_stride, off0);
    bv = *(bias ? bias + min(col, N - 1) : scales);
#pragma unroll
    for (int v = 0; v < 4; v++) {
        const bool need = accumulate && orow + v < m && col < N;
        old[v] = *(need ? c + (size_t)(orow + v) * ldc + col : c);
    }
}

// The row exponent from the row's n <= 8 per-wavefront maxima (bits of |x|, all ones for a
// non-finite input).
__device__ __forceinline__ int32_t exponent_from_slots(const uint32_t *slots, int n) {
    uint32_t mx = 0;
#pragma unroll
    for (int s = 0; s < 8; s++)
        if (s < n) mx = max(mx, slots[s]);
    return mx == 0xffffffffu ? EXP_NONFINITE : row_exponent_of(__uint_as_float(mx));
}

// Rows are split into 4-input chunks, ceil(KB / 4) wavefronts of them per row (the tail of the
// last wavefront idle); wavefront w holds chunk wavefronts w + WAVES j (j < J) in registers. The
// rows are read once, before the weights, so the weight loads stay in flight while the rows are
// digitised.
template <int WAVES, int KBC, int J, int Q8>
__global__ __launch_bounds__(WAVES * 64) void gemv_mfma_kernel(const float *__restrict__ a, size_t lda, int m, int k,
                                                               const uint8_t *__restrict__ wv,
                                                               const float *__restrict__ scales, int N, int P, int KB,
                                                               int NB, float *__restrict__ c, size_t ldc,
                                                               const float *__restrict__ bias, uint32_t act,
                                                               float escale, int accumulate, size_t panel_stride,
                                                               size_t blk_stride) {
    extern __shared__ __attribute__((aligned(16))) uint8_t sqa[];  // KB x (hi, lo) x 1 KB operands
    __shared__ uint32_t slot[WAVES * J];                           // max |x| bits per wavefront of chunks
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    // Chunk wavefront q = wave + WAVES j covers chunks 64 (q - r spr) + [0, 64) of row
    // r = q / spr, where spr = ceil(KB / 4) wavefronts cover a row (its tail idle). All of it is
    // uniform over the wavefront; q / spr is (q inv) >> 16, exact for q < 1024 and spr <= 8.
    const int spr = (KB + 3) / 4, inv = (65536 + spr - 1) / spr;
    const int wq = __builtin_amdgcn_readfirstlane(wave);
    const int step = gridDim.x * WAVES;
    int p = blockIdx.x * WAVES + wave;

    // One 16-byte load per chunk (rows 16-byte aligned, k % 4 == 0); chunks past the rows read
    // the zero chunk. Every load is unconditional and used as loaded, so the loads stay ahead of
    // the weight loads and waiting for them never waits for the weights.
    v4f x[J];
#pragma unroll
    for (int j = 0; j < J; j++) {
        const int q = wq + WAVES * j, r = (q * inv) >> 16;
        const int i0 = ((q - r * spr) * 64 + lane) * 4;
        const float *src = (r < m && i0 < k) ? a + (size_t)r * lda + i0 : ZERO_CHUNK;
        x[j] = *reinterpret_cast<const v4f *>(src);
    }
    // Panel fetches are unconditional (a wavefront past the last panel re-reads panel P - 1 and
    // never uses it): under a branch the compiler's load counting would wait for them early.
    // int8: whole 16-byte operands and one scale per column. Q8_0: 8-byte halves and block scales.
    const int off0 = (16 * ((lane >> 4) >> 1) + (lane & 15)) * 16 + 8 * ((lane >> 4) & 1);
    v4i wr[Q8 ? 1 : KBC];
    long wh[Q8 ? KBC : 1][2];
    float sq[Q8 ? KBC : 1][2];
    float sc = 0.0f, bv, old[4];
    if constexpr (Q8)
        fetch_panel_q8<KBC>(wh, sq, bv, old, min(p, P - 1), lane, wv, panel_stride, blk_stride, KB, NB, off0, scales,
                            bias, c, ldc, N, m, accumulate);
    else
        fetch_panel<KBC>(wr, sc, bv, old, min(p, P - 1), lane, wv, panel_stride, blk_stride, KB, scales, bias, c,
                         ldc, N, m, accumulate);

#pragma unroll
    for (int j = 0; j < J; j++) {
        const int q = wq + WAVES * j, r = (q * inv) >> 16;
        if (r < m) {
            const v4f v = x[j];
            const bool bad = !__builtin_isfinite(v.x) | !__builtin_isfinite(v.y) | !__builtin_isfinite(v.z) |
                             !__builtin_isfinite(v.w);
            const float mx = fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w)));
            const uint32_t b = wave_max_u(bad ? 0xffffffffu : __float_as_uint(mx));
            if (lane == 0) slot[q] = b;
        }
    }
    __syncthreads();
    // Lane r < m of every wavefront holds row r's exponent; the rest read it from there.
    const int32_t e_lane = lane < m ? exponent_from_slots(slot + lane * spr, spr) : 0;
    // Digits: chunk cc of row r holds inputs 4 cc .. 4 cc + 3, i.e. k-block cc / 16 and bytes
    // 4 (cc % 16) .. of that block's 64; they go where lane 16 (cc % 16 / 4) + r reads its A operand.
#pragma unroll
    for (int j = 0; j < J; j++) {
        const int q = wq + WAVES * j, r = (q * inv) >> 16;
        if (r < m) {
            const int cc = (q - r * spr) * 64 + lane;
            if (cc < KB * 16) {
                const int32_t e = __builtin_amdgcn_readlane(e_lane, r);
                uint32_t h, l;
                digits4(x[j].x, x[j].y, x[j].z, x[j].w, e, h, l);
                uint8_t *d = sqa + (cc >> 4) * 2048 + ((cc & 15) >> 2) * 256 + r * 16 + (cc & 3) * 4;
                *reinterpret_cast<uint32_t *>(d) = h;
                *reinterpret_cast<uint32_t *>(d + 1024) = l;
            }
        }
    }
    // C operand of the MFMA: element v of lane l is row 4 (l / 16) + v, column l % 16. Rows m..15
    // of the A operands are never written; their outputs are never stored.
    const int orow = (lane >> 4) * 4, ocol = lane & 15;
    int32_t erow[4];
#pragma unroll
    for (int v = 0; v < 4; v++) erow[v] = __shfl(e_lane, min(orow + v, 15), 64);
    __syncthreads();

    const uint8_t *ap = sqa + lane * 16;
    for (; p < P; p += step) {
        v4i acc_hi = {0, 0, 0, 0}, acc_lo = {0, 0, 0, 0};
        v4f accq = {0.0f, 0.0f, 0.0f, 0.0f};
        const uint8_t *wp = wv + (size_t)p * panel_stride;
        for (int c0 = 0; c0 < KB; c0 += KBC) {
            if constexpr (Q8) {
                if (c0 > 0)
                    load_q8<KBC>(wh, sq, wp, scales + (size_t)p * NB * PANEL + (lane & 15), c0, KB, NB, blk_stride,
                                 off0);
#pragma unroll
                for (int t = 0; t < KBC; t++) {
                    if (c0 + t < KB) {
#pragma unroll
                        for (int h = 0; h < 2; h++) {
                            const uint8_t *aq = sqa + (c0 + t) * 2048 + off0 + h * 512;
                            const long ahi = *reinterpret_cast<const long *>(aq);
                            const long alo = *reinterpret_cast<const long *>(aq + 1024);
                            const v4i hh = __builtin_amdgcn_mfma_i32_16x16x32_i8(ahi, wh[t][h], v4i{0, 0, 0, 0}, 0, 0, 0);
                            const v4i ll = __builtin_amdgcn_mfma_i32_16x16x32_i8(alo, wh[t][h], v4i{0, 0, 0, 0}, 0, 0, 0);
#pragma unroll
                            for (int v = 0; v < 4; v++)
                                accq[v] = __builtin_fmaf(sq[t][h], (float)(hh[v] * 256 + ll[v]), accq[v]);
                        }
                    }
                }
            } else {
                if (c0 > 0) {
#pragma unroll
                    for (int t = 0; t < KBC; t++)
                        wr[t] = *reinterpret_cast<const v4i *>(wp + lane * 16 + (size_t)min(c0 + t, KB - 1) * blk_stride);
                }
#pragma unroll
                for (int t = 0; t < KBC; t++) {
                    if (c0 + t < KB) {
                        const v4i ahi = *reinterpret_cast<const v4i *>(ap + (c0 + t) * 2048);
                        const v4i alo = *reinterpret_cast<const v4i *>(ap + (c0 + t) * 2048 + 1024);
                        acc_hi = __builtin_amdgcn_mfma_i32_16x16x64_i8(ahi, wr[t], acc_hi, 0, 0, 0);
                        acc_lo = __builtin_amdgcn_mfma_i32_16x16x64_i8(alo, wr[t], acc_lo, 0, 0, 0);
                    }
                }
            }
        }
        const float sc0 = sc, bv0 = bv;
        float old0[4];
#pragma unroll
        for (int v = 0; v < 4; v++) old0[v] = old[v];
        if constexpr (Q8)
            fetch_panel_q8<KBC>(wh, sq, bv, old, min(p + step, P - 1), lane, wv, panel_stride, blk_stride, KB, NB, off0,
                                scales, bias, c, ldc, N, m, accumulate);
        else
            fetch_panel<KBC>(wr, sc, bv, old, min(p + step, P - 1), lane, wv, panel_stride, blk_stride, KB, scales,
                             bias, c, ldc, N, m, accumulate);
        const int col = p * PANEL + ocol;
        if (col < N) {
#pragma unroll
            for (int v = 0; v < 4; v++) {
                if (orow + v < m) {
                    float s;
                    if constexpr (Q8)
                        s = erow[v] == EXP_NONFINITE ? __builtin_nanf("") : __builtin_ldexpf(accq[v], -erow[v]);
                    else
                        s = dequant(acc_hi[v], acc_lo[v], erow[v], sc0);
                    c[(size_t)(orow + v) * ldc + col] =
                        epilogue_vals(s, bias != nullptr, bv0, act, escale, accumulate != 0, old0[v]);
                }
            }
        }
    }
}

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

template <int WAVES, int KBC, int J>
void launch_mfma_t(const float *a, size_t lda, size_t m, const DeviceWeights &w, float *c, size_t ldc,
                   const EpiArgs &epi, size_t blocks, hipStream_t s) {
    const bool q8 = w.precision == Q8_0;
    hipLaunchKernelGGL(q8 ? (gemv_mfma_kernel<WAVES, KBC, J, 1>) : (gemv_mfma_kernel<WAVES, KBC, J, 0>),
                       dim3((unsigned)blocks), dim3(WAVES * 64), w.kb * 2048, s, a, lda, (int)m, (int)w.k, w.values,
                       w.scales, (int)w.n, (int)w.panels, (int)w.kb, (int)(w.k / Q8_BLOCK), c, ldc,
                       epi.bias, epi.act, epi.scale, epi.accumulate, w.panel_stride, w.blk_stride);
}

template <int WAVES, int KBC>
void launch_mfma_j(size_t j, const float *a, size_t lda, size_t m, const DeviceWeights &w, float *c,
                   size_t ldc, const EpiArgs &epi, size_t blocks, hipStream_t s) {
    if (j <= 1) launch_mfma_t<WAVES, KBC, 1>(a, lda, m, w, c, ldc, epi, blocks, s);
    else if (j <= 2) launch_mfma_t<WAVES, KBC, 2>(a, lda, m, w, c, ldc, epi, blocks, s);
    else if (j <= 3) launch_mfma_t<WAVES, KBC, 3>(a, lda, m, w, c, ldc, epi, blocks, s);
    else if (j <= 4) launch_mfma_t<WAVES, KBC, 4>(a, lda, m, w, c, ldc, epi, blocks, s);
    else if (j <= 6) launch_mfma_t<WAVES, KBC, 6>(a, lda, m, w, c, ldc, epi, blocks, s);
    else if (j <= 8) launch_mfma_t<WAVES, KBC, 8>(a, lda, m, w, c, ldc, epi, blocks, s);
    else if (j <= 12) launch_mfma_t<WAVES, KBC, 12>(a, lda, m, w, c, ldc, epi, blocks, s);
    else launch_mfma_t<WAVES, KBC, 16>(a, lda, m, w, c, ldc, epi, blocks, s);
}

hipError_t launch_mfma(const float *a, size_t lda, size_t m, const DeviceWeights &w, float *c, size_t ldc,
                       const EpiArgs &epi, hipStream_t s) {
    const size_t chunks = m * div_ceil(w.kb, (size_t)4) * 64;
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
        if (w.kb <= 10) launch_mfma_j<2, 10>(j, a, lda, m, w, c, ldc, epi, blocks, s);
        else launch_mfma_j<2, 16>(j, a, lda, m, w, c, ldc, epi, blocks, s);
    } else {
        if (w.kb <= 10) launch_mfma_j<4, 10>(j, a, lda, m, w, c, ldc, epi, blocks, s);
        else launch_mfma_j<4, 16>(j, a, lda, m, w, c, ldc, epi, blocks, s);
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
