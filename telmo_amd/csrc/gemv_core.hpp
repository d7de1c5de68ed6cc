// The GEMV of the decode steps (m <= 16 rows, k <= 1984) as a device-function template over where
// its input rows come from and where its outputs go, so the plain GEMV and the fused TDT step share
// one body. The rows are read once into registers ahead of the weights, split into two int8 digits
// in LDS as 16 x 64 MFMA A operands, and every 1 KB weight block costs one 16-byte LDS read per digit
// and two v_mfma_i32_16x16x64_i8 (Q8_0: four 16x16x32 MFMAs and a per-block f32 fold). With DOTR > 0
// (int8 weights, at most DOTR rows) the block costs each row two 16-byte LDS reads and eight
// v_dot4_i32_i8 instead, no MFMA, and the four 16-input groups of a column meet across the
// wavefront after the k-loop; the sums, and so the outputs, are the same integers.
// Workgroups stay resident and walk the panels, requesting the next panel's weights, scales, bias
// and old outputs before the current panel's epilogue.
#pragma once
#include "tg_internal.hpp"

namespace tg {
namespace gemv {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef float v4f __attribute__((ext_vector_type(4)));

// Four zero inputs: what the GEMV loads for chunks past the end of a row. Never written; not const,
// so that it lives in global memory like the rows and the loads stay global loads.
static __device__ __attribute__((aligned(16))) float ZERO_CHUNK[4] = {0.0f, 0.0f, 0.0f, 0.0f};

// Input rows read from memory: row r at a + r lda (16-byte aligned rows, k % 4 == 0).
struct RowsIn {
    const float *a;
    size_t lda;
    __device__ __forceinline__ v4f load(int r, int i0, int m, int k) const {
        const float *src = (r < m && i0 < k) ? a + (size_t)r * lda + i0 : ZERO_CHUNK;
        return *reinterpret_cast<const v4f *>(src);
    }
};

// Outputs stored to c (row stride ldc).
struct StoreC {
    float *c;
    size_t ldc;
    __device__ __forceinline__ void store(int r, int col, float v) { c[(size_t)r * ldc + col] = v; }
};

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

// What one wavefront needs of panel p: its KBC first weight blocks (k-blocks kw, kw + ks, ...), and
// for its lane's column the scale, the bias and the old outputs of its four rows (when accumulating).
template <int KBC>
__device__ __forceinline__ void fetch_panel(v4i (&wr)[KBC], float &sc, float &bv, float (&old)[4], int p, int lane,
                                            const uint8_t *wv, size_t panel_stride, size_t blk_stride, int KB,
                                            const float *scales, const float *bias, const float *c, size_t ldc,
                                            int N, int m, int accumulate, int kw = 0, int ks = 1) {
    const uint8_t *wp = wv + (size_t)p * panel_stride + lane * 16;
#pragma unroll
    for (int t = 0; t < KBC; t++)
        wr[t] = *reinterpret_cast<const v4i *>(wp + (size_t)min(kw + ks * t, KB - 1) * blk_stride);
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

// A wavefront's operands of one panel in registers: the first KBC weight blocks (int8: whole
// 16-byte operands and one scale per column; Q8_0: 8-byte halves and block scales), the bias and
// the old outputs of its column.
template <int KBC, int Q8>
struct Panel {
    v4i wr[Q8 ? 1 : KBC];
    long wh[Q8 ? KBC : 1][2];
    float sq[Q8 ? KBC : 1][2];
    float sc, bv, old[4];
};

// The first panel mfma_body<WAVES, ..., KS> gives this wavefront, fetched as its body would fetch it:
// for callers whose input rows depend on loads of their own (a control block, another kernel's
// outputs), so that the weights are requested first and arrive while those loads resolve. The panel
// fetch is unconditional (a wavefront past the last panel re-reads panel P - 1 and never uses it).
template <int WAVES, int KBC, int Q8, int KS = 1>
__device__ __forceinline__ void fetch_first(Panel<KBC, Q8> &pn, int m, const uint8_t *__restrict__ wv,
                                            const float *__restrict__ scales, int N, int P, int KB, int NB,
                                            const float *__restrict__ c, size_t ldc, const float *__restrict__ bias,
                                            int accumulate, size_t panel_stride, size_t blk_stride) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int kw = KS > 1 ? wave : 0;
    const int p = KS > 1 ? blockIdx.x : blockIdx.x * WAVES + wave;
    const int off0 = (16 * ((lane >> 4) >> 1) + (lane & 15)) * 16 + 8 * ((lane >> 4) & 1);
    pn.sc = 0.0f;
    if constexpr (Q8)
        fetch_panel_q8<KBC>(pn.wh, pn.sq, pn.bv, pn.old, min(p, P - 1), lane, wv, panel_stride, blk_stride, KB, NB,
                            off0, scales, bias, c, ldc, N, m, accumulate);
    else
        fetch_panel<KBC>(pn.wr, pn.sc, pn.bv, pn.old, min(p, P - 1), lane, wv, panel_stride, blk_stride, KB, scales,
                         bias, c, ldc, N, m, accumulate, kw, KS);
}

// The chunks of the input rows this thread holds in mfma_body: rows are split into 4-input chunks,
// ceil(KB / 4) wavefronts of them per row (the tail of the last wavefront idle); wavefront w holds
// chunk wavefronts w + WAVES j (j < J). Chunk wavefront q = wave + WAVES j covers chunks
// 64 (q - r spr) + [0, 64) of row r = q / spr, spr = ceil(KB / 4); q / spr is (q inv) >> 16, exact
// for q < 1024 and spr <= 8. One 16-byte load per chunk (rows 16-byte aligned, k % 4 == 0); chunks
// past the rows read the zero chunk. Every load is unconditional.
template <int WAVES, int J, class In>
__device__ __forceinline__ void load_rows(const In &in, v4f (&x)[J], int m, int k, int KB) {
    const int lane = threadIdx.x & 63;
    const int spr = (KB + 3) / 4, inv = (65536 + spr - 1) / spr;
    const int wq = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
#pragma unroll
    for (int j = 0; j < J; j++) {
        const int q = wq + WAVES * j, r = (q * inv) >> 16;
        x[j] = in.load(r, ((q - r * spr) * 64 + lane) * 4, m, k);
    }
}

// Rows are split into 4-input chunks, ceil(KB / 4) wavefronts of them per row (the tail of the
// last wavefront idle); wavefront w holds chunk wavefronts w + WAVES j (j < J) in registers. The
// rows are read once, before the weights, so the weight loads stay in flight while the rows are
// digitised. With PRE, pn holds the first panel already (fetch_first, called before the rows).
template <int WAVES, int KBC, int J, int Q8, class In, class Out, int DOTR, int KS, bool PRE>
__device__ __forceinline__ void mfma_body_impl(const In &in, Out &out, int m, int k, const uint8_t *__restrict__ wv,
                                               const float *__restrict__ scales, int N, int P, int KB, int NB,
                                               const float *__restrict__ c, size_t ldc, const float *__restrict__ bias,
                                               uint32_t act, float escale, int accumulate, size_t panel_stride,
                                               size_t blk_stride, uint8_t *sqa, uint32_t *slot, Panel<KBC, Q8> &pn) {
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    // Chunk wavefront q = wave + WAVES j covers chunks 64 (q - r spr) + [0, 64) of row
    // r = q / spr, where spr = ceil(KB / 4) wavefronts cover a row (its tail idle). All of it is
    // uniform over the wavefront; q / spr is (q inv) >> 16, exact for q < 1024 and spr <= 8.
    const int spr = (KB + 3) / 4, inv = (65536 + spr - 1) / spr;
    const int wq = __builtin_amdgcn_readfirstlane(wave);
    // KS > 1 (int8, KS = WAVES): the workgroup's wavefronts share each panel, wavefront kw taking
    // k-blocks kw, kw + KS, ...; their integer sums meet in LDS and wavefront 0 stores the panel.
    // For products of few panels, where one wavefront per panel would leave most SIMDs idle and
    // walk long rows of k-blocks alone.
    static_assert(KS == 1 || (KS == WAVES && !Q8), "the k-split takes the whole workgroup, int8 weights");
    const int kw = KS > 1 ? wave : 0;
    const int nkb = KS > 1 ? (KB - kw + KS - 1) / KS : KB;  // this wavefront's k-blocks
    const int step = KS > 1 ? gridDim.x : gridDim.x * WAVES;
    int p = KS > 1 ? blockIdx.x : blockIdx.x * WAVES + wave;

    // The rows' loads are used as loaded and issued ahead of the weight loads, so waiting for them
    // never waits for the weights.
    v4f x[J];
    load_rows<WAVES, J>(in, x, m, k, KB);
    // Panel fetches are unconditional (a wavefront past the last panel re-reads panel P - 1 and
    // never uses it): under a branch the compiler's load counting would wait for them early.
    // int8: whole 16-byte operands and one scale per column. Q8_0: 8-byte halves and block scales.
    const int off0 = (16 * ((lane >> 4) >> 1) + (lane & 15)) * 16 + 8 * ((lane >> 4) & 1);
    if constexpr (!PRE) {
        pn.sc = 0.0f;
        if constexpr (Q8)
            fetch_panel_q8<KBC>(pn.wh, pn.sq, pn.bv, pn.old, min(p, P - 1), lane, wv, panel_stride, blk_stride, KB,
                                NB, off0, scales, bias, c, ldc, N, m, accumulate);
        else
            fetch_panel<KBC>(pn.wr, pn.sc, pn.bv, pn.old, min(p, P - 1), lane, wv, panel_stride, blk_stride, KB,
                             scales, bias, c, ldc, N, m, accumulate, kw, KS);
    }
    auto &wr = pn.wr;
    auto &wh = pn.wh;
    auto &sq = pn.sq;
    float &sc = pn.sc, &bv = pn.bv;
    auto &old = pn.old;

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
    constexpr bool DOT = DOTR > 0 && !Q8;
    // DOTR rows: lane (g = l / 16, j = l % 16) reads row r's operand lane 16 g + r (the digits of
    // the inputs its weights multiply) and sums with v_dot4_i32_i8.
    const uint8_t *dp = sqa + (lane >> 4) * 256;
    int par = 0;
    for (; p < P; p += step) {
        v4i acc_hi = {0, 0, 0, 0}, acc_lo = {0, 0, 0, 0};
        v4f accq = {0.0f, 0.0f, 0.0f, 0.0f};
        int dh[DOTR > 0 ? DOTR : 1], dl[DOTR > 0 ? DOTR : 1];
#pragma unroll
        for (int r = 0; r < (DOTR > 0 ? DOTR : 1); r++) dh[r] = dl[r] = 0;
        const uint8_t *wp = wv + (size_t)p * panel_stride;
        for (int c0 = 0; c0 < nkb; c0 += KBC) {
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
                        wr[t] = *reinterpret_cast<const v4i *>(wp + lane * 16 +
                                                               (size_t)min(kw + KS * (c0 + t), KB - 1) * blk_stride);
                }
#pragma unroll
                for (int t = 0; t < KBC; t++) {
                    if (c0 + t < nkb) {
                        const int kt = kw + KS * (c0 + t);  // the k-block
                        if constexpr (DOT) {
#pragma unroll
                            for (int r = 0; r < DOTR; r++) {
                                const v4i ahi = *reinterpret_cast<const v4i *>(dp + kt * 2048 + r * 16);
                                const v4i alo = *reinterpret_cast<const v4i *>(dp + kt * 2048 + 1024 + r * 16);
                                int h = dh[r], l = dl[r];
                                h = __builtin_amdgcn_sdot4(ahi.x, wr[t].x, h, false);
                                h = __builtin_amdgcn_sdot4(ahi.y, wr[t].y, h, false);
                                h = __builtin_amdgcn_sdot4(ahi.z, wr[t].z, h, false);
                                h = __builtin_amdgcn_sdot4(ahi.w, wr[t].w, h, false);
                                l = __builtin_amdgcn_sdot4(alo.x, wr[t].x, l, false);
                                l = __builtin_amdgcn_sdot4(alo.y, wr[t].y, l, false);
                                l = __builtin_amdgcn_sdot4(alo.z, wr[t].z, l, false);
                                l = __builtin_amdgcn_sdot4(alo.w, wr[t].w, l, false);
                                dh[r] = h;
                                dl[r] = l;
                            }
                        } else {
                            const v4i ahi = *reinterpret_cast<const v4i *>(ap + kt * 2048);
                            const v4i alo = *reinterpret_cast<const v4i *>(ap + kt * 2048 + 1024);
                            acc_hi = __builtin_amdgcn_mfma_i32_16x16x64_i8(ahi, wr[t], acc_hi, 0, 0, 0);
                            acc_lo = __builtin_amdgcn_mfma_i32_16x16x64_i8(alo, wr[t], acc_lo, 0, 0, 0);
                        }
                    }
                }
            }
        }
        if constexpr (DOT) {
            // The four input groups of a column meet (lanes j, j + 16, j + 32, j + 48); lane
            // (g, j) then holds rows 4 g .. 4 g + 3 of column j as the MFMA's C operand would.
#pragma unroll
            for (int r = 0; r < DOTR; r++) {
                dh[r] += __shfl_xor(dh[r], 16, 64);
                dh[r] += __shfl_xor(dh[r], 32, 64);
                dl[r] += __shfl_xor(dl[r], 16, 64);
                dl[r] += __shfl_xor(dl[r], 32, 64);
            }
            const bool upper = DOTR > 4 && (lane >> 4) == 1;
#pragma unroll
            for (int v = 0; v < 4; v++) {
                acc_hi[v] = upper ? dh[(4 + v) % DOTR] : dh[v % DOTR];
                acc_lo[v] = upper ? dl[(4 + v) % DOTR] : dl[v % DOTR];
            }
        }
        if constexpr (KS > 1) {
            // Two sets of slots, alternating by panel: a set is rewritten two panels on, after a
            // barrier that wavefront 0 reaches only once it has read the set.
            __shared__ v4i part[2][KS][2][64];
            v4i(*mine)[2][64] = part[par];
            mine[kw][0][lane] = acc_hi;
            mine[kw][1][lane] = acc_lo;
            __syncthreads();
            if (kw == 0) {
#pragma unroll
                for (int w = 1; w < KS; w++) {
                    acc_hi += mine[w][0][lane];
                    acc_lo += mine[w][1][lane];
                }
            }
            par ^= 1;
        }
        const float sc0 = sc, bv0 = bv;
        float old0[4];
#pragma unroll
        for (int v = 0; v < 4; v++) old0[v] = old[v];
        // The next panel's operands, when there is one (a uniform branch: the last panel's wavefront
        // leaves without loads still on the way).
        if (p + step < P) {
            if constexpr (Q8)
                fetch_panel_q8<KBC>(wh, sq, bv, old, p + step, lane, wv, panel_stride, blk_stride, KB, NB, off0, scales,
                                    bias, c, ldc, N, m, accumulate);
            else
                fetch_panel<KBC>(wr, sc, bv, old, p + step, lane, wv, panel_stride, blk_stride, KB, scales, bias, c,
                                 ldc, N, m, accumulate, kw, KS);
        }
        const int col = p * PANEL + ocol;
        if (col < N && kw == 0) {
#pragma unroll
            for (int v = 0; v < 4; v++) {
                if (orow + v < m) {
                    float s;
                    if constexpr (Q8)
                        s = erow[v] == EXP_NONFINITE ? __builtin_nanf("") : __builtin_ldexpf(accq[v], -erow[v]);
                    else
                        s = dequant(acc_hi[v], acc_lo[v], erow[v], sc0);
                    out.store(orow + v, col,
                              epilogue_vals(s, bias != nullptr, bv0, act, escale, accumulate != 0, old0[v]));
                }
            }
        }
    }
}

// The GEMV body, fetching its first panel after the rows.
template <int WAVES, int KBC, int J, int Q8, class In, class Out, int DOTR = 0, int KS = 1>
__device__ __forceinline__ void mfma_body(const In &in, Out &out, int m, int k, const uint8_t *__restrict__ wv,
                                          const float *__restrict__ scales, int N, int P, int KB, int NB,
                                          const float *__restrict__ c, size_t ldc, const float *__restrict__ bias,
                                          uint32_t act, float escale, int accumulate, size_t panel_stride,
                                          size_t blk_stride, uint8_t *sqa, uint32_t *slot) {
    Panel<KBC, Q8> pn;
    mfma_body_impl<WAVES, KBC, J, Q8, In, Out, DOTR, KS, false>(in, out, m, k, wv, scales, N, P, KB, NB, c, ldc, bias,
                                                                act, escale, accumulate, panel_stride, blk_stride,
                                                                sqa, slot, pn);
}

// The GEMV body on a first panel the caller fetched with fetch_first<WAVES, KBC, Q8, KS>.
template <int WAVES, int KBC, int J, int Q8, class In, class Out, int DOTR = 0, int KS = 1>
__device__ __forceinline__ void mfma_body_pre(const In &in, Out &out, int m, int k, const uint8_t *__restrict__ wv,
                                              const float *__restrict__ scales, int N, int P, int KB, int NB,
                                              const float *__restrict__ c, size_t ldc, const float *__restrict__ bias,
                                              uint32_t act, float escale, int accumulate, size_t panel_stride,
                                              size_t blk_stride, uint8_t *sqa, uint32_t *slot, Panel<KBC, Q8> &pn) {
    mfma_body_impl<WAVES, KBC, J, Q8, In, Out, DOTR, KS, true>(in, out, m, k, wv, scales, N, P, KB, NB, c, ldc, bias,
                                                               act, escale, accumulate, panel_stride, blk_stride,
                                                               sqa, slot, pn);
}

}  // namespace gemv
}  // namespace tg
