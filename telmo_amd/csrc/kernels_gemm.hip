// The encoder-shaped int8-weight GEMM on gfx950 matrix cores.
//
// c[m, n] = epilogue(dequant(sum_k hi[m, k] q[n, k], sum_k lo[m, k] q[n, k])), where hi/lo are
// the two int8 digits of each activation (the QA rows) and q the int8 weights in the MFMA
// layout. Both sums run on v_mfma_i32_16x16x64_i8 and are exact, so the result does not depend
// on tiling, k-order or splits; the f32 arithmetic happens once per output in the epilogue.
//
// Tiling: a workgroup of 4 wavefronts owns a BM x BN = 128 x 128 output tile; each wavefront a
// 64 x 64 quarter as 4 x 4 MFMA blocks of 16 x 16, with one i32 accumulator set per digit
// (128 accumulator VGPRs). Per k-block of 64 inputs the tile's A (128 rows x 128 digit bytes)
// and B (8 panels x 1 KB) are staged through LDS, double-buffered, with 16-byte coalesced global
// loads issued one k-block ahead.
#include "tg_internal.hpp"

namespace tg {

typedef int v4i __attribute__((ext_vector_type(4)));

namespace {

constexpr int BM = 128;
constexpr int BN = 128;
constexpr int BP = BN / PANEL;          // panels per tile
constexpr int A_STRIDE = 128 + 16;      // LDS bytes per A row (padded against bank conflicts)
constexpr int A_TILE = BM * A_STRIDE;   // 18432
constexpr int B_TILE = BP * 1024;       // 8192
constexpr int STAGE = A_TILE + B_TILE;  // 26624
constexpr int THREADS = 256;

__global__ __launch_bounds__(THREADS) void gemm_i8_kernel(const uint8_t *__restrict__ qa,
                                                          const int32_t *__restrict__ exps, int M,
                                                          const uint8_t *__restrict__ wv,
                                                          const float *__restrict__ scales, int N, int P, int KB,
                                                          float *__restrict__ c, size_t ldc,
                                                          const float *__restrict__ bias, uint32_t act, float escale,
                                                          int accumulate) {
    __shared__ __attribute__((aligned(16))) uint8_t smem[2 * STAGE];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave & 1, wn = wave >> 1;
    const int m0 = blockIdx.y * BM, p0 = blockIdx.x * BP;
    const size_t qa_stride = (size_t)KB * 128;

    // Global -> LDS assignment. A: 128 rows x 8 chunks of 16 bytes, 4 chunks per thread.
    // B: 8 panels x 64 chunks, 2 per thread. Rows and panels past the edge read the last valid
    // one; their results are never stored.
    const uint8_t *a_src[4];
    int a_dst[4];
    for (int i = 0; i < 4; i++) {
        const int row = (tid >> 3) + 32 * i;
        const int grow = min(m0 + row, M - 1);
        a_src[i] = qa + (size_t)grow * qa_stride + (tid & 7) * 16;
        a_dst[i] = row * A_STRIDE + (tid & 7) * 16;
    }
    const uint8_t *b_src[2];
    int b_dst[2];
    for (int i = 0; i < 2; i++) {
        const int pl = (tid >> 6) + 4 * i;
        const int gp = min(p0 + pl, P - 1);
        b_src[i] = wv + (size_t)gp * KB * 1024 + (tid & 63) * 16;
        b_dst[i] = A_TILE + pl * 1024 + (tid & 63) * 16;
    }

    v4i acc_hi[4][4], acc_lo[4][4];
    for (int i = 0; i < 4; i++)
        for (int j = 0; j < 4; j++) {
            acc_hi[i][j] = v4i{0, 0, 0, 0};
            acc_lo[i][j] = v4i{0, 0, 0, 0};
        }

    uint4 ra[4], rb[2];
    auto load_global = [&](int t) {
        for (int i = 0; i < 4; i++) ra[i] = *reinterpret_cast<const uint4 *>(a_src[i] + (size_t)t * 128);
        for (int i = 0; i < 2; i++) rb[i] = *reinterpret_cast<const uint4 *>(b_src[i] + (size_t)t * 1024);
    };
    auto store_lds = [&](int stage) {
        uint8_t *st = smem + stage * STAGE;
        for (int i = 0; i < 4; i++) *reinterpret_cast<uint4 *>(st + a_dst[i]) = ra[i];
        for (int i = 0; i < 2; i++) *reinterpret_cast<uint4 *>(st + b_dst[i]) = rb[i];
    };

    if (KB > 0) {
        load_global(0);
        store_lds(0);
    }
    __syncthreads();

    const int frag_row = lane & 15, frag_k = (lane >> 4) * 16;
    for (int t = 0; t < KB; t++) {
        const uint8_t *st = smem + (t & 1) * STAGE;
        if (t + 1 < KB) load_global(t + 1);
        v4i bw[4];
        for (int cb = 0; cb < 4; cb++)
            bw[cb] = *reinterpret_cast<const v4i *>(st + A_TILE + (wn * 4 + cb) * 1024 + lane * 16);
        for (int rb_ = 0; rb_ < 4; rb_++) {
            const uint8_t *ap = st + (wm * 64 + rb_ * 16 + frag_row) * A_STRIDE + frag_k;
            const v4i ahi = *reinterpret_cast<const v4i *>(ap);
            const v4i alo = *reinterpret_cast<const v4i *>(ap + 64);
            for (int cb = 0; cb < 4; cb++) {
                acc_hi[rb_][cb] = __builtin_amdgcn_mfma_i32_16x16x64_i8(ahi, bw[cb], acc_hi[rb_][cb], 0, 0, 0);
                acc_lo[rb_][cb] = __builtin_amdgcn_mfma_i32_16x16x64_i8(alo, bw[cb], acc_lo[rb_][cb], 0, 0, 0);
            }
        }
        if (t + 1 < KB) store_lds((t + 1) & 1);
        __syncthreads();
    }

    // Accumulator element v of lane l holds output row 4 (l / 16) + v, column l % 16 of its block.
    const int out_col = lane & 15, out_row = (lane >> 4) * 4;
    for (int rb_ = 0; rb_ < 4; rb_++) {
        for (int cb = 0; cb < 4; cb++) {
            const int col = (p0 + wn * 4 + cb) * PANEL + out_col;
            if (col >= N) continue;
            const float sc = scales[col];
            for (int v = 0; v < 4; v++) {
                const int row = m0 + wm * 64 + rb_ * 16 + out_row + v;
                if (row >= M) continue;
                float *cp = c + (size_t)row * ldc + col;
                const float s = dequant(acc_hi[rb_][cb][v], acc_lo[rb_][cb][v], exps[row], sc);
                *cp = epilogue(s, bias, (size_t)col, act, escale, accumulate != 0, cp);
            }
        }
    }
}

}  // namespace

hipError_t launch_gemm_i8(const uint8_t *qa, const int32_t *exps, size_t m, const DeviceWeights &w, float *c,
                          size_t ldc, const EpiArgs &epi, hipStream_t s) {
    if (m == 0 || w.n == 0) return hipSuccess;
    dim3 grid((unsigned)div_ceil(w.panels, BP), (unsigned)div_ceil(m, BM));
    hipLaunchKernelGGL(gemm_i8_kernel, grid, dim3(THREADS), 0, s, qa, exps, (int)m, w.values, w.scales, (int)w.n,
                       (int)w.panels, (int)w.kb, c, ldc, epi.bias, epi.act, epi.scale, epi.accumulate);
    return hipGetLastError();
}

}  // namespace tg
