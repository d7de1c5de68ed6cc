// The encoder-shaped int8-weight GEMM on gfx950 matrix cores.
//
// c[m, n] = epilogue(dequant(sum_k hi[m, k] q[n, k], sum_k lo[m, k] q[n, k])), where hi/lo are
// the two int8 digits of each activation and q the int8 weights. Both sums run on
// v_mfma_i32_16x16x64_i8 and are exact, so the result does not depend on tiling, k-order or
// splits; the f32 arithmetic happens once per output in the epilogue.
//
// Both the quantised rows (fragment-major QA) and the weights (MFMA layout) store each 16 x 64
// MFMA operand as 1 KB in lane order, so one 16-byte load per lane is one operand, fully coalesced.
// Four kernels share that layout:
//   gemm_lds_kernel    operands copied from global memory straight into an LDS ring
//                      (global_load_lds_dwordx4), one copy per workgroup: 128 x 128 tiles when
//                      they fill the chip twice over, 64 x 64 tiles for products of >= 2048 outputs;
//                      the sums come out transposed and are stored from registers (store_transposed);
//   gemm_i8_kernel     2 x 2 independent wavefronts loading their operands straight into a
//                      register ring (no LDS, no barriers): narrower products; its sums come out
//                      transposed and are stored from registers too (750 x 1024 -> 1024:
//                      7.5 -> 6.7 us);
//   gemm_i8_kq_kernel  the narrower products with long inputs: each wavefront takes the whole
//                      48 x 64 or 64 x 64 tile over a quarter of the k-blocks, and the integer
//                      partial sums meet in LDS;
//   gemm_q8_lds_kernel Q8_0 weights (a scale per 32 inputs): per-block sums on
//                      v_mfma_i32_16x16x32_i8 folded in f32 in block order, on the LDS ring.
// The k-split kernel, whose partial sums meet in LDS anyway, stages its sums there and stores them
// through TileStore (the register-stored form was 0.5 us slower on it). launch_gemm_i8 at the end
// picks one by shape.
#include <type_traits>

#include "tg_internal.hpp"

namespace tg {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef float v4f __attribute__((ext_vector_type(4)));

namespace {

constexpr int THREADS = 256;
constexpr size_t GFX950_CUS = 256;  // compute units of an MI355X

// Whether every hi sum of the wavefront's RB x CB accumulators takes dequant_i32 (one vote).
template <int RB, int CB>
__device__ __forceinline__ bool wave_fits_i32(const v4i (&acc_hi)[RB][CB]) {
    bool ok = true;
#pragma unroll
    for (int r = 0; r < RB; r++)
#pragma unroll
        for (int cb = 0; cb < CB; cb++)
#pragma unroll
            for (int v = 0; v < 4; v++) ok &= dequant_fits(acc_hi[r][cb][v]);
    return __all(ok);
}

// The store of a wavefront's WM x WN tile of sums through the epilogue into c[m0.., n0..]. Lane l
// owns the runs of four outputs at column 4 (l % (WN / 4)) of rows l / (WN / 4), + 64 / (WN / 4),
// ...: per run one 16-byte load of the old outputs (when accumulating), one 16-byte LDS read of the
// staged sums (rows C_STRIDE floats apart) and one 16-byte store, marked nontemporal: the outputs
// are read by the next kernel, not this one, and streaming them out as they are stored leaves less
// to write back when the kernel ends (1-1.5 us less per launch on the 4096-output products).
// begin() issues the loads of the bias and old outputs before the sums are staged, so their
// latency overlaps the staging (for tiles of up to eight runs per lane; larger ones load in
// finish(), where the accumulators no longer hold registers). finish() stores, and nothing waits
// for a store, so the wavefront ends once its stores are issued. Runs past the right edge of c, or
// in a c or ldc not 16-byte aligned, go one output at a time; rows past M are skipped.
template <int WM, int WN, int C_STRIDE>
struct TileStore {
    static constexpr int RPR = WN / 4, STEP = 64 / RPR, PER = WM / STEP;
    static constexpr bool EARLY = PER <= 8;
    static_assert(WN % 4 == 0 && 64 % RPR == 0 && WM % STEP == 0, "whole runs per lane");
    static_assert(C_STRIDE % 4 == 0, "16-byte aligned staged rows");
    int cr, r0, col;
    bool vec;
    v4f b, old[PER];

    __device__ __forceinline__ void begin(int lane, const float *__restrict__ c, size_t ldc, int m0, int n0, int M,
                                          int N, const float *__restrict__ bias, int accumulate) {
        cr = lane % RPR;
        r0 = lane / RPR;
        col = n0 + 4 * cr;
        vec = ((reinterpret_cast<uintptr_t>(c) | ldc * sizeof(float)) % 16 == 0) && col + 4 <= N;
        b = v4f{0.0f, 0.0f, 0.0f, 0.0f};
        if (bias) {
#pragma unroll
            for (int j = 0; j < 4; j++) b[j] = col + j < N ? bias[col + j] : 0.0f;
        }
        if constexpr (EARLY) load_old(c, ldc, m0, M, N, accumulate);
    }

    __device__ __forceinline__ void load_old(const float *__restrict__ c, size_t ldc, int m0, int M, int N,
                                             int accumulate) {
#pragma unroll
        for (int u = 0; u < PER; u++) {
            old[u] = v4f{0.0f, 0.0f, 0.0f, 0.0f};
            const int row = m0 + r0 + u * STEP;
            if (accumulate && row < M) {
                const float *src = c + (size_t)row * ldc + col;
                if (vec) {
                    old[u] = *reinterpret_cast<const v4f *>(src);
                } else {
#pragma unroll
                    for (int j = 0; j < 4; j++)
                        if (col + j < N) old[u][j] = src[j];
                }
            }
        }
    }

    // With rmax, also each run's largest |y| over its columns below N, as unsigned bits (all ones
    // for a NaN or an infinity; 0 for rows past M). ACT: the activation, fixed at compile time
    // (finish() dispatches on act once) so that the unrolled runs hold no branch per output.
    template <uint32_t ACT>
    __device__ __forceinline__ void finish_act(const float *tile, float *__restrict__ c, size_t ldc, int m0, int M,
                                               int N, bool has_bias, float escale, int accumulate,
                                               uint32_t *rmax) {
        if constexpr (!EARLY) load_old(c, ldc, m0, M, N, accumulate);
#pragma unroll
        for (int u = 0; u < PER; u++) {
            const int row = m0 + r0 + u * STEP;
            if (rmax) rmax[u] = 0u;
            if (row >= M) continue;
            v4f v = *reinterpret_cast<const v4f *>(tile + (r0 + u * STEP) * C_STRIDE + 4 * cr);
#pragma unroll
            for (int j = 0; j < 4; j++)
                v[j] = epilogue_sel<ACT>(v[j], has_bias, b[j], ACT, escale, accumulate != 0, old[u][j]);
            if (rmax) {
                uint32_t mx = 0u;
#pragma unroll
                for (int j = 0; j < 4; j++)
                    if (col + j < N)
                        mx = max(mx, __builtin_isfinite(v[j]) ? __float_as_uint(fabsf(v[j])) : 0xffffffffu);
                rmax[u] = mx;
            }
            float *dst = c + (size_t)row * ldc + col;
            if (vec) {
                __builtin_nontemporal_store(v, reinterpret_cast<v4f *>(dst));
            } else {
#pragma unroll
                for (int j = 0; j < 4; j++)
                    if (col + j < N) dst[j] = v[j];
            }
        }
    }

    __device__ __forceinline__ void finish(const float *tile, float *__restrict__ c, size_t ldc, int m0, int M, int N,
                                           bool has_bias, uint32_t act, float escale, int accumulate,
                                           uint32_t *rmax = nullptr) {
        if (act == ACT_NONE) finish_act<ACT_NONE>(tile, c, ldc, m0, M, N, has_bias, escale, accumulate, rmax);
        else if (act == ACT_RELU) finish_act<ACT_RELU>(tile, c, ldc, m0, M, N, has_bias, escale, accumulate, rmax);
        else finish_act<ACT_SILU>(tile, c, ldc, m0, M, N, has_bias, escale, accumulate, rmax);
    }
};

// The GLU of a pair of staged tiles, the a and b halves of the same rows and columns (rows
// C_STRIDE floats apart): out[r, col] = va / (1 + exp(0 - vb)) with va and vb the sums through
// the epilogue (bias, activation, scale; no accumulation), the values tg_linear_device writes and
// tg_glu_device then combines. The b half's bias sits Nh columns on. Runs of four outputs per lane
// as TileStore, 16-byte nontemporal stores when out's rows are 16-byte aligned.
template <uint32_t ACT, int WM, int WN, int C_STRIDE>
__device__ __forceinline__ void glu_store_act(const float *ta, const float *tb, int lane, float *__restrict__ out,
                                              size_t ldo, int m0, int n0, int M, int Nh, const float *__restrict__ bias,
                                              float escale) {
    constexpr int RPR = WN / 4, STEP = 64 / RPR, PER = WM / STEP;
    static_assert(WN % 4 == 0 && 64 % RPR == 0 && WM % STEP == 0, "whole runs per lane");
    const int cr = lane % RPR, r0 = lane / RPR, col = n0 + 4 * cr;
    const bool vec = ((reinterpret_cast<uintptr_t>(out) | ldo * sizeof(float)) % 16 == 0) && col + 4 <= Nh;
    v4f ba = {0.0f, 0.0f, 0.0f, 0.0f}, bb = {0.0f, 0.0f, 0.0f, 0.0f};
    if (bias) {
#pragma unroll
        for (int j = 0; j < 4; j++)
            if (col + j < Nh) {
                ba[j] = bias[col + j];
                bb[j] = bias[Nh + col + j];
            }
    }
#pragma unroll
    for (int u = 0; u < PER; u++) {
        const int row = m0 + r0 + u * STEP;
        if (row >= M) continue;
        const v4f a = *reinterpret_cast<const v4f *>(ta + (r0 + u * STEP) * C_STRIDE + 4 * cr);
        const v4f b = *reinterpret_cast<const v4f *>(tb + (r0 + u * STEP) * C_STRIDE + 4 * cr);
        v4f o;
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const float va = epilogue_sel<ACT>(a[j], bias != nullptr, ba[j], ACT, escale, false, 0.0f);
            const float vb = epilogue_sel<ACT>(b[j], bias != nullptr, bb[j], ACT, escale, false, 0.0f);
            o[j] = va / (1.0f + exp_simd(0.0f - vb));
        }
        float *dst = out + (size_t)row * ldo + col;
        if (vec) {
            __builtin_nontemporal_store(o, reinterpret_cast<v4f *>(dst));
        } else {
#pragma unroll
            for (int j = 0; j < 4; j++)
                if (col + j < Nh) dst[j] = o[j];
        }
    }
}

// glu_store_act with the activation chosen once.
template <int WM, int WN, int C_STRIDE>
__device__ __forceinline__ void glu_store(const float *ta, const float *tb, int lane, float *__restrict__ out,
                                          size_t ldo, int m0, int n0, int M, int Nh, const float *__restrict__ bias,
                                          uint32_t act, float escale) {
#define TG_GLU(A) glu_store_act<A, WM, WN, C_STRIDE>(ta, tb, lane, out, ldo, m0, n0, M, Nh, bias, escale)
    if (act == ACT_NONE) TG_GLU(ACT_NONE);
    else if (act == ACT_RELU) TG_GLU(ACT_RELU);
    else TG_GLU(ACT_SILU);
#undef TG_GLU
}

// Order in which workgroups take tiles. Workgroup L of a launch goes to XCD L % 8 (each XCD has
// its own L2). XCD: hand each XCD a contiguous run of tiles (rows of the tile grid), so the A row
// blocks its tiles share stay in its L2. G > 0: walk the tiles G tile-rows at a time, column by
// column, so a weight panel is reused by G row blocks while it is hot.
template <int XCD, int G>
__device__ __forceinline__ void tile_of(int &bx, int &by) {
    bx = blockIdx.x;
    by = blockIdx.y;
    if constexpr (XCD || G) {
        const int gx = gridDim.x, gy = gridDim.y, total = gx * gy;
        int L = by * gx + bx;
        if constexpr (XCD) {
            const int full = total - total % 8;
            if (L < full) L = (L % 8) * (full / 8) + L / 8;
        }
        if constexpr (G > 0) {
            const int group = L / (G * gx), first = group * G, rows = min(G, gy - first), local = L - group * G * gx;
            by = first + local % rows;
            bx = local / rows;
        } else {
            by = L / gx;
            bx = L % gx;
        }
    }
}

// The wavefront's f32 sums staged in LDS (element v of lane l: row 4 (l / 16) + v, column l % 16 of
// each 16 x 16 block, rows C_STRIDE floats apart), through dequant_i32 when the whole wavefront's
// sums fit it, else dequant: the same values either way.
template <int RB, int CB, int C_STRIDE>
__device__ __forceinline__ void stage_sums(float *tile, const v4i (&acc_hi)[RB][CB], const v4i (&acc_lo)[RB][CB],
                                           const int32_t (&e_row)[RB][4], const float (&s_col)[CB], int out_row,
                                           int out_col) {
    if (wave_fits_i32<RB, CB>(acc_hi)) {
#pragma unroll
        for (int r = 0; r < RB; r++)
#pragma unroll
            for (int cb = 0; cb < CB; cb++)
#pragma unroll
                for (int v = 0; v < 4; v++)
                    tile[(r * 16 + out_row + v) * C_STRIDE + cb * 16 + out_col] =
                        dequant_i32(acc_hi[r][cb][v], acc_lo[r][cb][v], e_row[r][v], s_col[cb]);
    } else {
#pragma unroll
        for (int r = 0; r < RB; r++)
#pragma unroll
            for (int cb = 0; cb < CB; cb++)
#pragma unroll
                for (int v = 0; v < 4; v++)
                    tile[(r * 16 + out_row + v) * C_STRIDE + cb * 16 + out_col] =
                        dequant(acc_hi[r][cb][v], acc_lo[r][cb][v], e_row[r][v], s_col[cb]);
    }
}

// The epilogue of a wavefront whose MFMAs took the weights as the first operand and the rows as
// the second, so that the accumulators hold the transposed blocks: element v of lane l in block
// (r, cb) is the sum of row m0 + 16 r + l % 16, column n0 + 16 cb + 4 (l / 16) + v. Each lane then
// owns runs of four consecutive outputs and stores them from registers (16-byte nontemporal
// stores), with no staging in LDS and no barrier (the 12000 x 1024 -> 4096 product takes 140 us
// against 150 us with its sums staged in LDS). e[r] is the exponent of the lane's row in row block
// r, sc[cb] the scales of its four columns in block cb. With rmax, also each row block's largest
// |y| over the wavefront's columns below N (all ones for a NaN or an infinity, 0 past M), the same
// in the 16 lanes l % 16 of a row. Rows past M are skipped.
//
// FAST (a wave-uniform choice): every column of the wavefront lies below N and c, ldc and bias
// are 16-byte aligned, so the bias, the old outputs and the outputs move 16 bytes at a time with
// no column checks. Otherwise they move one output at a time, columns past N skipped. FITS: every
// sum of the wavefront takes dequant_i32 (else dequant); ACT: the activation (ACT_ANY: act).
// Both are wave-uniform and chosen once before the unrolled loops, which then hold no branch per
// output: with the choices inside, the epilogue of a 128 x 128 tile ran 700 branches.
template <bool FAST, bool FITS, uint32_t ACT, int RB, int CB>
__device__ __forceinline__ void store_transposed_as(const v4i (&acc_hi)[RB][CB], const v4i (&acc_lo)[RB][CB],
                                                    const int32_t (&e)[RB], const v4f (&sc)[CB], int lane,
                                                    float *__restrict__ c, size_t ldc, int m0, int n0, int M, int N,
                                                    const float *__restrict__ bias, uint32_t act, float escale,
                                                    int accumulate, uint32_t *rmax) {
    const int mr = lane & 15, nq = 4 * (lane >> 4);
    v4f b[CB];
#pragma unroll
    for (int cb = 0; cb < CB; cb++) {
        b[cb] = v4f{0.0f, 0.0f, 0.0f, 0.0f};
        const int col = n0 + 16 * cb + nq;
        if (bias) {
            if constexpr (FAST) {
                b[cb] = *reinterpret_cast<const v4f *>(bias + col);
            } else {
#pragma unroll
                for (int j = 0; j < 4; j++) b[cb][j] = col + j < N ? bias[col + j] : 0.0f;
            }
        }
    }
#pragma unroll
    for (int r = 0; r < RB; r++) {
        const int row = m0 + 16 * r + mr;
        float *dst = c + (size_t)row * ldc + n0 + nq;
        uint32_t mx = 0u;
        if (row < M) {
            v4f old[CB];
#pragma unroll
            for (int cb = 0; cb < CB; cb++) {
                old[cb] = v4f{0.0f, 0.0f, 0.0f, 0.0f};
                const int col = n0 + 16 * cb + nq;
                if (accumulate) {
                    if constexpr (FAST) {
                        old[cb] = *reinterpret_cast<const v4f *>(dst + 16 * cb);
                    } else {
#pragma unroll
                        for (int j = 0; j < 4; j++)
                            if (col + j < N) old[cb][j] = dst[16 * cb + j];
                    }
                }
            }
#pragma unroll
            for (int cb = 0; cb < CB; cb++) {
                const int col = n0 + 16 * cb + nq;
                v4f v;
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    const float d = FITS ? dequant_i32(acc_hi[r][cb][j], acc_lo[r][cb][j], e[r], sc[cb][j])
                                         : dequant(acc_hi[r][cb][j], acc_lo[r][cb][j], e[r], sc[cb][j]);
                    v[j] = epilogue_sel<ACT>(d, bias != nullptr, b[cb][j], act, escale, accumulate != 0, old[cb][j]);
                    if (rmax && (FAST || col + j < N))
                        mx = max(mx, __builtin_isfinite(v[j]) ? __float_as_uint(fabsf(v[j])) : 0xffffffffu);
                }
                if constexpr (FAST) {
                    __builtin_nontemporal_store(v, reinterpret_cast<v4f *>(dst + 16 * cb));
                } else {
#pragma unroll
                    for (int j = 0; j < 4; j++)
                        if (col + j < N) dst[16 * cb + j] = v[j];
                }
            }
        }
        if (rmax) {
            mx = max(mx, (uint32_t)__shfl_xor((int)mx, 16, 64));
            mx = max(mx, (uint32_t)__shfl_xor((int)mx, 32, 64));
            rmax[r] = mx;
        }
    }
}

// EDGE = 0: the launcher has checked that every wavefront is FAST (16-byte aligned c, ldc and bias,
// and N a multiple of the workgroup's columns), so the kernel carries the FAST code alone: an
// instruction footprint that fits the instruction cache (the kernel with both variants runs the
// 12000 x 1024 -> 2048 product 7% slower). EDGE = 1: each wavefront picks.
template <int EDGE, int RB, int CB>
__device__ __forceinline__ void store_transposed(const v4i (&acc_hi)[RB][CB], const v4i (&acc_lo)[RB][CB],
                                                 const int32_t (&e)[RB], const v4f (&sc)[CB], int lane,
                                                 float *__restrict__ c, size_t ldc, int m0, int n0, int M, int N,
                                                 const float *__restrict__ bias, uint32_t act, float escale,
                                                 int accumulate, uint32_t *rmax = nullptr) {
    const bool fast = !EDGE || (((reinterpret_cast<uintptr_t>(c) | ldc * sizeof(float) |
                                  reinterpret_cast<uintptr_t>(bias)) % 16) == 0 &&
                                n0 + 16 * CB <= N);
    const bool fits = wave_fits_i32<RB, CB>(acc_hi);
#define TG_ST(F, I, A)                                                                                          \
    store_transposed_as<F, I, A>(acc_hi, acc_lo, e, sc, lane, c, ldc, m0, n0, M, N, bias, act, escale, accumulate, \
                                 rmax)
#define TG_ST_ACTS(F)                              \
    do {                                           \
        if (!fits) TG_ST(F, false, ACT_ANY);       \
        else if (act == ACT_NONE) TG_ST(F, true, ACT_NONE); \
        else if (act == ACT_RELU) TG_ST(F, true, ACT_RELU); \
        else TG_ST(F, true, ACT_SILU);             \
    } while (0)
    if (fast) TG_ST_ACTS(true);
    else TG_ST_ACTS(false);
#undef TG_ST_ACTS
#undef TG_ST
}

template <int RB, int CB, int S, int OCC, int XCD, int G>
__global__ __launch_bounds__(THREADS, OCC) void gemm_i8_kernel(const uint8_t *__restrict__ qf,
                                                               const int32_t *__restrict__ exps, int M,
                                                               const uint8_t *__restrict__ wv,
                                                               const float *__restrict__ scales, int N, int P, int KB,
                                                               float *__restrict__ c, size_t ldc,
                                                               const float *__restrict__ bias, uint32_t act,
                                                               float escale, int accumulate, size_t b_panel,
                                                               size_t b_blk) {
    constexpr int WM = RB * 16, WN = CB * 16;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave & 1, wn = wave >> 1;
    int bx, by;
    tile_of<XCD, G>(bx, by);
    const int m0 = by * 2 * WM + wm * WM, n0 = bx * 2 * WN + wn * WN;
    const int R0 = m0 / 16, P0 = n0 / 16, RLAST = (M + 15) / 16 - 1;

    // The epilogue's row exponents and column scales (the transposed blocks' layout: lane l holds
    // row l % 16 and columns 4 (l / 16) + [0, 4) of each block), fetched first so their latency
    // hides under the main loop. Rows and columns past the edge read the last valid one and are
    // never stored.
    int32_t e[RB];
    v4f sc[CB];
#pragma unroll
    for (int r = 0; r < RB; r++) e[r] = exps[min(m0 + r * 16 + (lane & 15), M - 1)];
#pragma unroll
    for (int cb = 0; cb < CB; cb++)
#pragma unroll
        for (int v = 0; v < 4; v++) sc[cb][v] = scales[min(n0 + cb * 16 + 4 * (lane >> 4) + v, P * 16 - 1)];

    // Operand blocks of this wavefront: row block R of the QA at (R * KB + t) * 2048 (+1024 for
    // the lo digits), panel p of the weights at p * b_panel + t * b_blk.
    const uint8_t *ap[RB];
    const uint8_t *bp[CB];
#pragma unroll
    for (int r = 0; r < RB; r++) ap[r] = qf + (size_t)min(R0 + r, RLAST) * KB * 2048 + lane * 16;
#pragma unroll
    for (int cb = 0; cb < CB; cb++) bp[cb] = wv + (size_t)min(P0 + cb, P - 1) * b_panel + lane * 16;

    v4i acc_hi[RB][CB], acc_lo[RB][CB];
#pragma unroll
    for (int i = 0; i < RB; i++)
#pragma unroll
        for (int j = 0; j < CB; j++) acc_hi[i][j] = acc_lo[i][j] = v4i{0, 0, 0, 0};

    v4i fa[S][RB][2], fb[S][CB];
#define TG_LOAD(st, tt)                                                                                \
    do {                                                                                               \
        const size_t t_ = (size_t)(tt);                                                                \
        _Pragma("unroll") for (int r = 0; r < RB; r++) {                                               \
            fa[st][r][0] = *reinterpret_cast<const v4i *>(ap[r] + t_ * 2048);                          \
            fa[st][r][1] = *reinterpret_cast<const v4i *>(ap[r] + t_ * 2048 + 1024);                   \
        }                                                                                              \
        _Pragma("unroll") for (int cb = 0; cb < CB; cb++) fb[st][cb] =                                 \
            *reinterpret_cast<const v4i *>(bp[cb] + t_ * b_blk);                                       \
    } while (0)
#define TG_MMA(st)                                                                                     \
    do {                                                                                               \
        _Pragma("unroll") for (int r = 0; r < RB; r++)                                                 \
            _Pragma("unroll") for (int cb = 0; cb < CB; cb++) {                                        \
                acc_hi[r][cb] = __builtin_amdgcn_mfma_i32_16x16x64_i8(fb[st][cb], fa[st][r][0], acc_hi[r][cb], 0, 0, 0); \
                acc_lo[r][cb] = __builtin_amdgcn_mfma_i32_16x16x64_i8(fb[st][cb], fa[st][r][1], acc_lo[r][cb], 0, 0, 0); \
            }                                                                                          \
    } while (0)

    if (KB > 0) {
        // Ring of S register stages: block t sits in stage t % S. Loads past the end reload the
        // last block (in bounds, never used).
#pragma unroll
        for (int s = 0; s < S - 1; s++) TG_LOAD(s, min(s, KB - 1));
        int t = 0;
        for (; t + S <= KB; t += S) {
#pragma unroll
            for (int s = 0; s < S; s++) {
                TG_LOAD((s + S - 1) % S, min(t + s + S - 1, KB - 1));
                TG_MMA(s);
            }
        }
        // At most S - 1 blocks remain: block t + j is already in stage j.
#pragma unroll
        for (int j = 0; j < S - 1; j++)
            if (t + j < KB) TG_MMA(j);
    }
#undef TG_LOAD
#undef TG_MMA

    // Epilogue: the weights were the MFMAs' first operand, so each lane holds four consecutive
    // columns of one row per block and stores them from registers.
    store_transposed<1, RB, CB>(acc_hi, acc_lo, e, sc, lane, c, ldc, m0, n0, M, N, bias, act, escale, accumulate);
}

template <int RB, int CB, int S, int OCC, int XCD, int G>
hipError_t launch_tile(const uint8_t *qf, const int32_t *exps, size_t m, const DeviceWeights &w, float *c, size_t ldc,
                       const EpiArgs &epi, hipStream_t s) {
    const size_t bm = 2 * RB * 16, bn = 2 * CB * 16;
    dim3 grid((unsigned)div_ceil(w.panels * PANEL, bn), (unsigned)div_ceil(m, bm));
    hipLaunchKernelGGL((gemm_i8_kernel<RB, CB, S, OCC, XCD, G>), grid, dim3(THREADS), 0, s, qf, exps, (int)m, w.values,
                       w.scales, (int)w.n, (int)w.panels, (int)w.kb, c, ldc, epi.bias, epi.act, epi.scale,
                       epi.accumulate, w.panel_stride, w.blk_stride);
    return hipGetLastError();
}


// The k-split kernel for products with few output tiles. Each of the four wavefronts of a
// workgroup computes the whole 64 x 64 tile (4 row blocks x 4 panels) over every fourth k-block
// (wavefront w takes k-blocks w, w + 4, ...), so every operand byte crosses the CU's L1 once, where
// the 2 x 2 kernel loads each twice. The four integer partial sums are then combined through LDS:
// wavefront q keeps row block q, receives the other three wavefronts' sums for it and stores its
// 16 x 64 strip. The sums are exact integers, so the split changes no result.
template <int RB, int S, int XCD, int G>
__global__ __launch_bounds__(THREADS, 1) void gemm_i8_kq_kernel(const uint8_t *__restrict__ qf,
                                                                const int32_t *__restrict__ exps, int M,
                                                                const uint8_t *__restrict__ wv,
                                                                const float *__restrict__ scales, int N, int P, int KB,
                                                                float *__restrict__ c, size_t ldc,
                                                                const float *__restrict__ bias, uint32_t act,
                                                                float escale, int accumulate, size_t b_panel,
                                                                size_t b_blk) {
    static_assert(RB == 3 || RB == 4, "three or four row blocks: wavefront q < RB stores row block q");
    constexpr int CB = 4, WN = CB * 16, C_STRIDE = WN + 4;
    constexpr int SLOT = CB * 2 * 64;          // v4i per partial strip (one row block, hi and lo)
    constexpr int PARTS = RB * 3 * SLOT * 16;  // bytes: three strips for each row block
    constexpr int STAGE = 16 * C_STRIDE * 4;   // bytes of one wavefront's staged strip
    __shared__ __attribute__((aligned(16))) uint8_t smem[PARTS + 4 * STAGE];
    const int tid = threadIdx.x, lane = tid & 63, q = tid >> 6;
    int bx, by;
    tile_of<XCD, G>(bx, by);
    const int R0 = by * RB, P0 = bx * CB, RLAST = (M + 15) / 16 - 1;
    const int m0 = R0 * 16, n0 = P0 * 16;
    const int out_col = lane & 15, out_row = (lane >> 4) * 4;

    int32_t e_row[4];
    float s_col[CB];
#pragma unroll
    for (int v = 0; v < 4; v++) e_row[v] = exps[min(m0 + min(q, RB - 1) * 16 + out_row + v, M - 1)];
#pragma unroll
    for (int cb = 0; cb < CB; cb++) s_col[cb] = scales[min(n0 + cb * 16 + out_col, P * 16 - 1)];

    const int NB = KB > q ? (KB - q + 3) / 4 : 0;
    const uint8_t *ap[RB];
    const uint8_t *bp[CB];
#pragma unroll
    for (int r = 0; r < RB; r++) ap[r] = qf + ((size_t)min(R0 + r, RLAST) * KB + q) * 2048 + lane * 16;
#pragma unroll
    for (int cb = 0; cb < CB; cb++) bp[cb] = wv + (size_t)min(P0 + cb, P - 1) * b_panel + q * b_blk + lane * 16;

    v4i acc_hi[RB][CB], acc_lo[RB][CB];
#pragma unroll
    for (int i = 0; i < RB; i++)
#pragma unroll
        for (int j = 0; j < CB; j++) acc_hi[i][j] = acc_lo[i][j] = v4i{0, 0, 0, 0};

    v4i fa[S][RB][2], fb[S][CB];
#define TG_LOAD(st, ii)                                                                                \
    do {                                                                                               \
        const size_t t_ = (size_t)(ii) * 4;                                                            \
        _Pragma("unroll") for (int r = 0; r < RB; r++) {                                               \
            fa[st][r][0] = *reinterpret_cast<const v4i *>(ap[r] + t_ * 2048);                          \
            fa[st][r][1] = *reinterpret_cast<const v4i *>(ap[r] + t_ * 2048 + 1024);                   \
        }                                                                                              \
        _Pragma("unroll") for (int cb = 0; cb < CB; cb++) fb[st][cb] =                                 \
            *reinterpret_cast<const v4i *>(bp[cb] + t_ * b_blk);                                       \
    } while (0)
#define TG_MMA(st)                                                                                     \
    do {                                                                                               \
        _Pragma("unroll") for (int r = 0; r < RB; r++)                                                 \
            _Pragma("unroll") for (int cb = 0; cb < CB; cb++) {                                        \
                acc_hi[r][cb] = __builtin_amdgcn_mfma_i32_16x16x64_i8(fa[st][r][0], fb[st][cb], acc_hi[r][cb], 0, 0, 0); \
                acc_lo[r][cb] = __builtin_amdgcn_mfma_i32_16x16x64_i8(fa[st][r][1], fb[st][cb], acc_lo[r][cb], 0, 0, 0); \
            }                                                                                          \
    } while (0)

    if (NB > 0) {
        // Ring of S register stages: the wavefront's i-th block sits in stage i % S; loads past
        // the end reload its last block (in bounds, never used).
#pragma unroll
        for (int s = 0; s < S - 1; s++) TG_LOAD(s, min(s, NB - 1));
        int i = 0;
        for (; i + S <= NB; i += S) {
#pragma unroll
            for (int s = 0; s < S; s++) {
                TG_LOAD((s + S - 1) % S, min(i + s + S - 1, NB - 1));
                TG_MMA(s);
            }
        }
#pragma unroll
        for (int j = 0; j < S - 1; j++)
            if (i + j < NB) TG_MMA(j);
    }
#undef TG_LOAD
#undef TG_MMA

    // Wavefront q stores row block q; with three row blocks the fourth only contributes partials
    // (it still takes part in every barrier), its rows clamped to the tile's end, never stored.
    const bool stores = q < RB;
    const int mq = stores ? m0 + q * 16 : M;
    TileStore<16, WN, C_STRIDE> out;
    out.begin(lane, c, ldc, mq, n0, M, N, bias, accumulate);

    // Row block r's strip from wavefront w != r goes to slot (r, w - (w > r)).
    v4i *part = reinterpret_cast<v4i *>(smem);
#pragma unroll
    for (int r = 0; r < RB; r++) {
        if (r == q) continue;
        v4i *slot = part + (r * 3 + (q > r ? q - 1 : q)) * SLOT;
#pragma unroll
        for (int cb = 0; cb < CB; cb++) {
            slot[(cb * 2) * 64 + lane] = acc_hi[r][cb];
            slot[(cb * 2 + 1) * 64 + lane] = acc_lo[r][cb];
        }
    }
    v4i mine_hi[CB], mine_lo[CB];
#pragma unroll
    for (int cb = 0; cb < CB; cb++) {
        mine_hi[cb] = acc_hi[0][cb];
        mine_lo[cb] = acc_lo[0][cb];
#pragma unroll
        for (int r = 1; r < RB; r++)
            if (r == q) {
                mine_hi[cb] = acc_hi[r][cb];
                mine_lo[cb] = acc_lo[r][cb];
            }
    }
    __syncthreads();
#pragma unroll
    for (int w = 0; w < 3; w++) {
        const v4i *slot = part + (min(q, RB - 1) * 3 + w) * SLOT;
#pragma unroll
        for (int cb = 0; cb < CB; cb++) {
            mine_hi[cb] += slot[(cb * 2) * 64 + lane];
            mine_lo[cb] += slot[(cb * 2 + 1) * 64 + lane];
        }
    }

    // Epilogue: the strip (element v of lane l: row 4 (l / 16) + v, column l % 16 of each 16 x 16
    // block) is staged in the wavefront's own LDS area and stored in 16-byte runs.
    float *tile = reinterpret_cast<float *>(smem + PARTS + q * STAGE);
    {
        v4i hi1[1][CB], lo1[1][CB];
        int32_t e1[1][4] = {{e_row[0], e_row[1], e_row[2], e_row[3]}};
#pragma unroll
        for (int cb = 0; cb < CB; cb++) {
            hi1[0][cb] = mine_hi[cb];
            lo1[0][cb] = mine_lo[cb];
        }
        stage_sums<1, CB, C_STRIDE>(tile, hi1, lo1, e1, s_col, out_row, out_col);
    }
    __syncthreads();
    out.finish(tile, c, ldc, mq, M, N, bias != nullptr, act, escale, accumulate);
}

template <int RB, int S, int XCD, int G>
hipError_t launch_kq(const uint8_t *qf, const int32_t *exps, size_t m, const DeviceWeights &w, float *c, size_t ldc,
                     const EpiArgs &epi, hipStream_t s) {
    const dim3 grid((unsigned)div_ceil(w.panels, (size_t)4), (unsigned)div_ceil(div_ceil(m, (size_t)16), (size_t)RB));
    hipLaunchKernelGGL((gemm_i8_kq_kernel<RB, S, XCD, G>), grid, dim3(THREADS), 0, s, qf, exps, (int)m, w.values,
                       w.scales, (int)w.n, (int)w.panels, (int)w.kb, c, ldc, epi.bias, epi.act, epi.scale,
                       epi.accumulate, w.panel_stride, w.blk_stride);
    return hipGetLastError();
}


// ---------------------------------------------------------------------------- LDS-staged GEMM
//
// The workgroup's operands go from global memory straight into LDS with global_load_lds_dwordx4
// (no VGPRs, no ds_write): per k-block one stage of 2 TM + TN chunks of 1 KB in lane order (A: TM
// row blocks x hi, lo; B: TN panels), in a ring of NS buffers. Each wavefront moves a quarter of
// the chunks, waits for its own copies with s_waitcnt vmcnt, and a barrier makes the stage visible
// to all four; a buffer is refilled only after every wavefront has read it. The four wavefronts
// (2 x 2, each TM / 2 row blocks by TN / 2 panels) then read their MFMA operands with linear
// 16-byte LDS reads. Loading each operand once per workgroup instead of once per wavefront halves
// the L1 traffic of the direct kernel. Instances: 128 x 128 tiles in XCD order for products that
// fill the chip twice over; 64 x 64 tiles grouped four tile-rows at a time for mid-size products
// of at least 2048 outputs.

// The LDS address of p (the offset within the workgroup's LDS).
__device__ __forceinline__ uint32_t lds_address(const void *p) {
    return (uint32_t)(uintptr_t)(__attribute__((address_space(3))) const void *)p;
}

// 64 lanes x 16 bytes from base + voff (a wave-uniform base address in scalar registers plus each
// lane's byte offset) to LDS at lds (the wave-uniform LDS address; lane l's bytes land at lds +
// 16 l when voff = 16 l). M0 holds the LDS address; it is set before every copy and nothing else
// here uses it.
__device__ __forceinline__ void copy_to_lds_s(const uint8_t *base, uint32_t voff, uint32_t lds) {
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
    asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dwordx4 %1, %2" ::"s"(lds), "v"(voff), "s"(base) : "memory", "m0");
#pragma clang diagnostic pop
}

template <int N>
__device__ __forceinline__ void wait_copies() {
    static_assert(N >= 0 && N < 64, "vmcnt holds 6 bits");
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

// Waits until at most `ahead` stages of CPW copies each are still on the way (ahead <= A, with A
// = NS - 2 at the top of the recursion). `ahead` is uniform, so the branches are scalar.
template <int CPW, int A>
__device__ __forceinline__ void wait_stages(int ahead) {
    static_assert(A >= 0 && A * CPW < 64, "vmcnt holds 6 bits");
    if constexpr (A == 0) {
        wait_copies<0>();
    } else {
        if (ahead >= A) wait_copies<A * CPW>();
        else wait_stages<CPW, A - 1>(ahead);
    }
}

// The row maxima of gemm_lds_kernel<..., QOUT = 1>: for each row and workgroup column bx, the
// largest |y| over the workgroup's columns as unsigned bits (all ones when one of them is a NaN or
// an infinity), at tmax[row * strips + bx]; the streaming quantiser (launch_quantize_known) takes
// the row's exponent from them.
struct TileMax {
    uint32_t *tmax;
    int strips;
};

template <int TM, int TN, int NS, int XCD, int G, int GLU, int QOUT, int EDGE>
__global__ __launch_bounds__(THREADS, 2) void gemm_lds_kernel(const uint8_t *__restrict__ qf,
                                                              const int32_t *__restrict__ exps, int M,
                                                              const uint8_t *__restrict__ wv,
                                                              const float *__restrict__ scales, int N, int P, int KB,
                                                              float *__restrict__ c, size_t ldc,
                                                              const float *__restrict__ bias, uint32_t act,
                                                              float escale, int accumulate, size_t b_panel,
                                                              size_t b_blk, int hp, TileMax tmx) {
    constexpr int RB = TM / 2, CB = TN / 2;  // 16 x 16 blocks per wavefront
    constexpr int CH = 2 * TM + TN;          // 1 KB chunks per stage
    static_assert(CH % 4 == 0, "the chunks split evenly over four wavefronts");
    static_assert(NS >= 3, "block t + 1 lands while block t is multiplied, block t - 1's buffer refills");
    constexpr int CPW = CH / 4, STAGE = CH * 1024;
    constexpr int WM = RB * 16, WN = CB * 16, C_STRIDE = WN + 4;
    static_assert(4 * WM * C_STRIDE * 4 <= NS * STAGE, "the epilogue reuses the ring");
    __shared__ __attribute__((aligned(16))) uint8_t smem[NS * STAGE];
    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave & 1, wn = wave >> 1;
    int bx, by;
    tile_of<XCD, G>(bx, by);
    const int R0 = by * TM, P0 = bx * TN, RLAST = (M + 15) / 16 - 1;
    const int m0 = by * TM * 16 + wm * WM, n0 = bx * TN * 16 + wn * WN;
    const int out_col = lane & 15, out_row = (lane >> 4) * 4;
    // Weight panel of B chunk cc (0 <= cc < TN). GLU: the first TN / 2 chunks are panels of the
    // first half of the outputs and the rest their partners hp panels on, so the wavefronts with
    // wn = 0 hold the a half of a GLU and those with wn = 1 the b half of the same columns.
    auto panel_of = [&](int cc) {
        if constexpr (GLU) return cc < TN / 2 ? bx * (TN / 2) + cc : hp + bx * (TN / 2) + cc - TN / 2;
        return P0 + cc;
    };

    // The epilogue's row exponents and column scales, one per thread, loaded before the k-loop so
    // that their latency passes under it, and handed over through LDS after it. Rows and columns
    // past the edge read the last valid one and are never stored.
    constexpr int NPRE = TM * 16 + TN * 16;
    static_assert(NPRE <= THREADS, "one exponent or scale per thread");
    __shared__ __attribute__((aligned(16))) uint32_t s_pre[NPRE];
    uint32_t pre = 0u;
    if (tid < TM * 16) {
        pre = (uint32_t)exps[min(by * TM * 16 + tid, M - 1)];
    } else if (tid < NPRE) {
        const int j = tid - TM * 16;
        pre = __float_as_uint(scales[min(panel_of(j >> 4) * 16 + (j & 15), P * 16 - 1)]);
    }

    // This wavefront's copies: chunk ch = wave + 4 i is row block R0 + ch / 2, digit ch % 2 when
    // ch < 2 TM, else panel P0 + ch - 2 TM; rows and panels past the edge repeat the last one. The
    // bases are wave-uniform (scalar registers); each lane adds its 16 bytes' offset.
    const uint8_t *g[CPW];
    size_t gs[CPW];
#pragma unroll
    for (int i = 0; i < CPW; i++) {
        const int ch = wave + 4 * i;
        if (ch < 2 * TM) {
            g[i] = qf + (size_t)min(R0 + (ch >> 1), RLAST) * KB * 2048 + (ch & 1) * 1024;
            gs[i] = 2048;
        } else {
            g[i] = wv + (size_t)min(panel_of(ch - 2 * TM), P - 1) * b_panel;
            gs[i] = b_blk;
        }
    }
    const uint32_t voff = lane * 16, lds0 = __builtin_amdgcn_readfirstlane(lds_address(smem));
    auto issue = [&](int buf, int tt) {
#pragma unroll
        for (int i = 0; i < CPW; i++)
            copy_to_lds_s(g[i] + (size_t)tt * gs[i], voff, lds0 + buf * STAGE + (wave + 4 * i) * 1024);
    };
    // This wavefront's operands of one k-block from LDS buffer buf: row blocks wm * RB + r (hi and lo
    // digits) and panels wn * CB + cb.
    auto read_frags = [&](int buf, v4i (&fa)[RB][2], v4i (&fb)[CB]) {
        const uint8_t *st = smem + buf * STAGE;
#pragma unroll
        for (int cb = 0; cb < CB; cb++)
            fb[cb] = *reinterpret_cast<const v4i *>(st + 2 * TM * 1024 + (wn * CB + cb) * 1024 + lane * 16);
#pragma unroll
        for (int r = 0; r < RB; r++) {
            fa[r][0] = *reinterpret_cast<const v4i *>(st + ((wm * RB + r) * 2) * 1024 + lane * 16);
            fa[r][1] = *reinterpret_cast<const v4i *>(st + ((wm * RB + r) * 2 + 1) * 1024 + lane * 16);
        }
    };
    // TR (every product but the GLU): the weights are the first MFMA operand, so the accumulators
    // hold the transposed blocks that store_transposed writes out from registers. The GLU pairs
    // the two halves' sums through LDS and keeps the rows first.
    constexpr bool TR = !GLU;
    v4i acc_hi[RB][CB], acc_lo[RB][CB];
#pragma unroll
    for (int i = 0; i < RB; i++)
#pragma unroll
        for (int j = 0; j < CB; j++) acc_hi[i][j] = acc_lo[i][j] = v4i{0, 0, 0, 0};
    auto mma = [&](const v4i (&fa)[RB][2], const v4i (&fb)[CB]) {
#pragma unroll
        for (int r = 0; r < RB; r++)
#pragma unroll
            for (int cb = 0; cb < CB; cb++) {
                if constexpr (TR) {
                    acc_hi[r][cb] = __builtin_amdgcn_mfma_i32_16x16x64_i8(fb[cb], fa[r][0], acc_hi[r][cb], 0, 0, 0);
                    acc_lo[r][cb] = __builtin_amdgcn_mfma_i32_16x16x64_i8(fb[cb], fa[r][1], acc_lo[r][cb], 0, 0, 0);
                } else {
                    acc_hi[r][cb] = __builtin_amdgcn_mfma_i32_16x16x64_i8(fa[r][0], fb[cb], acc_hi[r][cb], 0, 0, 0);
                    acc_lo[r][cb] = __builtin_amdgcn_mfma_i32_16x16x64_i8(fa[r][1], fb[cb], acc_lo[r][cb], 0, 0, 0);
                }
            }
    };

    // k-block t sits in buffer t % NS. Two register sets of fragments: while the MFMAs of block t
    // run on one, block t + 1's fragments are read into the other, so the LDS latency passes under
    // the MFMAs. Iteration t waits for block t + 1's copies, and after the barrier (every
    // wavefront has consumed block t - 1's fragments) reuses block t - 1's buffer for block
    // t + NS - 1.
    v4i fa0[RB][2], fb0[CB], fa1[RB][2], fb1[CB];
#pragma unroll
    for (int s = 0; s < NS - 1; s++)
        if (s < KB) issue(s, s);
    wait_stages<CPW, NS - 2>(min(NS - 2, KB - 1));
    __syncthreads();
    read_frags(0, fa0, fb0);
    auto step = [&](int t, const v4i (&ca)[RB][2], const v4i (&cb)[CB], v4i (&na)[RB][2], v4i (&nb)[CB]) {
        if (t + 1 < KB) {
            wait_stages<CPW, NS - 3>(min(NS - 3, KB - 2 - t));
            __syncthreads();
            if (t + NS - 1 < KB) issue((t + NS - 1) % NS, t + NS - 1);
            read_frags((t + 1) % NS, na, nb);
        }
        mma(ca, cb);
    };
    int t = 0;
    for (; t + 1 < KB; t += 2) {
        step(t, fa0, fb0, fa1, fb1);
        step(t + 1, fa1, fb1, fa0, fb0);
    }
    if (t < KB) step(t, fa0, fb0, fa1, fb1);
    if (tid < NPRE) s_pre[tid] = pre;
    if constexpr (TR) {
        __syncthreads();  // s_pre
        int32_t e[RB];
        v4f sc[CB];
#pragma unroll
        for (int r = 0; r < RB; r++) e[r] = (int32_t)s_pre[wm * WM + r * 16 + (lane & 15)];
#pragma unroll
        for (int cb = 0; cb < CB; cb++)
            sc[cb] = *reinterpret_cast<const v4f *>(s_pre + TM * 16 + (wn * CB + cb) * 16 + 4 * (lane >> 4));
        if constexpr (QOUT) {
            // Each row's largest |y| over the workgroup's columns: over this wavefront's (the lanes
            // of a row), then over the two wavefronts of the row (LDS).
            __shared__ uint32_t smax[2][TM * 16];
            uint32_t rmax[RB];
            store_transposed<EDGE, RB, CB>(acc_hi, acc_lo, e, sc, lane, c, ldc, m0, n0, M, N, bias, act, escale,
                                           accumulate, rmax);
            if (lane < 16) {
#pragma unroll
                for (int r = 0; r < RB; r++) smax[wn][wm * WM + r * 16 + lane] = rmax[r];
            }
            __syncthreads();
            for (int rr = tid; rr < TM * 16; rr += THREADS) {
                const int row = by * TM * 16 + rr;
                if (row < M) tmx.tmax[(size_t)row * tmx.strips + bx] = max(smax[0][rr], smax[1][rr]);
            }
        } else {
            store_transposed<EDGE, RB, CB>(acc_hi, acc_lo, e, sc, lane, c, ldc, m0, n0, M, N, bias, act, escale,
                                           accumulate);
        }
        return;
    }
    __syncthreads();  // every wavefront is done with the ring before it holds the staged outputs
    int32_t e_row[RB][4];
    float s_col[CB];
#pragma unroll
    for (int r = 0; r < RB; r++)
#pragma unroll
        for (int v = 0; v < 4; v++) e_row[r][v] = (int32_t)s_pre[wm * WM + r * 16 + out_row + v];
#pragma unroll
    for (int cb = 0; cb < CB; cb++) s_col[cb] = __uint_as_float(s_pre[TM * 16 + (wn * CB + cb) * 16 + out_col]);

    float *tile = reinterpret_cast<float *>(smem) + wave * WM * C_STRIDE;
    stage_sums<RB, CB, C_STRIDE>(tile, acc_hi, acc_lo, e_row, s_col, out_row, out_col);
    __syncthreads();
    if constexpr (GLU) {
        // Wavefronts (wm, 0) and (wm, 1) hold the a and b halves of the same rows and columns; each
        // stores the GLU of half of those rows. c is the GLU output, hp * 16 columns wide.
        const float *ta = reinterpret_cast<const float *>(smem) + wm * WM * C_STRIDE + wn * (WM / 2) * C_STRIDE;
        glu_store<WM / 2, WN, C_STRIDE>(ta, ta + 2 * WM * C_STRIDE, lane, c, ldc, m0 + wn * (WM / 2), bx * WN, M,
                                        hp * 16, bias, act, escale);
    }
}

template <int TM, int TN, int NS, int XCD, int G, int GLU = 0, int QOUT = 0>
hipError_t launch_lds(const uint8_t *qf, const int32_t *exps, size_t m, const DeviceWeights &w, float *c, size_t ldc,
                      const EpiArgs &epi, hipStream_t s, const TileMax &q = TileMax{}) {
    static_assert(!QOUT || !GLU, "row maxima of plain products");
    // GLU: a workgroup column covers TN / 2 panels of each half (the launcher checks that they
    // divide the half's panels).
    const size_t hp = w.panels / 2, cols = GLU ? hp / (TN / 2) : div_ceil(w.panels, (size_t)TN);
    const dim3 grid((unsigned)cols, (unsigned)div_ceil(div_ceil(m, (size_t)16), (size_t)TM));
    // The FAST-only kernel when every tile is whole in columns and the outputs and bias are 16-byte
    // aligned; the GLU stores through LDS and has one kernel.
    auto kernel = &gemm_lds_kernel<TM, TN, NS, XCD, G, GLU, QOUT, 0>;
    if constexpr (!GLU) {
        const bool fast = ((reinterpret_cast<uintptr_t>(c) | ldc * sizeof(float) |
                            reinterpret_cast<uintptr_t>(epi.bias)) % 16) == 0 &&
                          w.n % (TN * PANEL) == 0;
        if (!fast) kernel = &gemm_lds_kernel<TM, TN, NS, XCD, G, GLU, QOUT, 1>;
    }
    hipLaunchKernelGGL(kernel, grid, dim3(THREADS), 0, s, qf, exps, (int)m, w.values, w.scales, (int)w.n,
                       (int)w.panels, (int)w.kb, c, ldc, epi.bias, epi.act, epi.scale, epi.accumulate, w.panel_stride,
                       w.blk_stride, (int)hp, q);
    return hipGetLastError();
}

// 64 lanes x 4 bytes from base + voff to LDS at lds + 4 l (lane l), as copy_to_lds_s.
__device__ __forceinline__ void copy_dword_to_lds_s(const uint8_t *base, uint32_t voff, uint32_t lds) {
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
    asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dword %1, %2" ::"s"(lds), "v"(voff), "s"(base) : "memory", "m0");
#pragma clang diagnostic pop
}

// Q8_0 weights: one scale per 32 inputs of each output. Each 32-input half of a k-block runs on
// v_mfma_i32_16x16x32_i8 from zero, giving the block's exact sums H (hi digits) and L (lo digits);
// T = 256 H + L (|T| < 2^31) is folded into an f32 accumulator as fmaf(d, (float)T, F), blocks in
// order, so k is never split. The 8-byte operands come from the same 1 KB k-block layouts as the
// int8 path: for half h, lane 16 g + x reads bytes 8 (g % 2) .. of layout lane 16 (2 h + g / 2) +
// x, i.e. inputs 32 h + 8 g .. + 8 of its row (A) or output (B), the same k for both operands.
//
// The operands travel on gemm_lds_kernel's ring. A stage holds one k-block: 2 TM + TN chunks of
// 1 KB (A: TM row blocks x hi, lo; B: TN panels) and the scales of the k-block's two 32-input
// blocks for the TN panels (128 bytes a panel), copied once per workgroup: each wavefront moves
// its share of the chunks and 256 bytes of scales (two panels: lanes 0-31 the first, lanes 32-63
// the second; lanes 16-31 of each the second block). The four wavefronts (2 x 2, TM / 2 row blocks
// by TN / 2 panels) read their operands and their columns' scales from LDS. When k is an odd
// number of blocks the last k-block's second block does not exist: its lanes copy the first
// block's scales, and its fold is skipped. Copying each operand once per workgroup, where
// wavefronts loading their own operands into registers load each twice, took the T = 750 Q8_0
// layer step from 0.250 to 0.224 ms on 64 x 64 tiles, and the smaller tiles the registers freed
// (more workgroups per CU on the narrower products) to 0.204 ms.
template <int TM, int TN, int NS, int XCD, int G, int GLU>
__global__ __launch_bounds__(THREADS, 2) void gemm_q8_lds_kernel(const uint8_t *__restrict__ qf,
                                                                 const int32_t *__restrict__ exps, int M,
                                                                 const uint8_t *__restrict__ wv,
                                                                 const float *__restrict__ scales, int N, int P,
                                                                 int KB, int NB, float *__restrict__ c, size_t ldc,
                                                                 const float *__restrict__ bias, uint32_t act,
                                                                 float escale, int accumulate, size_t b_panel,
                                                                 size_t b_blk, int hp) {
    constexpr int RB = TM / 2, CB = TN / 2;  // 16 x 16 blocks per wavefront
    constexpr int CH = 2 * TM + TN;          // 1 KB chunks per stage
    static_assert(TN <= 8, "four 256-byte scale copies cover eight panels");
    static_assert(!GLU || TN % 4 == 0, "a scale copy's two panels lie in one half of the GLU");
    static_assert(NS >= 3, "block t + 1 lands while block t is multiplied, block t - 1's buffer refills");
    // Chunk copies per wavefront: CPW for waves below FULL, CPW - 1 for the rest; each also copies
    // its 256 bytes of scales.
    constexpr int CPW = (CH + 3) / 4, FULL = CH - 4 * (CPW - 1), SC = CH * 1024, STAGE = SC + 1024;
    constexpr int WM = RB * 16, WN = CB * 16, C_STRIDE = WN + 4;
    static_assert(4 * WM * C_STRIDE * 4 <= NS * STAGE, "the epilogue reuses the ring");
    __shared__ __attribute__((aligned(16))) uint8_t smem[NS * STAGE];
    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave & 1, wn = wave >> 1;
    int bx, by;
    tile_of<XCD, G>(bx, by);
    const int R0 = by * TM, P0 = bx * TN, RLAST = (M + 15) / 16 - 1;
    const int m0 = by * TM * 16 + wm * WM, n0 = bx * TN * 16 + wn * WN;
    const int out_col = lane & 15, out_row = (lane >> 4) * 4, g = lane >> 4;
    // Weight panel of B chunk cc (0 <= cc < TN; past the edge, the last panel). GLU: the first
    // TN / 2 chunks are panels of the first half of the outputs and the rest their partners hp
    // panels on, so the wavefronts with wn = 0 hold the a half of a GLU and those with wn = 1 the b
    // half of the same columns (as gemm_lds_kernel's GLU).
    auto panel_of = [&](int cc) {
        if constexpr (GLU) return cc < TN / 2 ? bx * (TN / 2) + cc : hp + bx * (TN / 2) + cc - TN / 2;
        return min(P0 + cc, P - 1);
    };

    int32_t e_row[RB][4];
#pragma unroll
    for (int r = 0; r < RB; r++)
#pragma unroll
        for (int v = 0; v < 4; v++) e_row[r][v] = exps[min(m0 + r * 16 + out_row + v, M - 1)];

    // This wavefront's chunk copies (chunk ch = wave + 4 i: row block R0 + ch / 2, digit ch % 2 when
    // ch < 2 TM, else panel P0 + ch - 2 TM; rows and panels past the edge repeat the last one) and
    // its scale copy: lane l reads scales[((p NB + 2 t + b) 16 + j] for the panel p of chunk
    // 2 wave + l / 32 (the last chunk's past TN), block b = (l / 16) % 2 and column j = l % 16, as
    // the wave-uniform base (the panel of chunk 2 wave, block 2 t) plus a lane offset below
    // NB * 64 + 128 bytes (the two panels are consecutive or the same).
    const uint8_t *gp[CPW];
    size_t gs[CPW];
#pragma unroll
    for (int i = 0; i < CPW; i++) {
        const int ch = min(wave + 4 * i, CH - 1);
        if (ch < 2 * TM) {
            gp[i] = qf + (size_t)min(R0 + (ch >> 1), RLAST) * KB * 2048 + (ch & 1) * 1024;
            gs[i] = 2048;
        } else {
            gp[i] = wv + (size_t)panel_of(ch - 2 * TM) * b_panel;
            gs[i] = b_blk;
        }
    }
    const int s_first = panel_of(min(2 * wave, TN - 1)), s_blk = (lane >> 4) & 1;
    const int s_panel = panel_of(min(2 * wave + (lane >> 5), TN - 1)) - s_first;
    const uint32_t s_off = (uint32_t)(((s_panel * NB + s_blk) * PANEL + (lane & 15)) * sizeof(float));
    const uint32_t s_off_one = s_off - (uint32_t)(s_blk * PANEL * sizeof(float));
    const uint8_t *sbase = reinterpret_cast<const uint8_t *>(scales + (size_t)s_first * NB * PANEL);
    const uint32_t voff = lane * 16, lds0 = __builtin_amdgcn_readfirstlane(lds_address(smem));
    const bool full = wave < FULL;
    auto issue = [&](int buf, int tt) {
#pragma unroll
        for (int i = 0; i < CPW; i++)
            if (i < CPW - 1 || full)
                copy_to_lds_s(gp[i] + (size_t)tt * gs[i], voff, lds0 + buf * STAGE + (wave + 4 * i) * 1024);
        copy_dword_to_lds_s(sbase + (size_t)tt * 2 * PANEL * sizeof(float), 2 * tt + 1 < NB ? s_off : s_off_one,
                            lds0 + buf * STAGE + SC + wave * 256);
    };

    // Byte offsets, within a 1 KB chunk, of this lane's 8 bytes for halves 0 and 1.
    const int off0 = (16 * (g >> 1) + out_col) * 16 + 8 * (g & 1), off1 = off0 + 32 * 16;
    auto read_frags = [&](int buf, long (&fa)[RB][2][2], long (&fb)[CB][2], float (&fs)[CB][2]) {
        const uint8_t *st = smem + buf * STAGE;
#pragma unroll
        for (int cb = 0; cb < CB; cb++) {
            const uint8_t *b = st + 2 * TM * 1024 + (wn * CB + cb) * 1024;
            fb[cb][0] = *reinterpret_cast<const long *>(b + off0);
            fb[cb][1] = *reinterpret_cast<const long *>(b + off1);
            const float *sc = reinterpret_cast<const float *>(st + SC + (wn * CB + cb) * 128) + out_col;
            fs[cb][0] = sc[0];
            fs[cb][1] = sc[PANEL];
        }
#pragma unroll
        for (int r = 0; r < RB; r++)
#pragma unroll
            for (int d = 0; d < 2; d++) {
                const uint8_t *a = st + ((wm * RB + r) * 2 + d) * 1024;
                fa[r][d][0] = *reinterpret_cast<const long *>(a + off0);
                fa[r][d][1] = *reinterpret_cast<const long *>(a + off1);
            }
    };

    v4f acc[RB][CB];
#pragma unroll
    for (int i = 0; i < RB; i++)
#pragma unroll
        for (int j = 0; j < CB; j++) acc[i][j] = v4f{0.0f, 0.0f, 0.0f, 0.0f};
    // k-block t: the fold of its blocks 2 t and 2 t + 1 (the second only when it exists).
    auto mma = [&](int t, const long (&fa)[RB][2][2], const long (&fb)[CB][2], const float (&fs)[CB][2]) {
        const int halves = 2 * t + 1 < NB ? 2 : 1;
#pragma unroll
        for (int h = 0; h < 2; h++) {
            if (h >= halves) break;
#pragma unroll
            for (int r = 0; r < RB; r++)
#pragma unroll
                for (int cb = 0; cb < CB; cb++) {
                    const v4i hh = __builtin_amdgcn_mfma_i32_16x16x32_i8(fa[r][0][h], fb[cb][h], v4i{0, 0, 0, 0}, 0, 0, 0);
                    const v4i ll = __builtin_amdgcn_mfma_i32_16x16x32_i8(fa[r][1][h], fb[cb][h], v4i{0, 0, 0, 0}, 0, 0, 0);
#pragma unroll
                    for (int v = 0; v < 4; v++)
                        acc[r][cb][v] = __builtin_fmaf(fs[cb][h], (float)(hh[v] * 256 + ll[v]), acc[r][cb][v]);
                }
        }
    };

    // The ring as gemm_lds_kernel's: k-block t in buffer t % NS, block t + 1's fragments read from
    // LDS while block t's MFMAs run.
    if (KB > 0) {
        long fa0[RB][2][2], fb0[CB][2], fa1[RB][2][2], fb1[CB][2];
        float fs0[CB][2], fs1[CB][2];
#pragma unroll
        for (int s = 0; s < NS - 1; s++)
            if (s < KB) issue(s, s);
        // Waits until at most `ahead` stages of this wavefront's copies are still on the way.
        auto wait_ahead = [&](auto stages, int ahead) {
            constexpr int A = decltype(stages)::value;
            if (full) wait_stages<CPW + 1, A>(ahead);
            else wait_stages<CPW, A>(ahead);
        };
        wait_ahead(std::integral_constant<int, NS - 2>{}, min(NS - 2, KB - 1));
        __syncthreads();
        read_frags(0, fa0, fb0, fs0);
        auto step = [&](int t, const long (&ca)[RB][2][2], const long (&cb)[CB][2], const float (&cs)[CB][2],
                        long (&na)[RB][2][2], long (&nb)[CB][2], float (&ns)[CB][2]) {
            if (t + 1 < KB) {
                wait_ahead(std::integral_constant<int, NS - 3>{}, min(NS - 3, KB - 2 - t));
                __syncthreads();
                if (t + NS - 1 < KB) issue((t + NS - 1) % NS, t + NS - 1);
                read_frags((t + 1) % NS, na, nb, ns);
            }
            mma(t, ca, cb, cs);
        };
        int t = 0;
        for (; t + 1 < KB; t += 2) {
            step(t, fa0, fb0, fs0, fa1, fb1, fs1);
            step(t + 1, fa1, fb1, fs1, fa0, fb0, fs0);
        }
        if (t < KB) step(t, fa0, fb0, fs0, fa1, fb1, fs1);
    }

    TileStore<WM, WN, C_STRIDE> out;
    if constexpr (!GLU) out.begin(lane, c, ldc, m0, n0, M, N, bias, accumulate);
    __syncthreads();  // every wavefront is done with the ring before it holds the staged outputs
    float *tile = reinterpret_cast<float *>(smem) + wave * WM * C_STRIDE;
#pragma unroll
    for (int r = 0; r < RB; r++)
#pragma unroll
        for (int cb = 0; cb < CB; cb++)
#pragma unroll
            for (int v = 0; v < 4; v++) {
                const int32_t e = e_row[r][v];
                tile[(r * 16 + out_row + v) * C_STRIDE + cb * 16 + out_col] =
                    e == EXP_NONFINITE ? __builtin_nanf("") : __builtin_ldexpf(acc[r][cb][v], -e);
            }
    __syncthreads();
    if constexpr (GLU) {
        // Wavefronts (wm, 0) and (wm, 1) hold the a and b halves of the same rows and columns; each
        // stores the GLU of half of those rows. c is the GLU output, hp * 16 columns wide.
        const float *ta = reinterpret_cast<const float *>(smem) + wm * WM * C_STRIDE + wn * (WM / 2) * C_STRIDE;
        glu_store<WM / 2, WN, C_STRIDE>(ta, ta + 2 * WM * C_STRIDE, lane, c, ldc, m0 + wn * (WM / 2), bx * WN, M,
                                        hp * 16, bias, act, escale);
    } else {
        out.finish(tile, c, ldc, m0, M, N, bias != nullptr, act, escale, accumulate);
    }
}

// GLU: a workgroup column covers TN / 2 panels of each half (the caller checks that they divide the
// half's panels).
template <int TM, int TN, int NS, int XCD, int G, int GLU = 0>
hipError_t launch_q8_lds(const uint8_t *qf, const int32_t *exps, size_t m, const DeviceWeights &w, float *c,
                         size_t ldc, const EpiArgs &epi, hipStream_t s) {
    const size_t hp = w.panels / 2, cols = GLU ? hp / (TN / 2) : div_ceil(w.panels, (size_t)TN);
    const dim3 grid((unsigned)cols, (unsigned)div_ceil(div_ceil(m, (size_t)16), (size_t)TM));
    hipLaunchKernelGGL((gemm_q8_lds_kernel<TM, TN, NS, XCD, G, GLU>), grid, dim3(THREADS), 0, s, qf, exps, (int)m,
                       w.values, w.scales, (int)w.n, (int)w.panels, (int)w.kb, (int)(w.k / Q8_BLOCK), c, ldc,
                       epi.bias, epi.act, epi.scale, epi.accumulate, w.panel_stride, w.blk_stride, (int)hp);
    return hipGetLastError();
}

}  // namespace

// 128 x 128 workgroup tiles when there are at least 1024 of them (two per CU, twice over), else
// 64 x 64 tiles, which keep more CUs busy on short products.
int gemm_tile_choice(size_t m, size_t panels) {
    const size_t big = div_ceil(m, 128) * div_ceil(panels * PANEL, 128);
    return big >= 1024 ? 0 : 1;
}

hipError_t launch_gemm_i8(const uint8_t *qf, const int32_t *exps, size_t m, const DeviceWeights &w, float *c,
                          size_t ldc, const EpiArgs &epi, hipStream_t s) {
    if (m == 0 || w.n == 0) return hipSuccess;
    if (w.precision == Q8_0) {
        // LDS-staged tiles, in contiguous row-major runs per XCD (the rows the row kernels leave in
        // each XCD's L2): 64 x 64 from three per CU (750 x 1024 -> 4096, 768 tiles: 21.3 us against
        // 24.0 on 32 x 64), 32 x 64 from one per CU (750 x 1024 -> 3072 18.8 against 20.1 us,
        // x 1024 -> 2048 13.1 against 15.1), 32 x 32 below (750 x 4096 -> 1024, 768 workgroups:
        // 31.4 against 32.4 on 32 x 64, 36.4 on 96 x 32; 38.9 before LDS staging). Four-stage
        // rings were slower on both small tiles.
        const size_t tiles64 = div_ceil(m, (size_t)64) * div_ceil(w.panels, (size_t)4);
        if (tiles64 >= 3 * GFX950_CUS) return launch_q8_lds<4, 4, 3, 1, 0>(qf, exps, m, w, c, ldc, epi, s);
        if (tiles64 >= GFX950_CUS) return launch_q8_lds<2, 4, 3, 1, 0>(qf, exps, m, w, c, ldc, epi, s);
        return launch_q8_lds<2, 2, 3, 1, 0>(qf, exps, m, w, c, ldc, epi, s);
    }
    if (gemm_tile_choice(m, w.panels) == 0) return launch_lds<8, 8, 3, 1, 0>(qf, exps, m, w, c, ldc, epi, s);
    // Mid-size products: LDS staging pays from 2048 outputs (the direct kernel's duplicate operand
    // loads dominate there), on 128 x 128 tiles from 384 of them (each tile's operands copied once
    // for four times the 64 x 64 tile's work: 2000 x 1024 -> 4096 25.4 against 29.6 us, 3000 rows
    // 39.8 against 44.0, 1500 rows 23.0 against 24.9; at 256-288 tiles, 1000 x 1024 -> 4096 and
    // 1500 x 1024 -> 3072, the 64 x 64 tiles' fuller chip wins: 15.7 against 16.9, 20.6 against
    // 21.4 us). Narrower ones take 128 x 128 tiles once there are 256 of them (one per CU: 7500 x
    // 4096 -> 1024 runs 81 us against 123 us on the direct kernel), else the direct kernel, or the
    // k-split kernel when the inputs are long (at least 32 k-blocks) and the tiles too few to fill
    // the CUs twice.
    // The 64 x 64 tiles go to the XCDs in runs of four tile rows (tile_of<1, 4>: at 750 x 1024 ->
    // 4096 four rows by 24 columns per XCD), so that each XCD reads 1.5 of the 4 MB of weights
    // (12.1 against 13.5 us alone; with the k-split kernel's alike, the T = 750 layer step 0.1372 ->
    // 0.1359 ms on one GPU, the two measured in turn).
    // Below one 64 x 64 tile per CU the direct kernel's 32 x 64 tiles fill more of the chip (100 x
    // 1024 -> 4096 6.9 -> 5.1 us, 250 x 1024 -> 2048 7.1 -> 4.8 us; at 256 tiles and above the
    // LDS-staged tiles tie or win: 200 x 1024 -> 4096 7.1 / 7.2, 300 rows 8.1 / 9.8).
    const size_t tiles64 = div_ceil(m, (size_t)64) * div_ceil(w.n, (size_t)64);
    if (w.panels >= 128) {
        if (div_ceil(m, (size_t)128) * div_ceil(w.panels, (size_t)8) >= 384)
            return launch_lds<8, 8, 3, 1, 0>(qf, exps, m, w, c, ldc, epi, s);
        if (tiles64 < GFX950_CUS) return launch_tile<1, 2, 6, 4, 1, 0>(qf, exps, m, w, c, ldc, epi, s);
        return launch_lds<4, 4, 3, 1, 4>(qf, exps, m, w, c, ldc, epi, s);
    }
    if (div_ceil(m, (size_t)128) * div_ceil(w.panels, (size_t)8) >= 256)
        return launch_lds<8, 8, 3, 1, 0>(qf, exps, m, w, c, ldc, epi, s);
    if (w.kb >= 32 && div_ceil(m, (size_t)64) * div_ceil(w.panels, (size_t)4) < 512) {
        // 48-row tiles when their workgroups (one per CU) fit the chip in one round: every CU
        // busy and a quarter less work each (750 x 4096 -> 1024: 192 -> 256 workgroups, 15.7 ->
        // 14.2 us), with a six-stage register ring (four, five, seven, eight stages: 15.9, 15.1,
        // 14.9, 15.5 against 14.1 us), in runs of four tile rows by eight columns per XCD (each
        // XCD reads half the weights: 13.1 -> 11.4 us alone, against 14.2 / 13.0 for runs of two
        // or eight tile rows); else 64-row tiles (at 1000 rows 336 workgroups would take two
        // rounds: 25 against 16.4 us), and the LDS-staged 64 x 64 kernel once there are more than
        // 256 of those (1500 x 2048 -> 1024 20.5 -> 13.2 us; at 1000 x 4096 -> 1024, 256 tiles, the
        // k-split kernel keeps 17.5 against 19.5 us). With 64 k-blocks or more the 48-row tiles
        // also win when they fill two rounds at least seven eighths full (1500 x 4096 -> 1024: 512
        // workgroups, 25.1 us against 28.6 on 64 x 64 tiles and 32.1 on 64-row ones; 1440 rows
        // 25.4 against 30.1).
        const size_t wg3 = div_ceil(div_ceil(m, (size_t)16), (size_t)3) * div_ceil(w.panels, (size_t)4);
        if (wg3 <= GFX950_CUS || (w.kb >= 64 && wg3 <= 2 * GFX950_CUS && wg3 * 8 >= 2 * GFX950_CUS * 7))
            return launch_kq<3, 6, 1, 4>(qf, exps, m, w, c, ldc, epi, s);
        if (div_ceil(m, (size_t)64) * div_ceil(w.panels, (size_t)4) <= GFX950_CUS)
            return launch_kq<4, 5, 1, 0>(qf, exps, m, w, c, ldc, epi, s);
        return launch_lds<4, 4, 3, 1, 4>(qf, exps, m, w, c, ldc, epi, s);
    }
    // The direct kernel: 64 x 64 tiles when they give about one workgroup per CU (161 to 256 of
    // them), else 32 x 64 tiles, four workgroups per CU, on small grids (750 x 1024 -> 640: 6.3 ->
    // 4.9 us; 300 x 1024 -> 1000: 6.9 -> 5.4 us; 750 x 1024 -> 1024 keeps 64 x 64, 6.6 against
    // 7.3 us). Beyond 256 tiles of 64 x 64 the LDS-staged kernel on them (in runs of four tile rows
    // per XCD) copies each operand once per workgroup: 3000 x 1024 -> 1024 18.6 -> 13.4 us, 3000 x
    // 4096 -> 1024 54.9 -> 35.1 us, 1500 x 1024 -> 1024 10.4 -> 9.2 us against the 32 x 64 tiles.
    if (tiles64 > 160 && tiles64 <= GFX950_CUS) return launch_tile<2, 2, 6, 2, 1, 0>(qf, exps, m, w, c, ldc, epi, s);
    if (tiles64 > GFX950_CUS) return launch_lds<4, 4, 3, 1, 4>(qf, exps, m, w, c, ldc, epi, s);
    return launch_tile<1, 2, 6, 4, 1, 0>(qf, exps, m, w, c, ldc, epi, s);
}

// The product's f32 outputs and their row maxima per workgroup column (TileMax), on the tiles
// launch_gemm_i8 would pick: 128 x 128 when they fill the chip twice over, else 64 x 64.
int gemm_qout_strips(size_t m, const DeviceWeights &w) {
    return (int)div_ceil(w.panels, (size_t)(gemm_tile_choice(m, w.panels) == 0 ? 8 : 4));
}

hipError_t launch_gemm_i8_qout(const uint8_t *qf, const int32_t *exps, size_t m, const DeviceWeights &w,
                               const EpiArgs &epi, float *h, size_t ldh, uint32_t *tmax, hipStream_t s) {
    if (m == 0 || w.n == 0) return hipSuccess;
    if (w.precision != INT8 || epi.accumulate) return hipErrorInvalidValue;
    const TileMax q{tmax, gemm_qout_strips(m, w)};
    if (gemm_tile_choice(m, w.panels) == 0) return launch_lds<8, 8, 3, 1, 0, 0, 1>(qf, exps, m, w, h, ldh, epi, s, q);
    return launch_lds<4, 4, 3, 1, 0, 0, 1>(qf, exps, m, w, h, ldh, epi, s, q);
}

// The GLU-fused product: 128 x 128 tiles (four panels of each half) from 512 of them when the half
// has a multiple of 64 outputs, else 64 x 64 tiles (two panels of each half), which need a multiple
// of 32 (x 1024 -> 2048: 7500 rows 43.0 against 49.2 us, 6000 rows 36.0 against 39.3; at 3000
// rows, 384 tiles, 21.4 against 20.8), and 32 x 64 tiles below two 64 x 64 tiles per CU (750 x
// 1024 -> 2048: 7.6 against 8.1 us, the T = 750 layer step 0.1383 -> 0.1367 ms; at 750 x 1024 ->
// 4096 and 1500 rows the 64 x 64 tiles keep 11.8 against 12.2 and 11.4 against 12.6 us).
bool gemm_glu_fits(size_t n) { return n % 64 == 0; }

hipError_t launch_gemm_i8_glu(const uint8_t *qf, const int32_t *exps, size_t m, const DeviceWeights &w, float *out,
                              size_t ldo, const EpiArgs &epi, hipStream_t s) {
    if (m == 0 || w.n == 0) return hipSuccess;
    if ((w.precision != INT8 && w.precision != Q8_0) || !gemm_glu_fits(w.n)) return hipErrorInvalidValue;
    if (w.precision == Q8_0) {
        // The Q8_0 product's tiles (64 x 64 from three per CU, else 32 x 64: the 32 x 32 tiles' one
        // panel per wavefront column cannot hold both halves).
        if (div_ceil(m, (size_t)64) * div_ceil(w.panels, (size_t)4) >= 3 * GFX950_CUS)
            return launch_q8_lds<4, 4, 3, 1, 0, 1>(qf, exps, m, w, out, ldo, epi, s);
        return launch_q8_lds<2, 4, 3, 1, 0, 1>(qf, exps, m, w, out, ldo, epi, s);
    }
    const size_t half = w.n / 2;
    if (half % 64 == 0 && div_ceil(m, (size_t)128) * div_ceil(w.panels, (size_t)8) >= 512)
        return launch_lds<8, 8, 3, 1, 0, 1>(qf, exps, m, w, out, ldo, epi, s);
    if (div_ceil(m, (size_t)64) * div_ceil(w.panels, (size_t)4) < 2 * GFX950_CUS)
        return launch_lds<2, 4, 3, 1, 0, 1>(qf, exps, m, w, out, ldo, epi, s);
    return launch_lds<4, 4, 3, 1, 0, 1>(qf, exps, m, w, out, ldo, epi, s);
}

}  // namespace tg
