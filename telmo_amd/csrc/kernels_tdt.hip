// The greedy TDT decode of Parakeet (src/parakeet.rs:1412-1577) with every step on the device: the
// joint, both argmaxes, the blank / duration bookkeeping, the prediction network's LSTM layers and
// its projection run as one chain of kernels per step, with no host round trip per token.
//
// Each kernel is the GEMV of gemv_core.hpp with its own input rows and outputs: the dot4 body for
// the one-row products of int8 weights (the LSTM layers and the projection of a decode step), the
// MFMA body for the joint's window of frames, for predictions of several rows and for Q8_0; int8
// predictions of up to eight rows split each panel's k-blocks over a workgroup. No kernel
// waits for, or counts, the workgroups of its own grid: what a step decides is computed from one
// kernel's outputs by the next kernel, after the boundary between them has made them visible.
//
// * tdt_joint_kernel scores a window of up to TDT_ROWS consecutive frames t, t + 1, ... against
//   the same prediction in one GEMV (z = relu(enc_proj[f] + pred), the joint's bias): a row's logits
//   do not depend on the other rows, so this equals that many separate joints while the prediction
//   is unchanged. Each workgroup leaves, per row, the best vocabulary entry of its panels; the
//   first and the duration logits are kept as well. Workgroup 0 snapshots the control block.
// * tdt_lstm_kernel, layer 0 of the decode, first decides the step in every workgroup alike from
//   the joint's partials and the snapshot: the rows' tokens and durations, then the frames walked as
//   the reference's loop does (blank: skip max(duration, 1) frames; a token: record it, hand it to
//   the prediction network, move by its duration) until a token is emitted, the window is used up
//   or the frames end. Workgroup 0 publishes the outcome. The window shrinks after a token (tokens
//   come close together) and grows back over blanks.
// * tdt_lstm_kernel runs layer l on weights whose rows are interleaved at set-up (output 4 u + q is
//   gate q of unit u), so the four gates of a unit land in four adjacent lanes of one MFMA output
//   and the cell update happens in the epilogue. The state is read from one buffer and written to
//   the other (the decode flips between them), so no workgroup reads a state another has replaced.
// * tdt_proj_kernel writes pred = W_p h_last + b_p.
#include "gemv_core.hpp"

namespace tg {

namespace {

using gemv::v4f;

constexpr int TDT_WAVES = 4;
constexpr int TDT_THREADS = TDT_WAVES * 64;
constexpr int TDT_MAX_GRID = 1024;  // workgroups of a persistent GEMV grid
constexpr int TDT_EXTRA = 1 + TDT_MAX_DURATIONS;  // per joint row: the first logit, the duration logits

struct Best {
    float v;
    int i;
};

// Whether (v, i) comes before (bv, bi) in the reference's argmax (the first largest value; a NaN is
// never larger, so NaN entries lose to everything). An empty best is (NaN, INT32_MAX).
__device__ __forceinline__ bool before(float v, int i, float bv, int bi) {
    if (__builtin_isnan(v)) return false;
    if (__builtin_isnan(bv)) return true;
    return v > bv || (v == bv && i < bi);
}

__device__ __forceinline__ int load_i(const int32_t *p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void store_i(int32_t *p, int v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Joint input row r: relu(enc_proj[min(t + r, frames - 1)] + pred), as (e + p).max(0.0).
struct JointIn {
    const float *enc;
    size_t lde;
    const float *pred;
    int t, frames;
    __device__ __forceinline__ v4f load(int r, int i0, int m, int k) const {
        const bool ok = r < m && i0 < k;
        const int f = min(t + r, frames - 1);
        const v4f e = *reinterpret_cast<const v4f *>(ok ? enc + (size_t)f * lde + i0 : gemv::ZERO_CHUNK);
        const v4f p = *reinterpret_cast<const v4f *>(ok ? pred + i0 : gemv::ZERO_CHUNK);
        v4f z;
        z.x = fmaxf(e.x + p.x, 0.0f);
        z.y = fmaxf(e.y + p.y, 0.0f);
        z.z = fmaxf(e.z + p.z, 0.0f);
        z.w = fmaxf(e.w + p.w, 0.0f);
        return z;
    }
};

// Joint outputs: per lane the best vocabulary entry of its four rows so far; the first logit and the
// duration logits of each row go to extras (row r at r * TDT_EXTRA: first, then the durations).
struct JointOut {
    float *extras;
    int vocab;
    float bv[4];
    int bi[4];
    __device__ __forceinline__ void store(int r, int col, float v) {
        if (col < vocab) {
            if (before(v, col, bv[r & 3], bi[r & 3])) {
                bv[r & 3] = v;
                bi[r & 3] = col;
            }
            if (col == 0) extras[r * TDT_EXTRA] = v;
        } else {
            extras[r * TDT_EXTRA + 1 + (col - vocab)] = v;
        }
    }
};

// LSTM layer l input row r: [x; h_l] with x = embedding[tok[r]] (l = 0) or the new h_{l-1} (from
// the output state). The tokens sit in LDS (a register array indexed by row would live in scratch
// memory).
struct LstmIn {
    const float *emb;
    const float *s_in, *s_out;
    size_t width;
    int h, l;
    const int *tok;
    __device__ __forceinline__ v4f load(int r, int i0, int m, int k) const {
        const bool ok = r < m && i0 < k;
        const int rr = ok ? r : 0;
        const size_t row = (size_t)rr * width;
        const float *src = i0 < h ? (l == 0 ? emb + (size_t)tok[rr] * h + i0 : s_out + row + (size_t)(l - 1) * 2 * h + i0)
                                  : s_in + row + (size_t)l * 2 * h + (i0 - h);
        return *reinterpret_cast<const v4f *>(ok ? src : gemv::ZERO_CHUNK);
    }
};

__device__ __forceinline__ float sigmoid(float x) { return 1.0f / (1.0f + expf(0.0f - x)); }

// The value of quad lane Q (0..3) in every lane of the quad (DPP quad_perm [Q, Q, Q, Q]).
template <int Q>
__device__ __forceinline__ float quad_lane(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), Q * 0x55, 0xF, 0xF, false));
}

// LSTM outputs on interleaved rows: output col = 4 u + q is gate q (i, f, g, o) of unit u. The four
// lanes of a quad hold one unit's gates for the same row; lane q = 0 applies the cell update
// (src/parakeet.rs:1549-1562): c = f c + i g, h = o tanh(c), each product rounded before the sum.
struct LstmOut {
    const float *s_in;
    float *s_out;
    size_t width;
    int h, l;
    __device__ __forceinline__ void store(int r, int col, float v) {
        const float gi = quad_lane<0>(v), gf = quad_lane<1>(v), gg = quad_lane<2>(v), go = quad_lane<3>(v);
        if ((col & 3) == 0) {
            const size_t at = (size_t)r * width + (size_t)l * 2 * h + (col >> 2);
            const float i = sigmoid(gi), f = sigmoid(gf), g = tanhf(gg), o = sigmoid(go);
            const float c = f * s_in[at + h] + i * g;
            s_out[at + h] = c;
            s_out[at] = o * tanhf(c);
        }
    }
};

struct Weights {
    const uint8_t *values;
    const float *scales;
    int n, k, P, KB, NB;
    size_t panel_stride, blk_stride;
};

template <int KBC, int J, int Q8>
__global__ __launch_bounds__(TDT_THREADS) void tdt_joint_kernel(TdtCtl *ctl, const float *__restrict__ enc, size_t lde,
                                                                const float *__restrict__ pred, int frames, Weights w,
                                                                const float *__restrict__ bias, int vocab,
                                                                Best *partials, float *extras) {
    extern __shared__ __attribute__((aligned(16))) uint8_t sqa[];
    __shared__ uint32_t slot[TDT_WAVES * J];
    __shared__ Best red[TDT_WAVES][TDT_ROWS];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const bool lead = blockIdx.x == 0 && tid == 0;
    // The control values head the chain: they are requested first, the weights (which do not depend
    // on them) right after, so that waiting for the control values never waits for the weights.
    const int done = load_i(&ctl->done), t = load_i(&ctl->t), rows = load_i(&ctl->rows);
    gemv::Panel<KBC, Q8> pn;
    gemv::fetch_first<TDT_WAVES, KBC, Q8>(pn, 1, w.values, w.scales, w.n, w.P, w.KB, w.NB, extras, 0, bias, 0,
                                          w.panel_stride, w.blk_stride);
    if (done) {
        if (lead) store_i(&ctl->snap.valid, 0);
        return;
    }
    if (t >= frames) {
        // Only the last prediction's state flip is left: the decode ends here.
        if (lead) {
            if (load_i(&ctl->active)) store_i(&ctl->cur, load_i(&ctl->cur) ^ 1);
            store_i(&ctl->active, 0);
            store_i(&ctl->done, 1);
            store_i(&ctl->snap.valid, 0);
        }
        return;
    }
    if (lead) {
        store_i(&ctl->snap.t, t);
        store_i(&ctl->snap.rows, rows);
        store_i(&ctl->snap.on_frame, load_i(&ctl->on_frame));
        store_i(&ctl->snap.ntok, load_i(&ctl->ntok));
        store_i(&ctl->snap.active, load_i(&ctl->active));
        store_i(&ctl->snap.cur, load_i(&ctl->cur));
        store_i(&ctl->snap.valid, 1);
    }
    JointOut out{extras, vocab, {}, {}};
#pragma unroll
    for (int v = 0; v < 4; v++) {
        out.bv[v] = __builtin_nanf("");
        out.bi[v] = INT32_MAX;
    }
    gemv::mfma_body_pre<TDT_WAVES, KBC, J, Q8>(JointIn{enc, lde, pred, t, frames}, out, rows, w.k, w.values, w.scales,
                                           w.n, w.P, w.KB, w.NB, extras, 0, bias, ACT_NONE, 1.0f, 0,
                                           w.panel_stride, w.blk_stride, sqa, slot, pn);
    // Lanes 16 g .. 16 g + 15 hold 16 columns of rows 4 g .. 4 g + 3: fold them, then the wavefronts.
#pragma unroll
    for (int v = 0; v < 4; v++) {
        float bv = out.bv[v];
        int bi = out.bi[v];
#pragma unroll
        for (int off = 1; off < 16; off <<= 1) {
            const float ov = __shfl_xor(bv, off, 64);
            const int oi = __shfl_xor(bi, off, 64);
            if (before(ov, oi, bv, bi)) {
                bv = ov;
                bi = oi;
            }
        }
        if ((lane & 15) == 0) red[wave][(lane >> 4) * 4 + v] = Best{bv, bi};
    }
    __syncthreads();
    if (tid < TDT_ROWS) {
        Best b = red[0][tid];
#pragma unroll
        for (int q = 1; q < TDT_WAVES; q++)
            if (before(red[q][tid].v, red[q][tid].i, b.v, b.i)) b = red[q][tid];
        partials[(size_t)blockIdx.x * TDT_ROWS + tid] = b;
    }
}

// What the decider of a step reads besides the control block.
struct Decide {
    const Best *partials;
    const float *extras;
    int joint_grid, vocab, blank, ndur, max_symbols, frames, cap;
    const int32_t *durations;
    int32_t *tokens;
};

// The step's decision, computed alike in every workgroup of the kernel after the joint (so it needs
// no communication between them). Every load it makes is independent of the others (the snapshot,
// the joint's partials, the first and duration logits of all TDT_ROWS rows, the durations), so they
// are all issued before any is used: one memory round trip. Returns the token handed to the
// prediction network, -1 when the step hands none on, or -2 when the joint made no step (the
// decode had ended); the state buffer to read is left in *cur. Workgroup 0 publishes the new
// control values.
__device__ __forceinline__ int decide_step(TdtCtl *ctl, const Decide &d, int *cur) {
    __shared__ int tok_s[TDT_ROWS], dur_s[TDT_ROWS], durs[TDT_MAX_DURATIONS], result;
    __shared__ float dlog[TDT_ROWS][TDT_MAX_DURATIONS];
    const int tid = threadIdx.x;
    // Thread (r, s) takes row r's partials of workgroups s, s + 16, ... (sixteen loads per round,
    // one round up to 256 joint workgroups), with the row's first and duration logits. Rows the
    // window does not hold are read as well (the buffers hold TDT_ROWS rows) and never used. The
    // partials and logits are requested first, the snapshot after them: a wait for a snapshot value
    // then covers only loads the decision needs anyway.
    const int r = tid >> 4, s = tid & 15, nb = d.joint_grid;
    const float *ex = d.extras + (size_t)r * TDT_EXTRA;
    Best x0[16];
#pragma unroll
    for (int u = 0; u < 16; u++) x0[u] = d.partials[(size_t)min(s + 16 * u, nb - 1) * TDT_ROWS + r];
    const float first = ex[0];
    float dl[4];
#pragma unroll
    for (int q = 0; q < 4; q++) dl[q] = ex[1 + min(s + 16 * q, d.ndur - 1)];
    const int dur_v = d.durations[min(tid, d.ndur - 1)];
    const int valid = load_i(&ctl->snap.valid);
    const int t = load_i(&ctl->snap.t), rows = load_i(&ctl->snap.rows);
    const int snap_cur = load_i(&ctl->snap.cur), snap_active = load_i(&ctl->snap.active);
    const int snap_on = load_i(&ctl->snap.on_frame), snap_ntok = load_i(&ctl->snap.ntok);
    {
        float bv = __builtin_nanf("");
        int bi = INT32_MAX;
#pragma unroll
        for (int u = 0; u < 16; u++)
            if (s + 16 * u < nb && before(x0[u].v, x0[u].i, bv, bi)) {
                bv = x0[u].v;
                bi = x0[u].i;
            }
        for (int b0 = s + 16 * 16; b0 < nb; b0 += 16 * 16) {
            Best x[16];
#pragma unroll
            for (int u = 0; u < 16; u++) x[u] = d.partials[(size_t)min(b0 + 16 * u, nb - 1) * TDT_ROWS + r];
#pragma unroll
            for (int u = 0; u < 16; u++)
                if (b0 + 16 * u < nb && before(x[u].v, x[u].i, bv, bi)) {
                    bv = x[u].v;
                    bi = x[u].i;
                }
        }
#pragma unroll
        for (int off = 1; off < 16; off <<= 1) {
            const float ov = __shfl_xor(bv, off, 64);
            const int oi = __shfl_xor(bi, off, 64);
            if (before(ov, oi, bv, bi)) {
                bv = ov;
                bi = oi;
            }
        }
        if (tid < d.ndur) durs[tid] = dur_v;
#pragma unroll
        for (int q = 0; q < 4; q++)
            if (s + 16 * q < d.ndur) dlog[r][s + 16 * q] = dl[q];
        if (s == 0) tok_s[r] = __builtin_isnan(first) || bi == INT32_MAX ? 0 : bi;  // a NaN first is never beaten
    }
    if (!valid) return -2;  // uniform: the joint made no step
    *cur = snap_cur ^ snap_active;  // the last prediction wrote the other buffer
    __syncthreads();
    if (tid < TDT_ROWS) {
        int k = 0;
        for (int i = 1; i < d.ndur; i++)
            if (dlog[tid][i] > dlog[tid][k]) k = i;
        dur_s[tid] = durs[k];
    }
    __syncthreads();
    if (tid == 0) {
        int tc = t, on = snap_on, ntok = snap_ntok, token = -1, done = 0;
        // The next window: after a token, twice the frames this one walked (at least 4); after a
        // window of blanks, the most.
        int next = TDT_ROWS;
        while (true) {
            const int r = tc - t;
            if (r >= rows) break;  // the next window scores the frames from tc
            const int tok = tok_s[r], dur = dur_s[r];
            if (tok == d.blank) {
                tc += max(dur, 1);
                on = 0;
                if (tc >= d.frames) {
                    done = 1;
                    break;
                }
                continue;
            }
            if (blockIdx.x == 0 && ntok < d.cap) {
                d.tokens[3 * ntok] = tok;
                d.tokens[3 * ntok + 1] = tc;
                d.tokens[3 * ntok + 2] = dur;
            }
            ntok++;
            token = tok;
            next = min(TDT_ROWS, max(4, 2 * (r + 1)));
            if (dur > 0) {
                tc += dur;
                on = 0;
            } else if (++on >= d.max_symbols) {
                tc += 1;
                on = 0;
            }
            break;
        }
        if (blockIdx.x == 0) {
            store_i(&ctl->t, tc);
            store_i(&ctl->on_frame, on);
            store_i(&ctl->ntok, ntok);
            store_i(&ctl->rows, next);
            store_i(&ctl->cur, *cur);
            store_i(&ctl->active, token >= 0);
            store_i(&ctl->done, done);
        }
        result = token;
    }
    __syncthreads();
    return result;
}

// State buffers of a prediction: a (rows x width) is read and b written when cur is 0, the other
// way round when it is 1. mode 0: a standalone prediction (cur 0, tokens by value); 1: a later layer
// of the decode (runs when a token was handed on); 2: layer 0 of the decode, which decides the step.
template <int KBC, int J, int Q8, int DOTR = 0, int KS = 1>
__global__ __launch_bounds__(TDT_THREADS) void tdt_lstm_kernel(TdtCtl *ctl, int mode, TdtTokens toks, Decide dec,
                                                               int m, int l, const float *__restrict__ emb,
                                                               float *sa, float *sb, size_t width, Weights w,
                                                               const float *__restrict__ bias) {
    extern __shared__ __attribute__((aligned(16))) uint8_t sqa[];
    __shared__ uint32_t slot[TDT_WAVES * J];
    __shared__ int tok_s[TDT_ROWS];
    const int h = w.k / 2;
    int cur = 0;
    if (mode == 1) {
        if (!load_i(&ctl->active)) return;
        cur = load_i(&ctl->cur);
    }
    if (mode == 2) {
        const int token = decide_step(ctl, dec, &cur);
        if (token < 0) return;
        if (threadIdx.x == 0) tok_s[0] = token;
    } else if (mode == 0) {
        if (threadIdx.x < TDT_ROWS) tok_s[threadIdx.x] = toks.tok[threadIdx.x];
    }
    __syncthreads();
    float *s_in = cur ? sb : sa, *s_out = cur ? sa : sb;
    LstmOut out{s_in, s_out, width, h, l};
    gemv::mfma_body<TDT_WAVES, KBC, J, Q8, LstmIn, LstmOut, DOTR, KS>(LstmIn{emb, s_in, s_out, width, h, l, tok_s}, out, m,
                                                                  w.k, w.values, w.scales, w.n, w.P, w.KB, w.NB, s_out,
                                                                  width, bias, ACT_NONE, 1.0f, 0, w.panel_stride,
                                                                  w.blk_stride, sqa, slot);
}

template <int KBC, int J, int Q8, int DOTR = 0, int KS = 1>
__global__ __launch_bounds__(TDT_THREADS) void tdt_proj_kernel(TdtCtl *ctl, int gated, int m, const float *sa,
                                                               const float *sb, size_t width, int layers, Weights w,
                                                               const float *__restrict__ bias, float *preds) {
    extern __shared__ __attribute__((aligned(16))) uint8_t sqa[];
    __shared__ uint32_t slot[TDT_WAVES * J];
    if (gated && !load_i(&ctl->active)) return;
    const float *s_out = (gated && load_i(&ctl->cur)) ? sa : sb;
    const int h = w.k;
    gemv::StoreC out{preds, (size_t)h};
    gemv::mfma_body<TDT_WAVES, KBC, J, Q8, gemv::RowsIn, gemv::StoreC, DOTR, KS>(
        gemv::RowsIn{s_out + (size_t)(layers - 1) * 2 * h, width}, out, m, w.k, w.values, w.scales, w.n, w.P, w.KB,
        w.NB, preds, (size_t)h, bias, ACT_NONE, 1.0f, 0, w.panel_stride, w.blk_stride, sqa, slot);
}

// Interleaves the rows of an LSTM matrix (4h outputs, gate-major: gate q of unit u at q h + u) so
// that output 4 u + q is gate q of unit u: a gather of the 16-byte lane operands within each
// k-block, and of the scales alike. One wavefront per (panel, k-block).
__global__ __launch_bounds__(64) void tdt_interleave_kernel(const uint8_t *__restrict__ src, uint8_t *__restrict__ dst,
                                                            const float *__restrict__ ssrc, float *__restrict__ sdst,
                                                            const float *__restrict__ bsrc, float *__restrict__ bdst,
                                                            int h, int KB, int NB, int q8, size_t panel_stride,
                                                            size_t blk_stride) {
    const int p = blockIdx.x / KB, t = blockIdx.x % KB, lane = threadIdx.x, g = lane >> 4, j = lane & 15;
    const int o = 16 * p + j, old = (o & 3) * h + (o >> 2), po = old >> 4, jo = old & 15;
    const uint4 v = *reinterpret_cast<const uint4 *>(src + (size_t)po * panel_stride + (size_t)t * blk_stride +
                                                     (size_t)(16 * g + jo) * 16);
    *reinterpret_cast<uint4 *>(dst + (size_t)p * panel_stride + (size_t)t * blk_stride + (size_t)lane * 16) = v;
    if (g == 0) {
        if (q8) {
            for (int b = t; b < NB; b += KB)
                sdst[((size_t)p * NB + b) * PANEL + j] = ssrc[((size_t)po * NB + b) * PANEL + jo];
        } else if (t == 0) {
            sdst[o] = ssrc[old];
        }
        if (t == 0) bdst[o] = bsrc[old];
    }
}

Weights weights_of(const DeviceWeights &d) {
    return Weights{d.values, d.scales, (int)d.n, (int)d.k, (int)d.panels, (int)d.kb, (int)(d.k / Q8_BLOCK),
                   d.panel_stride, d.blk_stride};
}

// Persistent grid as the plain MFMA GEMV sizes it: at most 1024 workgroups walking the panels.
unsigned grid_of(const DeviceWeights &d) {
    const size_t per_wave = div_ceil(d.panels, (size_t)TDT_WAVES * TDT_MAX_GRID);
    return (unsigned)div_ceil(d.panels, (size_t)TDT_WAVES * per_wave);
}

// Chunk registers per thread for m rows of k inputs: m * ceil(kb / 4) chunk wavefronts over 4.
int j_of(size_t m, const DeviceWeights &d) {
    const size_t j = div_ceil(m * div_ceil(d.kb, (size_t)4), (size_t)TDT_WAVES);
    return j <= 2 ? 2 : j <= 4 ? 4 : j <= 8 ? 8 : j <= 12 ? 12 : j <= 16 ? 16 : 20;
}

// The k-blocks fetched ahead: all of them up to 20 (one memory round trip for Parakeet's LSTM rows
// of 1280 inputs), 16 per round beyond.
#define TG_TDT_KBC(KERNEL, KBC, ...)                                                                          \
    do {                                                                                                      \
        if (jj_ == 2) hipLaunchKernelGGL(q8_ ? (KERNEL<KBC, 2, 1>) : (KERNEL<KBC, 2, 0>), g_, b_, lds_, s, __VA_ARGS__);          \
        else if (jj_ == 4) hipLaunchKernelGGL(q8_ ? (KERNEL<KBC, 4, 1>) : (KERNEL<KBC, 4, 0>), g_, b_, lds_, s, __VA_ARGS__);     \
        else if (jj_ == 8) hipLaunchKernelGGL(q8_ ? (KERNEL<KBC, 8, 1>) : (KERNEL<KBC, 8, 0>), g_, b_, lds_, s, __VA_ARGS__);     \
        else if (jj_ == 12) hipLaunchKernelGGL(q8_ ? (KERNEL<KBC, 12, 1>) : (KERNEL<KBC, 12, 0>), g_, b_, lds_, s, __VA_ARGS__);  \
        else if (jj_ == 16) hipLaunchKernelGGL(q8_ ? (KERNEL<KBC, 16, 1>) : (KERNEL<KBC, 16, 0>), g_, b_, lds_, s, __VA_ARGS__);  \
        else hipLaunchKernelGGL(q8_ ? (KERNEL<KBC, 20, 1>) : (KERNEL<KBC, 20, 0>), g_, b_, lds_, s, __VA_ARGS__);                 \
    } while (0)

// Predictions of int8 weights and up to eight rows: one workgroup per panel with the panel's
// k-blocks split over its four wavefronts (the GEMV's k-split), the dot4 body for one row (ONE).
// Q8_0 weights take the persistent MFMA grid of TG_TDT_DISPATCH.
#define TG_TDT_KS_J(KERNEL, KBC, ...)                                                                         \
    do {                                                                                                      \
        if (jj_ == 2) hipLaunchKernelGGL(dot_ ? (KERNEL<KBC, 2, 0, 1, 4>) : (KERNEL<KBC, 2, 0, 0, 4>), g_, b_, lds_, s, __VA_ARGS__);        \
        else if (jj_ == 4) hipLaunchKernelGGL(dot_ ? (KERNEL<KBC, 4, 0, 1, 4>) : (KERNEL<KBC, 4, 0, 0, 4>), g_, b_, lds_, s, __VA_ARGS__);   \
        else if (jj_ == 8) hipLaunchKernelGGL(dot_ ? (KERNEL<KBC, 8, 0, 1, 4>) : (KERNEL<KBC, 8, 0, 0, 4>), g_, b_, lds_, s, __VA_ARGS__);   \
        else if (jj_ == 12) hipLaunchKernelGGL(dot_ ? (KERNEL<KBC, 12, 0, 1, 4>) : (KERNEL<KBC, 12, 0, 0, 4>), g_, b_, lds_, s, __VA_ARGS__); \
        else hipLaunchKernelGGL(dot_ ? (KERNEL<KBC, 16, 0, 1, 4>) : (KERNEL<KBC, 16, 0, 0, 4>), g_, b_, lds_, s, __VA_ARGS__);                \
    } while (0)

#define TG_TDT_DISPATCH_KS(KERNEL, JJ, D, ONE, ...)                      \
    do {                                                                 \
        const bool dot_ = (ONE);                                         \
        const size_t lds_ = (D).kb * 2048, kq_ = div_ceil((D).kb, (size_t)4); \
        const dim3 g_((unsigned)(D).panels), b_(TDT_THREADS);            \
        const int jj_ = (JJ);                                            \
        if (kq_ <= 3) TG_TDT_KS_J(KERNEL, 3, __VA_ARGS__);               \
        else if (kq_ <= 5) TG_TDT_KS_J(KERNEL, 5, __VA_ARGS__);          \
        else TG_TDT_KS_J(KERNEL, 8, __VA_ARGS__);                        \
    } while (0)

// Whether a prediction of m rows on these weights takes the k-split launch.
bool tdt_split(size_t m, const DeviceWeights &d) {
    return d.precision == INT8 && m <= 8 && d.panels <= (size_t)TDT_MAX_GRID && j_of(m, d) <= 16;
}

#define TG_TDT_DISPATCH(KERNEL, JJ, D, ...)                              \
    do {                                                                 \
        const bool q8_ = (D).precision == Q8_0;                          \
        const size_t lds_ = (D).kb * 2048;                               \
        const dim3 g_(grid_of(D)), b_(TDT_THREADS);                      \
        const int jj_ = (JJ);                                            \
        if ((D).kb <= 10) TG_TDT_KBC(KERNEL, 10, __VA_ARGS__);           \
        else if ((D).kb <= 20) TG_TDT_KBC(KERNEL, 20, __VA_ARGS__);      \
        else TG_TDT_KBC(KERNEL, 16, __VA_ARGS__);                        \
    } while (0)

}  // namespace

size_t tdt_max_rows(const DeviceWeights &lstm) {
    const size_t spr = div_ceil(lstm.kb, (size_t)4);
    const size_t rows = (size_t)TDT_WAVES * 20 / spr;
    return rows < (size_t)TDT_ROWS ? rows : (size_t)TDT_ROWS;
}

size_t tdt_partials_bytes() { return (size_t)TDT_MAX_GRID * TDT_ROWS * sizeof(Best); }

hipError_t launch_tdt_interleave(const DeviceWeights &src, const float *bias, const DeviceWeights &dst,
                                 float *bias_dst, size_t h, hipStream_t s) {
    hipLaunchKernelGGL(tdt_interleave_kernel, dim3((unsigned)(src.panels * src.kb)), dim3(64), 0, s, src.values,
                       dst.values, src.scales, dst.scales, bias, bias_dst, (int)h, (int)src.kb,
                       (int)(src.k / Q8_BLOCK), src.precision == Q8_0 ? 1 : 0, src.panel_stride, src.blk_stride);
    return hipGetLastError();
}

hipError_t launch_tdt_predict(TdtCtl *ctl, const TdtTokens &toks, size_t m, const TdtNet &net, float *sa, float *sb,
                              float *preds, hipStream_t s) {
    const size_t width = net.layers * 2 * net.h;
    const Decide none{};
    for (size_t l = 0; l < net.layers; l++) {
        const DeviceWeights &d = *net.lstm[l];
        if (tdt_split(m, d))
            TG_TDT_DISPATCH_KS(tdt_lstm_kernel, j_of(m, d), d, m == 1, ctl, 0, toks, none, (int)m, (int)l, net.emb, sa,
                               sb, width, weights_of(d), net.lstm_b[l]);
        else
            TG_TDT_DISPATCH(tdt_lstm_kernel, j_of(m, d), d, ctl, 0, toks, none, (int)m, (int)l, net.emb, sa, sb, width,
                            weights_of(d), net.lstm_b[l]);
    }
    const DeviceWeights &p = *net.proj;
    if (tdt_split(m, p))
        TG_TDT_DISPATCH_KS(tdt_proj_kernel, j_of(m, p), p, m == 1, ctl, 0, (int)m, sa, sb, width, (int)net.layers,
                           weights_of(p), net.proj_b, preds);
    else
        TG_TDT_DISPATCH(tdt_proj_kernel, j_of(m, p), p, ctl, 0, (int)m, sa, sb, width, (int)net.layers, weights_of(p),
                        net.proj_b, preds);
    return hipGetLastError();
}

hipError_t launch_tdt_step(TdtCtl *ctl, const TdtNet &net, const float *enc, size_t lde, int frames, float *sa,
                           float *sb, float *pred, void *partials, float *extras, int32_t *tokens, int cap,
                           hipStream_t s) {
    const DeviceWeights &d = *net.joint;
    TG_TDT_DISPATCH(tdt_joint_kernel, j_of(TDT_ROWS, d), d, ctl, enc, lde, pred, frames, weights_of(d), net.joint_b,
                    (int)net.vocab, static_cast<Best *>(partials), extras);
    const Decide dec{static_cast<const Best *>(partials), extras, (int)grid_of(d), (int)net.vocab, (int)net.blank,
                     (int)net.ndur, (int)net.max_symbols, frames, cap, net.durations, tokens};
    const size_t width = net.layers * 2 * net.h;
    for (size_t l = 0; l < net.layers; l++) {
        const DeviceWeights &w = *net.lstm[l];
        if (tdt_split(1, w))
            TG_TDT_DISPATCH_KS(tdt_lstm_kernel, j_of(1, w), w, true, ctl, l == 0 ? 2 : 1, TdtTokens{}, dec, 1, (int)l,
                               net.emb, sa, sb, width, weights_of(w), net.lstm_b[l]);
        else
            TG_TDT_DISPATCH(tdt_lstm_kernel, j_of(1, w), w, ctl, l == 0 ? 2 : 1, TdtTokens{}, dec, 1, (int)l, net.emb,
                            sa, sb, width, weights_of(w), net.lstm_b[l]);
    }
    const DeviceWeights &p = *net.proj;
    if (tdt_split(1, p))
        TG_TDT_DISPATCH_KS(tdt_proj_kernel, j_of(1, p), p, true, ctl, 1, 1, sa, sb, width, (int)net.layers,
                           weights_of(p), net.proj_b, pred);
    else
        TG_TDT_DISPATCH(tdt_proj_kernel, j_of(1, p), p, ctl, 1, 1, sa, sb, width, (int)net.layers, weights_of(p),
                        net.proj_b, pred);
    return hipGetLastError();
}

size_t tdt_extras_bytes() { return (size_t)TDT_ROWS * TDT_EXTRA * sizeof(float); }

}  // namespace tg
