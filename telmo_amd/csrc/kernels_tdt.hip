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
#include <algorithm>

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

// Where a window's walk leaves the decode: the frame, tokens on it, tokens emitted, the token handed
// to the prediction network (-1: none), the next window's rows and whether the frames are used up.
struct Walked {
    int t, on, ntok, token, rows, done;
};

// The reference's loop over the window's rows (src/parakeet.rs:1412-1577): a blank skips
// max(duration, 1) frames; a token is recorded (when record is set and the buffer has room), handed
// to the prediction network and moves the frame by its duration, or counts towards max_symbols on
// its frame. The walk stops at the first token, at the end of the window or of the frames. The next
// window: after a token, twice the frames this one walked (at least 4); after a window of blanks,
// the most.
__device__ __forceinline__ Walked walk_window(int t, int rows, int on, int ntok, const int *tok_s, const int *dur_s,
                                              int blank, int frames, int max_symbols, int32_t *tokens, int cap,
                                              bool record) {
    int tc = t, token = -1, done = 0, next = TDT_ROWS;
    while (true) {
        const int r = tc - t;
        if (r >= rows) break;  // the next window scores the frames from tc
        const int tok = tok_s[r], dur = dur_s[r];
        if (tok == blank) {
            tc += max(dur, 1);
            on = 0;
            if (tc >= frames) {
                done = 1;
                break;
            }
            continue;
        }
        if (record && ntok < cap) {
            tokens[3 * ntok] = tok;
            tokens[3 * ntok + 1] = tc;
            tokens[3 * ntok + 2] = dur;
        }
        ntok++;
        token = tok;
        next = min(TDT_ROWS, max(4, 2 * (r + 1)));
        if (dur > 0) {
            tc += dur;
            on = 0;
        } else if (++on >= max_symbols) {
            tc += 1;
            on = 0;
        }
        break;
    }
    return Walked{tc, on, ntok, token, next, done};
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
        const Walked w = walk_window(t, rows, snap_on, snap_ntok, tok_s, dur_s, d.blank, d.frames, d.max_symbols,
                                     d.tokens, d.cap, blockIdx.x == 0);
        if (blockIdx.x == 0) {
            store_i(&ctl->t, w.t);
            store_i(&ctl->on_frame, w.on);
            store_i(&ctl->ntok, w.ntok);
            store_i(&ctl->rows, w.rows);
            store_i(&ctl->cur, *cur);
            store_i(&ctl->active, w.token >= 0);
            store_i(&ctl->done, w.done);
        }
        result = w.token;
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

// ------------------------------------------------------------------------------ the resident decode
//
// One cooperative launch makes up to ResArgs::steps decode steps with every matrix held in LDS: each
// workgroup copies its panels of the joint, of every LSTM layer and of the projection once, and a
// step then reads only the rows it scores. The step's stages are those of the kernels above (the
// joint over a window of frames, the decision in every workgroup alike, the LSTM layers with the
// cell update, the projection), with the same integer sums and the same f32 epilogues.
//
// Workgroups hand each other values through 8-byte words: a value and the tag of the step or
// prediction that wrote it, stored and loaded as one agent-scope atomic. A reader waits until every
// word it needs carries the tag it expects; no counter or barrier spans workgroups. Each kind of word
// has two buffers, alternating with the tag's parity, and a buffer is rewritten two tags on: every
// workgroup writes a joint word for every row of every step after its previous decision, and a
// decision needs all of them, so no buffer is rewritten while a reader still needs its values. Every
// wait has a deadline (and watches the error flag): a wait that passes it sets the flag and ends the
// launch, so every workgroup exits.

constexpr int RES_WAVES = 4;
constexpr int RES_THREADS = RES_WAVES * 64;
constexpr int RES_MAX_PANELS = 8;  // panels of one matrix per workgroup
constexpr int RES_MAX_GRID = 256;  // workgroups: a row's sixteen decider threads read sixteen words each
// Copies of every hand-over word: workgroup b reads copy b % RES_COPIES (its XCD, as workgroups are
// dealt to the eight XCDs in turn), so each word's line has about an eighth of the readers.
constexpr int RES_COPIES = 8;
constexpr int RES_DEC = 6;  // words of a decision: frame, tokens on it, tokens emitted, token, rows, done
constexpr uint32_t TAG_NONE = 0xffffffffu;

struct ResMat {
    const uint8_t *values;
    const float *scales, *bias;
    size_t panel_stride, blk_stride;
    int n, KB, P;
    int NB;  // Q8_0: 32-input blocks (k / 32); scales [(p NB + b) 16 + j]
};

struct ResArgs {
    ResMat joint, proj, lstm[TDT_MAX_LAYERS];
    const float *emb, *enc;
    size_t lde;
    const int32_t *durations;
    int32_t *tokens;
    TdtCtl *ctl;
    float *state, *pred;
    // Hand-over words in RES_COPIES copies, cs words apart, of: the prediction [2][h], the LSTM
    // outputs h [layers][2][h] and the decision [2][RES_DEC]; in the first copy only, each
    // workgroup's best vocabulary entry per joint row [2][TDT_ROWS][RES_MAX_GRID] and the
    // duration-holding joint workgroups' best duration entries [2][TDT_ROWS][TDT_ROWS], which only
    // workgroup 0 reads.
    uint64_t *w_pred, *w_h, *w_part, *w_dur, *w_dec;
    size_t cs;
    int h, vocab, ndur, layers, blank, max_symbols, frames, cap;
    // Workgroups 0 .. GP - 1 hold the projection's panels, PP each; workgroups qoff + j hold joint
    // panels (j < GJ, JP each) and LSTM panels (j < GL, LP of every layer each).
    int JP, GJ, LP, GL, PP, GP, qoff, grid;
    int steps;
    uint64_t wait_ticks;  // the longest wait, in wall-clock ticks
};

__device__ __forceinline__ uint64_t word_load(const uint64_t *p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void word_store(uint64_t *p, uint64_t v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// Stores v into every copy of a word.
__device__ __forceinline__ void word_store_all(uint64_t *p, size_t stride, uint64_t v) {
#pragma unroll
    for (int c = 0; c < RES_COPIES; c++) word_store(p + c * stride, v);
}
__device__ __forceinline__ uint64_t tagged(float v, uint32_t tag) {
    return ((uint64_t)tag << 32) | __float_as_uint(v);
}
__device__ __forceinline__ float word_value(uint64_t w) { return __uint_as_float((uint32_t)w); }
// A candidate of the resident decode's argmaxes as integers: k orders the values (larger k, larger
// value; 0 for NaN, which never wins, and for no entry), i is the index (0xffffffff: none). The
// reference's scan keeps the first of equal largest values: the larger k wins, then the smaller i.
struct Key {
    uint32_t k, i;
};
__device__ __forceinline__ uint32_t order_key(float v) {
    const uint32_t u = __float_as_uint(v);
    if (__builtin_isnan(v)) return 0u;
    if (u == 0x80000000u) return 0x80000000u;  // -0 equals +0
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}
__device__ __forceinline__ bool better(Key a, Key b) { return a.k > b.k || (a.k == b.k && a.i < b.i); }
template <int CTRL>
__device__ __forceinline__ uint32_t dpp_u32(uint32_t x) {
    return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, CTRL, 0xF, 0xF, false);
}
// The best candidate of each row of 16 lanes, in all 16: the largest k (a DPP max over quad_perm
// [1,0,3,2], [2,3,0,1], row_half_mirror, row_mirror), then the smallest i among the lanes holding it.
__device__ __forceinline__ Key fold16(Key x) {
    uint32_t m = x.k;
    m = max(m, dpp_u32<0xB1>(m));
    m = max(m, dpp_u32<0x4E>(m));
    m = max(m, dpp_u32<0x141>(m));
    m = max(m, dpp_u32<0x140>(m));
    uint32_t i = x.k == m ? x.i : 0xffffffffu;
    i = min(i, dpp_u32<0xB1>(i));
    i = min(i, dpp_u32<0x4E>(i));
    i = min(i, dpp_u32<0x141>(i));
    i = min(i, dpp_u32<0x140>(i));
    return Key{m, i};
}
__device__ __forceinline__ uint64_t tagged_key(Key x, uint32_t step) {
    return ((uint64_t)(step & 0xffffu) << 48) | ((uint64_t)(x.i & 0xffffu) << 32) | x.k;
}
__device__ __forceinline__ Key key_of(uint64_t w) {
    const uint32_t i = (uint32_t)(w >> 32) & 0xffffu;
    return Key{(uint32_t)w, i == 0xffffu ? 0xffffffffu : i};
}

// dequant, through its int32 form when the wavefront voted that every hi sum fits (the same value).
__device__ __forceinline__ float dequant_w(int32_t hi, int32_t lo, int32_t e, float sc, bool fits) {
    return fits ? dequant_i32(hi, lo, e, sc) : dequant(hi, lo, e, sc);
}

// v summed over lanes l, l ^ 16, l ^ 32, l ^ 48: v_permlane16_swap / v_permlane32_swap exchange
// rows 1 and 3 of one operand with rows 0 and 2 (halves 1 and 0) of the other; with both operands
// v, the two results of each lane are its own value and its partner's.
__device__ __forceinline__ int sum_groups(int v) {
    const auto a = __builtin_amdgcn_permlane16_swap((unsigned)v, (unsigned)v, false, false);
    v = (int)(a[0] + a[1]);
    const auto b = __builtin_amdgcn_permlane32_swap((unsigned)v, (unsigned)v, false, false);
    return (int)(b[0] + b[1]);
}

// Waits until word i (bit i of need) carries tag[i], reloading the words still pending each round.
// False when the deadline passes or another workgroup has set the error flag.
template <int N>
__device__ __forceinline__ bool wait_words(const uint64_t *const (&p)[N], uint32_t need, const uint32_t (&tag)[N],
                                           uint64_t (&w)[N], const int32_t *err, uint64_t deadline) {
    for (int round = 0;; round++) {
#pragma unroll
        for (int i = 0; i < N; i++)
            if (need >> i & 1) w[i] = word_load(p[i]);
#pragma unroll
        for (int i = 0; i < N; i++)
            if ((need >> i & 1) && (uint32_t)(w[i] >> 32) == tag[i]) need &= ~(1u << i);
        if (!need) return true;
        if ((round & 15) == 15 && ((uint64_t)wall_clock64() > deadline || load_i(err) != 0)) return false;
    }
}

// Copies np panels from p0 on of a matrix into LDS, panel pi's k-block t at (pi KB + t) * 1024.
__device__ __forceinline__ void copy_panels(uint8_t *dst, const ResMat &m, int p0, int np) {
    const int per = m.KB * 64, total = np * per;
    for (int i0 = 0; i0 < total; i0 += RES_THREADS * 8) {
        gemv::v4i v[8];
#pragma unroll
        for (int u = 0; u < 8; u++) {
            const int i = min(i0 + u * RES_THREADS + (int)threadIdx.x, total - 1);
            const int pi = i / per, rem = i - pi * per;
            v[u] = *reinterpret_cast<const gemv::v4i *>(m.values + (size_t)(p0 + pi) * m.panel_stride +
                                                        (size_t)(rem >> 6) * m.blk_stride + (rem & 63) * 16);
        }
#pragma unroll
        for (int u = 0; u < 8; u++) {
            const int i = i0 + u * RES_THREADS + (int)threadIdx.x;
            if (i < total) {
                const int pi = i / per, rem = i - pi * per;
                *reinterpret_cast<gemv::v4i *>(dst + ((size_t)pi * m.KB + (rem >> 6)) * 1024 + (rem & 63) * 16) = v[u];
            }
        }
    }
}

// The LDS of a resident workgroup besides its panels.
struct ResShared {
    float js[RES_MAX_PANELS * PANEL], jbias[RES_MAX_PANELS * PANEL];
    float ps[RES_MAX_PANELS * PANEL], pbias[RES_MAX_PANELS * PANEL], pst[RES_MAX_PANELS * PANEL];
    float ls[TDT_MAX_LAYERS][RES_MAX_PANELS * PANEL], lbias[TDT_MAX_LAYERS][RES_MAX_PANELS * PANEL];
    float hst[TDT_MAX_LAYERS][RES_MAX_PANELS * 4], cst[TDT_MAX_LAYERS][RES_MAX_PANELS * 4];
    __attribute__((aligned(16))) float pin[TDT_MAX_H];  // the prediction the joint adds
    Key red[RES_WAVES][TDT_ROWS], dred[RES_WAVES][TDT_ROWS];
    Key cand[RES_THREADS / 16], dcand[RES_THREADS / 16];  // the decider's 16-lane group bests
    int32_t kpart[RES_WAVES][2][PANEL];
    int32_t erow[TDT_ROWS];
    uint32_t slot[RES_WAVES];
    int tok_s[TDT_ROWS], dur_s[TDT_ROWS], durs[TDT_MAX_DURATIONS];
    int dec[6];
    int abort;
};

__device__ __forceinline__ void res_fail(const ResArgs &a, ResShared &sh) {
    sh.abort = 1;
    store_i(&a.ctl->err, 1);
}

// The exponent of a row from the workgroup's four wavefront maxima in sh.slot.
__device__ __forceinline__ int32_t res_exponent(const ResShared &sh) {
    const uint32_t m = max(max(sh.slot[0], sh.slot[1]), max(sh.slot[2], sh.slot[3]));
    return m == 0xffffffffu ? EXP_NONFINITE : row_exponent_of(__uint_as_float(m));
}

// The largest |x| of a chunk as bits, all ones for a non-finite input (as the GEMV's row maxima).
__device__ __forceinline__ uint32_t chunk_max(v4f v) {
    const bool bad = !__builtin_isfinite(v.x) | !__builtin_isfinite(v.y) | !__builtin_isfinite(v.z) |
                     !__builtin_isfinite(v.w);
    const float mx = fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w)));
    return bad ? 0xffffffffu : __float_as_uint(mx);
}

// One row of k = 4 CK inputs whose chunk c (inputs 4c .. 4c + 3) thread c % 256 holds in x[c / 256]:
// the row exponent, then the digits in the one-row layout (k-block t, 16-input group g: hi at
// sq + 128 t + 16 g, lo 64 bytes on), zero past the row up to KB k-blocks.
template <int NC>
__device__ __forceinline__ int32_t row_digits(const v4f (&x)[NC], int CK, int KB, uint8_t *sq, ResShared &sh) {
    const int tid = threadIdx.x;
    uint32_t mx = 0;
#pragma unroll
    for (int i = 0; i < NC; i++)
        if (tid + RES_THREADS * i < CK) mx = max(mx, chunk_max(x[i]));
    const uint32_t m = gemv::wave_max_u(mx);
    if ((tid & 63) == 0) sh.slot[tid >> 6] = m;
    __syncthreads();
    const int32_t e = res_exponent(sh);
#pragma unroll
    for (int i = 0; i < NC; i++) {
        const int c = tid + RES_THREADS * i;
        if (c < KB * 16) {
            const v4f v = c < CK ? x[i] : v4f{0.0f, 0.0f, 0.0f, 0.0f};
            uint32_t hi, lo;
            digits4(v.x, v.y, v.z, v.w, e, hi, lo);
            uint8_t *d = sq + (c >> 4) * 128 + ((c & 15) >> 2) * 16 + (c & 3) * 4;
            *reinterpret_cast<uint32_t *>(d) = hi;
            *reinterpret_cast<uint32_t *>(d + 64) = lo;
        }
    }
    __syncthreads();
    return e;
}

// Copies the Q8_0 block scales of np panels from p0 on into LDS (panel pi's at (pi NB + b) 16 + j).
__device__ __forceinline__ void copy_q8_scales(float *dst, const ResMat &m, int p0, int np) {
    const int total = np * m.NB * PANEL;
    for (int i = threadIdx.x; i < total; i += RES_THREADS) dst[i] = m.scales[(size_t)p0 * m.NB * PANEL + i];
}

// row_sums for Q8_0 weights: the sums of each 32-input block b (k-block t = b / 2, lane groups 2 (b %
// 2) and 2 (b % 2) + 1) as T = 256 H + L, left in tq[b 16 + j]; lanes j < 16 of wavefront 0 then fold
// F = fmaf(d_b, T_b, F) over the NB blocks in order from +0 (the integer oracle's order) and return
// F (other lanes: 0). ds holds the panel's block scales.
__device__ __forceinline__ float row_fold_q8(const uint8_t *pw, int KB, int NB, const float *ds, const uint8_t *sq,
                                             int32_t *tq) {
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    for (int t = wave; t < KB; t += RES_WAVES) {
        const gemv::v4i ahi = *reinterpret_cast<const gemv::v4i *>(sq + t * 128 + (lane >> 4) * 16);
        const gemv::v4i alo = *reinterpret_cast<const gemv::v4i *>(sq + t * 128 + 64 + (lane >> 4) * 16);
        const gemv::v4i wv = *reinterpret_cast<const gemv::v4i *>(pw + (size_t)t * 1024 + lane * 16);
        int dh = 0, dl = 0;
        dh = __builtin_amdgcn_sdot4(ahi.x, wv.x, dh, false);
        dh = __builtin_amdgcn_sdot4(ahi.y, wv.y, dh, false);
        dh = __builtin_amdgcn_sdot4(ahi.z, wv.z, dh, false);
        dh = __builtin_amdgcn_sdot4(ahi.w, wv.w, dh, false);
        dl = __builtin_amdgcn_sdot4(alo.x, wv.x, dl, false);
        dl = __builtin_amdgcn_sdot4(alo.y, wv.y, dl, false);
        dl = __builtin_amdgcn_sdot4(alo.z, wv.z, dl, false);
        dl = __builtin_amdgcn_sdot4(alo.w, wv.w, dl, false);
        dh += __shfl_xor(dh, 16, 64);  // groups 2 h' and 2 h' + 1: the 32 inputs of block 2 t + h'
        dl += __shfl_xor(dl, 16, 64);
        if (((lane >> 4) & 1) == 0) tq[(2 * t + (lane >> 5)) * PANEL + (lane & 15)] = dh * 256 + dl;
    }
    __syncthreads();
    // The fold in block order, its operands read from LDS sixteen blocks at a time (then eight, then
    // one) so that the chain of fused multiply-adds does not wait on a read per block (sixteen
    // against eight: 20.10 -> 19.99 us per token of the Q8_0 decode; twenty, 20.02).
    float f = 0.0f;
    if (wave == 0 && lane < PANEL) {
        int b = 0;
        for (; b + 16 <= NB; b += 16) {
            float dv[16];
            int32_t tv[16];
#pragma unroll
            for (int u = 0; u < 16; u++) {
                dv[u] = ds[(b + u) * PANEL + lane];
                tv[u] = tq[(b + u) * PANEL + lane];
            }
#pragma unroll
            for (int u = 0; u < 16; u++) f = __builtin_fmaf(dv[u], (float)tv[u], f);
        }
        for (; b + 8 <= NB; b += 8) {
            float dv[8];
            int32_t tv[8];
#pragma unroll
            for (int u = 0; u < 8; u++) {
                dv[u] = ds[(b + u) * PANEL + lane];
                tv[u] = tq[(b + u) * PANEL + lane];
            }
#pragma unroll
            for (int u = 0; u < 8; u++) f = __builtin_fmaf(dv[u], (float)tv[u], f);
        }
        for (; b < NB; b++) f = __builtin_fmaf(ds[b * PANEL + lane], (float)tq[b * PANEL + lane], f);
    }
    return f;
}

// The integer sums of one row (digits in sq, one-row layout) with panel pw (KB k-blocks in LDS): the
// four wavefronts take k-blocks w, w + 4, ...; v_dot4_i32_i8 per 16-input group, the groups meet
// across the wavefront and the wavefronts in sh.kpart. Lanes j < 16 of wavefront 0 read column j's
// sums (hi, lo) after the barrier that ends this call.
__device__ __forceinline__ void row_sums(const uint8_t *pw, int KB, const uint8_t *sq, ResShared &sh) {
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    int dh = 0, dl = 0;
    for (int t = wave; t < KB; t += RES_WAVES) {
        const gemv::v4i ahi = *reinterpret_cast<const gemv::v4i *>(sq + t * 128 + (lane >> 4) * 16);
        const gemv::v4i alo = *reinterpret_cast<const gemv::v4i *>(sq + t * 128 + 64 + (lane >> 4) * 16);
        const gemv::v4i wv = *reinterpret_cast<const gemv::v4i *>(pw + (size_t)t * 1024 + lane * 16);
        dh = __builtin_amdgcn_sdot4(ahi.x, wv.x, dh, false);
        dh = __builtin_amdgcn_sdot4(ahi.y, wv.y, dh, false);
        dh = __builtin_amdgcn_sdot4(ahi.z, wv.z, dh, false);
        dh = __builtin_amdgcn_sdot4(ahi.w, wv.w, dh, false);
        dl = __builtin_amdgcn_sdot4(alo.x, wv.x, dl, false);
        dl = __builtin_amdgcn_sdot4(alo.y, wv.y, dl, false);
        dl = __builtin_amdgcn_sdot4(alo.z, wv.z, dl, false);
        dl = __builtin_amdgcn_sdot4(alo.w, wv.w, dl, false);
    }
    dh = sum_groups(dh);
    dl = sum_groups(dl);
    if (lane < PANEL) {
        sh.kpart[wave][0][lane] = dh;
        sh.kpart[wave][1][lane] = dl;
    }
    __syncthreads();
}

// Q8: every matrix is Q8_0. Its block scales sit in LDS after the digit staging (joint, each LSTM
// layer, projection), then the one-row products' block sums (tq); the joint runs a 16x16x32 MFMA per
// 32-input half and folds each block's sums into f32 in block order, the one-row products fold
// theirs in row_fold_q8.
template <bool Q8>
__global__ __launch_bounds__(RES_THREADS) void tdt_resident_kernel(ResArgs a) {
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    __shared__ ResShared sh;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, b = blockIdx.x;
    const size_t rc = (size_t)(b % RES_COPIES) * a.cs;  // the copy this workgroup reads
    const int h = a.h, NJ = a.joint.n, KBJ = a.joint.KB, KBL = a.lstm[0].KB, KBP = a.proj.KB;
    const int KBJ4 = (KBJ + 3) & ~3;  // the joint's k-blocks padded with zero digits to whole groups of four
    const int bq = b - a.qoff;  // among the joint and LSTM workgroups
    const int pj0 = bq * a.JP, npj = bq >= 0 && bq < a.GJ ? min(a.JP, a.joint.P - pj0) : 0;
    const int pl0 = bq * a.LP, npl = bq >= 0 && bq < a.GL ? min(a.LP, a.lstm[0].P - pl0) : 0;
    const int pp0 = b * a.PP, npp = b < a.GP ? min(a.PP, a.proj.P - pp0) : 0;
    // The joint workgroups holding duration columns: nd of them from jd0 (at most 5 for 64 durations).
    const int jd0 = (a.vocab / PANEL) / a.JP, nd = ((NJ - 1) / PANEL) / a.JP - jd0 + 1;
    uint8_t *wj = lds;
    uint8_t *wl = wj + (size_t)a.JP * KBJ * 1024;
    uint8_t *wp = wl + (size_t)a.layers * a.LP * KBL * 1024;
    uint8_t *sq = wp + (size_t)a.PP * KBP * 1024;
    const int NBJ = a.joint.NB, NBL = a.lstm[0].NB, NBP = a.proj.NB;
    float *qsj = reinterpret_cast<float *>(sq + (size_t)max(KBJ4 * 2048, max(KBL, KBP) * 128));
    float *qsl = qsj + (size_t)a.JP * NBJ * PANEL;
    float *qsp = qsl + (size_t)a.layers * a.LP * NBL * PANEL;
    int32_t *tq = reinterpret_cast<int32_t *>(qsp + (size_t)a.PP * NBP * PANEL);

    copy_panels(wj, a.joint, pj0, npj);
    for (int l = 0; l < a.layers; l++) copy_panels(wl + (size_t)l * a.LP * KBL * 1024, a.lstm[l], pl0, npl);
    copy_panels(wp, a.proj, pp0, npp);
    if constexpr (Q8) {
        copy_q8_scales(qsj, a.joint, pj0, npj);
        for (int l = 0; l < a.layers; l++) copy_q8_scales(qsl + (size_t)l * a.LP * NBL * PANEL, a.lstm[l], pl0, npl);
        copy_q8_scales(qsp, a.proj, pp0, npp);
    }
    if (tid < npj * PANEL) {
        const int c = min(pj0 * PANEL + tid, NJ - 1);
        sh.js[tid] = a.joint.scales[c];
        sh.jbias[tid] = a.joint.bias[c];
    }
    if (tid < npl * PANEL) {
        for (int l = 0; l < a.layers; l++) {
            sh.ls[l][tid] = a.lstm[l].scales[pl0 * PANEL + tid];
            sh.lbias[l][tid] = a.lstm[l].bias[pl0 * PANEL + tid];
        }
    }
    if (tid < npl * 4) {
        const int u = pl0 * 4 + tid;
        for (int l = 0; l < a.layers; l++) {
            sh.hst[l][tid] = a.state[(size_t)l * 2 * h + u];
            sh.cst[l][tid] = a.state[(size_t)l * 2 * h + h + u];
        }
    }
    if (tid < npp * PANEL) {
        const int c = min(pp0 * PANEL + tid, h - 1);
        sh.ps[tid] = a.proj.scales[c];
        sh.pbias[tid] = a.proj.bias[c];
        sh.pst[tid] = a.pred[c];
    }
    if (tid < a.ndur) sh.durs[tid] = a.durations[tid];
    if (tid == 0) sh.abort = 0;
    int t = a.ctl->t, on = a.ctl->on_frame, ntok = a.ctl->ntok, rows = a.ctl->rows, done = a.ctl->done;
    uint32_t s = a.ctl->step, n = a.ctl->preds, pin_n = TAG_NONE;
    const uint32_t s_end = s + (uint32_t)a.steps;
    const int CH = h >> 2;  // 4-input chunks of h inputs
    __syncthreads();

    while (!done && s != s_end) {
        if (t >= a.frames) {
            done = 1;
            break;
        }
        const uint32_t par = s & 1;
        // ---- The joint over rows t .. t + rows - 1: z = relu(enc_proj[min(t + r, frames - 1)] + pred).
        if (npj > 0) {
            // Wavefront w holds rows w + 4 j, lane l chunks l + 64 i (h <= 992: at most 248 chunks).
            // The encoder rows are requested before the wait for the prediction.
            v4f e[4][4];
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const int r = wave + 4 * j, f = min(t + r, a.frames - 1);
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const int c = lane + 64 * i;
                    const bool ok = r < rows && c < CH;
                    e[j][i] = *reinterpret_cast<const v4f *>(ok ? a.enc + (size_t)f * a.lde + 4 * c : gemv::ZERO_CHUNK);
                }
            }
            if (pin_n != n) {
                const uint64_t *p[4];
                uint32_t tag[4];
                uint64_t w[4];
                uint32_t need = 0;
#pragma unroll
                for (int q = 0; q < 4; q++) {
                    const int i = tid + RES_THREADS * q;
                    p[q] = a.w_pred + rc + (size_t)(n & 1) * h + min(i, h - 1);
                    tag[q] = n;
                    if (i < h) need |= 1u << q;
                }
                if (!wait_words<4>(p, need, tag, w, &a.ctl->err, (uint64_t)wall_clock64() + a.wait_ticks)) res_fail(a, sh);
#pragma unroll
                for (int q = 0; q < 4; q++)
                    if (need >> q & 1) sh.pin[tid + RES_THREADS * q] = word_value(w[q]);
                pin_n = n;
                __syncthreads();
                if (sh.abort) break;
            }
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const int r = wave + 4 * j;
                if (r < rows) {
                    v4f z[4];
                    uint32_t mx = 0;
#pragma unroll
                    for (int i = 0; i < 4; i++) {
                        const int c = lane + 64 * i;
                        const v4f pv = c < CH ? *reinterpret_cast<const v4f *>(sh.pin + 4 * c) : v4f{0.0f, 0.0f, 0.0f, 0.0f};
                        z[i].x = fmaxf(e[j][i].x + pv.x, 0.0f);
                        z[i].y = fmaxf(e[j][i].y + pv.y, 0.0f);
                        z[i].z = fmaxf(e[j][i].z + pv.z, 0.0f);
                        z[i].w = fmaxf(e[j][i].w + pv.w, 0.0f);
                        if (c < CH) mx = max(mx, chunk_max(z[i]));
                    }
                    const uint32_t m = gemv::wave_max_u(mx);
                    const int32_t ex = m == 0xffffffffu ? EXP_NONFINITE : row_exponent_of(__uint_as_float(m));
#pragma unroll
                    for (int i = 0; i < 4; i++) {
                        const int c = lane + 64 * i;
                        if (c < KBJ4 * 16) {  // zero digits past the row (z is 0 there)
                            uint32_t hi, lo;
                            digits4(z[i].x, z[i].y, z[i].z, z[i].w, ex, hi, lo);
                            uint8_t *d = sq + (c >> 4) * 2048 + ((c & 15) >> 2) * 256 + r * 16 + (c & 3) * 4;
                            *reinterpret_cast<uint32_t *>(d) = hi;
                            *reinterpret_cast<uint32_t *>(d + 1024) = lo;
                        }
                    }
                    if (lane == 0) sh.erow[r] = ex;
                }
            }
            __syncthreads();
            // Wavefront w scores panels w, w + 4, ... of this workgroup: element v of lane l is row
            // 4 (l / 16) + v, column l % 16. Each row keeps its best vocabulary entry and its best
            // duration entry (index d for column vocab + d). A NaN first logit (column 0) is never
            // beaten in the reference's argmax: it enters as (+inf, 0), which nothing comes before;
            // a NaN first duration logit likewise.
            Key mine[4], dmine[4];
#pragma unroll
            for (int v = 0; v < 4; v++) mine[v] = dmine[v] = Key{0u, 0xffffffffu};
            const int orow = (lane >> 4) * 4, j16 = lane & 15;
            for (int pi = wave; pi < npj; pi += RES_WAVES) {
                gemv::v4i hi = {0, 0, 0, 0}, lo = {0, 0, 0, 0};
                float fq[4] = {0.0f, 0.0f, 0.0f, 0.0f};
                if constexpr (Q8) {
                    // Half hh of k-block t is block 2 t + hh: lane 16 g + x reads 8 bytes of layout
                    // lane 16 (2 hh + g / 2) + x, the same inputs for the digits and the weights. Both
                    // halves' MFMAs are issued before their folds, which run in block order.
                    const uint8_t *wb = wj + (size_t)pi * KBJ * 1024;
                    const float *ds = qsj + (size_t)pi * NBJ * PANEL + j16;
                    const int g = lane >> 4, off0 = (16 * (g >> 1) + j16) * 16 + 8 * (g & 1);
                    for (int t = 0; t < KBJ; t++) {
                        gemv::v4i H[2], L[2];
#pragma unroll
                        for (int hh = 0; hh < 2; hh++) {
                            const int off = off0 + hh * 512;
                            const long ah = *reinterpret_cast<const long *>(sq + t * 2048 + off);
                            const long al = *reinterpret_cast<const long *>(sq + t * 2048 + 1024 + off);
                            const long wv = *reinterpret_cast<const long *>(wb + (size_t)t * 1024 + off);
                            H[hh] = __builtin_amdgcn_mfma_i32_16x16x32_i8(ah, wv, gemv::v4i{0, 0, 0, 0}, 0, 0, 0);
                            L[hh] = __builtin_amdgcn_mfma_i32_16x16x32_i8(al, wv, gemv::v4i{0, 0, 0, 0}, 0, 0, 0);
                        }
#pragma unroll
                        for (int hh = 0; hh < 2; hh++) {
                            const int bk = 2 * t + hh;
                            if (bk < NBJ) {
                                const float d = ds[bk * PANEL];
#pragma unroll
                                for (int v = 0; v < 4; v++) fq[v] = __builtin_fmaf(d, (float)(H[hh][v] * 256 + L[hh][v]), fq[v]);
                            }
                        }
                    }
                } else {
                    const uint8_t *wb = wj + (size_t)pi * KBJ * 1024 + lane * 16;
                    // Four k-blocks' operands are read before their MFMAs, with no branch between: past
                    // KBJ the digits are zero (the weights read are the last block's, adding nothing).
                    for (int t0 = 0; t0 < KBJ4; t0 += 4) {
                        gemv::v4i ah[4], al[4], wv[4];
#pragma unroll
                        for (int u = 0; u < 4; u++) {
                            ah[u] = *reinterpret_cast<const gemv::v4i *>(sq + (t0 + u) * 2048 + lane * 16);
                            al[u] = *reinterpret_cast<const gemv::v4i *>(sq + (t0 + u) * 2048 + 1024 + lane * 16);
                            wv[u] = *reinterpret_cast<const gemv::v4i *>(wb + (size_t)min(t0 + u, KBJ - 1) * 1024);
                        }
#pragma unroll
                        for (int u = 0; u < 4; u++) {
                            hi = __builtin_amdgcn_mfma_i32_16x16x64_i8(ah[u], wv[u], hi, 0, 0, 0);
                            lo = __builtin_amdgcn_mfma_i32_16x16x64_i8(al[u], wv[u], lo, 0, 0, 0);
                        }
                    }
                }
                const int col = (pj0 + pi) * PANEL + j16;
                const float sc = sh.js[pi * PANEL + j16], bs = sh.jbias[pi * PANEL + j16];
                const bool fits = __all((int)dequant_fits(hi[0]) & (int)dequant_fits(hi[1]) &
                                        (int)dequant_fits(hi[2]) & (int)dequant_fits(hi[3]));
#pragma unroll
                for (int v = 0; v < 4; v++) {
                    const int r = orow + v;
                    if (r < rows && col < NJ) {
                        const int32_t er = sh.erow[r];
                        const float dq = Q8 ? (er == EXP_NONFINITE ? __builtin_nanf("") : __builtin_ldexpf(fq[v], -er))
                                            : dequant_w(hi[v], lo[v], er, sc, fits);
                        float val = epilogue_vals(dq, true, bs, ACT_NONE, 1.0f, false, 0.0f);
                        const bool voc = col < a.vocab;
                        const int idx = voc ? col : col - a.vocab;
                        if (idx == 0 && __builtin_isnan(val)) val = __builtin_inff();
                        // A lane meets its columns in increasing order: the strictly larger wins.
                        const uint32_t key = order_key(val);
                        Key &m = voc ? mine[v] : dmine[v];
                        if (key > m.k) m = Key{key, (uint32_t)idx};
                    }
                }
            }
            const bool has_dur = bq >= jd0 && bq < jd0 + nd;  // uniform: only these hold duration columns
#pragma unroll
            for (int v = 0; v < 4; v++) {
                mine[v] = fold16(mine[v]);
                if (has_dur) dmine[v] = fold16(dmine[v]);
                if (j16 == 0) {
                    sh.red[wave][orow + v] = mine[v];
                    sh.dred[wave][orow + v] = dmine[v];
                }
            }
        }
        __syncthreads();
        // Every workgroup's word for every row of the step (none from those without joint panels);
        // the joint workgroups holding duration columns also write their best duration entries.
        if (tid < TDT_ROWS) {
            Key x{0u, 0xffffffffu}, xd{0u, 0xffffffffu};
            if (npj > 0) {
#pragma unroll
                for (int q = 0; q < RES_WAVES; q++) {
                    if (better(sh.red[q][tid], x)) x = sh.red[q][tid];
                    if (better(sh.dred[q][tid], xd)) xd = sh.dred[q][tid];
                }
            }
            word_store(a.w_part + ((size_t)par * TDT_ROWS + tid) * RES_MAX_GRID + b, tagged_key(x, s));
            if (bq >= jd0 && bq < jd0 + nd)
                word_store(a.w_dur + ((size_t)par * TDT_ROWS + tid) * TDT_ROWS + (bq - jd0), tagged_key(xd, s));
        }
        // ---- The decision. Workgroup 0 (a projection workgroup, idle during the joint when the grid
        // has room for both) gathers the words, walks the window, records the token and publishes the
        // outcome in RES_COPIES copies; the others wait for their copy (six words on one line, where
        // every workgroup reading every joint word would queue thousands of line requests).
        if (b == 0) {
            // The window's rows rounded up to a power of two, R, share the threads: g = 256 / R per
            // row, thread j of row r reading the words of workgroups j, j + g, ... and, for j < nd,
            // duration word j; the loads are spread over all four wavefronts.
            const int R = rows <= 1 ? 1 : rows <= 2 ? 2 : rows <= 4 ? 4 : rows <= 8 ? 8 : TDT_ROWS;
            const int g = RES_THREADS / R, r = tid / g, j = tid - r * g;
            const bool live = r < rows;
            const uint64_t *pb = a.w_part + ((size_t)par * TDT_ROWS + r) * RES_MAX_GRID + j;
            const uint64_t *pd = a.w_dur + ((size_t)par * TDT_ROWS + r) * TDT_ROWS + min(j, TDT_ROWS - 1);
            uint64_t pw[16], dw = 0;
            uint32_t pneed = 0;
            bool dneed = live && j < nd;
#pragma unroll
            for (int u = 0; u < 16; u++)
                if (live && j + g * u < a.grid) pneed |= 1u << u;
            const uint64_t deadline = (uint64_t)wall_clock64() + a.wait_ticks;
            for (int round = 0;; round++) {
#pragma unroll
                for (int u = 0; u < 16; u++)
                    if (pneed >> u & 1) pw[u] = word_load(pb + g * u);
                if (dneed) dw = word_load(pd);
#pragma unroll
                for (int u = 0; u < 16; u++)
                    if ((pneed >> u & 1) && (uint32_t)(pw[u] >> 48) == (s & 0xffffu)) pneed &= ~(1u << u);
                if (dneed && (uint32_t)(dw >> 48) == (s & 0xffffu)) dneed = false;
                if (!pneed && !dneed) break;
                if ((round & 15) == 15 && ((uint64_t)wall_clock64() > deadline || load_i(&a.ctl->err) != 0)) {
                    res_fail(a, sh);
                    break;
                }
            }
            // Each group of 16 lanes (inside one row's threads, g >= 16) folds its entries; thread r
            // then takes the best of its row's g / 16 groups, and the duration entry of its first.
            Key x{0u, 0xffffffffu}, xd{0u, 0xffffffffu};
#pragma unroll
            for (int u = 0; u < 16; u++) {
                if (live && j + g * u < a.grid) {
                    const Key y = key_of(pw[u]);
                    if (better(y, x)) x = y;
                }
            }
            if (live && j < nd) xd = key_of(dw);
            x = fold16(x);
            xd = fold16(xd);
            if ((lane & 15) == 0) {
                sh.cand[tid >> 4] = x;
                sh.dcand[tid >> 4] = xd;
            }
            __syncthreads();
            if (tid < rows) {
                const int k0 = tid * (g / 16);
                Key bx = sh.cand[k0];
                for (int k = 1; k < g / 16; k++)
                    if (better(sh.cand[k0 + k], bx)) bx = sh.cand[k0 + k];
                const Key bd = sh.dcand[k0];
                sh.tok_s[tid] = bx.i == 0xffffffffu ? 0 : (int)bx.i;
                sh.dur_s[tid] = sh.durs[bd.i == 0xffffffffu ? 0 : bd.i];
            }
            __syncthreads();
            if (sh.abort) break;
            if (tid == 0) {
                const Walked wk = walk_window(t, rows, on, ntok, sh.tok_s, sh.dur_s, a.blank, a.frames, a.max_symbols,
                                              a.tokens, a.cap, true);
                sh.dec[0] = wk.t;
                sh.dec[1] = wk.on;
                sh.dec[2] = wk.ntok;
                sh.dec[3] = wk.token;
                sh.dec[4] = wk.rows;
                sh.dec[5] = wk.done;
            }
            __syncthreads();
            if (tid < RES_DEC * RES_COPIES)
                word_store(a.w_dec + (size_t)(tid / RES_DEC) * a.cs + par * RES_DEC + tid % RES_DEC,
                           tagged(__int_as_float(sh.dec[tid % RES_DEC]), s));
        } else {
            if (tid < RES_DEC) {
                const uint64_t *p[1] = {a.w_dec + rc + par * RES_DEC + tid};
                const uint32_t tag[1] = {s};
                uint64_t w[1];
                if (!wait_words<1>(p, 1u, tag, w, &a.ctl->err, (uint64_t)wall_clock64() + a.wait_ticks)) res_fail(a, sh);
                sh.dec[tid] = __float_as_int(word_value(w[0]));
            }
            __syncthreads();
            if (sh.abort) break;
        }
        t = sh.dec[0];
        on = sh.dec[1];
        ntok = sh.dec[2];
        const int token = sh.dec[3];
        rows = sh.dec[4];
        done = sh.dec[5];
        s++;
        if (token < 0) continue;

        // ---- The prediction for the token: the LSTM layers (input [x; h_l], x the embedding row or
        // the layer below's new h; tags n + 1 for the new values, n for the old), then the projection.
        const uint32_t nn = n + 1;
        bool stop = false;
        for (int l = 0; l < a.layers && !stop; l++) {
            if (npl == 0) continue;
            const uint8_t *wlay = wl + (size_t)l * a.LP * KBL * 1024;
            const uint64_t *hnew = a.w_h + rc + ((size_t)(l - 1) * 2 + (nn & 1)) * h;  // used for l >= 1
            const uint64_t *hold = a.w_h + rc + ((size_t)l * 2 + (n & 1)) * h;
            v4f x[2];
            const uint64_t *p[8];
            uint32_t tag[8];
            uint64_t w[8];
            uint32_t need = 0;
#pragma unroll
            for (int i = 0; i < 2; i++) {
                const int c = tid + RES_THREADS * i;
                x[i] = v4f{0.0f, 0.0f, 0.0f, 0.0f};
                const bool first = c < CH, second = !first && c < 2 * CH;
                if (first && l == 0) x[i] = *reinterpret_cast<const v4f *>(a.emb + (size_t)token * h + 4 * c);
#pragma unroll
                for (int qq = 0; qq < 4; qq++) {
                    p[4 * i + qq] = first ? hnew + min(4 * c + qq, h - 1) : hold + min(4 * (c - CH) + qq, h - 1);
                    tag[4 * i + qq] = first ? nn : n;
                    if ((first && l > 0) || second) need |= 1u << (4 * i + qq);
                }
            }
            if (!wait_words<8>(p, need, tag, w, &a.ctl->err, (uint64_t)wall_clock64() + a.wait_ticks)) res_fail(a, sh);
#pragma unroll
            for (int i = 0; i < 2; i++)
                if (need >> (4 * i) & 1)
                    x[i] = v4f{word_value(w[4 * i]), word_value(w[4 * i + 1]), word_value(w[4 * i + 2]),
                               word_value(w[4 * i + 3])};
            const int32_t e = row_digits<2>(x, 2 * CH, KBL, sq, sh);
            if (sh.abort) {
                stop = true;
                break;
            }
            for (int pi = 0; pi < npl; pi++) {
                float fq = 0.0f;
                if constexpr (Q8)
                    fq = row_fold_q8(wlay + (size_t)pi * KBL * 1024, KBL, NBL,
                                     qsl + ((size_t)l * a.LP + pi) * NBL * PANEL, sq, tq);
                else
                    row_sums(wlay + (size_t)pi * KBL * 1024, KBL, sq, sh);
                if (wave == 0) {
                    const int j = lane & 15;
                    float dq;
                    if constexpr (Q8) {
                        dq = e == EXP_NONFINITE ? __builtin_nanf("") : __builtin_ldexpf(fq, -e);
                    } else {
                        const int32_t shi =
                            sh.kpart[0][0][j] + sh.kpart[1][0][j] + sh.kpart[2][0][j] + sh.kpart[3][0][j];
                        const int32_t slo =
                            sh.kpart[0][1][j] + sh.kpart[1][1][j] + sh.kpart[2][1][j] + sh.kpart[3][1][j];
                        const bool fits = __all(dequant_fits(shi));
                        dq = dequant_w(shi, slo, e, sh.ls[l][pi * PANEL + j], fits);
                    }
                    const float v = epilogue_vals(dq, true, sh.lbias[l][pi * PANEL + j], ACT_NONE, 1.0f, false, 0.0f);
                    // Output 4 u + q is gate q (i, f, g, o) of unit u: the quad's lane 0 updates the
                    // cell (src/parakeet.rs:1549-1562): c = f c + i g, h = o tanh(c).
                    const float gi = quad_lane<0>(v), gf = quad_lane<1>(v), gg = quad_lane<2>(v), go = quad_lane<3>(v);
                    if (lane < PANEL && (j & 3) == 0) {
                        const int ul = pi * 4 + (j >> 2), u = pl0 * 4 + ul;
                        const float ig = sigmoid(gi), fg = sigmoid(gf), g = tanhf(gg), og = sigmoid(go);
                        const float c = fg * sh.cst[l][ul] + ig * g;
                        const float hn = og * tanhf(c);
                        sh.cst[l][ul] = c;
                        sh.hst[l][ul] = hn;
                        word_store_all(a.w_h + ((size_t)l * 2 + (nn & 1)) * h + u, a.cs, tagged(hn, nn));
                    }
                }
                __syncthreads();
            }
        }
        if (stop) break;
        if (npp > 0) {
            const uint64_t *hl = a.w_h + rc + ((size_t)(a.layers - 1) * 2 + (nn & 1)) * h;
            v4f x[1];
            const uint64_t *p[4];
            uint32_t tag[4];
            uint64_t w[4];
            uint32_t need = 0;
#pragma unroll
            for (int qq = 0; qq < 4; qq++) {
                p[qq] = hl + min(4 * tid + qq, h - 1);
                tag[qq] = nn;
                if (tid < CH) need |= 1u << qq;
            }
            if (!wait_words<4>(p, need, tag, w, &a.ctl->err, (uint64_t)wall_clock64() + a.wait_ticks)) res_fail(a, sh);
            x[0] = tid < CH ? v4f{word_value(w[0]), word_value(w[1]), word_value(w[2]), word_value(w[3])}
                            : v4f{0.0f, 0.0f, 0.0f, 0.0f};
            const int32_t e = row_digits<1>(x, CH, KBP, sq, sh);
            if (sh.abort) break;
            for (int pi = 0; pi < npp; pi++) {
                float fq = 0.0f;
                if constexpr (Q8)
                    fq = row_fold_q8(wp + (size_t)pi * KBP * 1024, KBP, NBP, qsp + (size_t)pi * NBP * PANEL, sq, tq);
                else
                    row_sums(wp + (size_t)pi * KBP * 1024, KBP, sq, sh);
                if (wave == 0 && lane < PANEL) {
                    const int col = (pp0 + pi) * PANEL + lane;
                    float dq;
                    if constexpr (Q8) {
                        dq = e == EXP_NONFINITE ? __builtin_nanf("") : __builtin_ldexpf(fq, -e);
                    } else {
                        const int32_t shi =
                            sh.kpart[0][0][lane] + sh.kpart[1][0][lane] + sh.kpart[2][0][lane] + sh.kpart[3][0][lane];
                        const int32_t slo =
                            sh.kpart[0][1][lane] + sh.kpart[1][1][lane] + sh.kpart[2][1][lane] + sh.kpart[3][1][lane];
                        const bool fits = __all(dequant_fits(shi));  // over the 16 active lanes
                        dq = dequant_w(shi, slo, e, sh.ps[pi * PANEL + lane], fits);
                    }
                    const float v = epilogue_vals(dq, true, sh.pbias[pi * PANEL + lane], ACT_NONE, 1.0f, false, 0.0f);
                    if (col < h) {
                        sh.pst[pi * PANEL + lane] = v;
                        word_store_all(a.w_pred + (size_t)(nn & 1) * h + col, a.cs, tagged(v, nn));
                    }
                }
                __syncthreads();
            }
        }
        n = nn;
    }

    // The state, the prediction and the position for the caller (or the next launch).
    if (tid < npl * 4) {
        const int u = pl0 * 4 + tid;
        for (int l = 0; l < a.layers; l++) {
            a.state[(size_t)l * 2 * h + u] = sh.hst[l][tid];
            a.state[(size_t)l * 2 * h + h + u] = sh.cst[l][tid];
        }
    }
    if (tid < npp * PANEL && pp0 * PANEL + tid < h) a.pred[pp0 * PANEL + tid] = sh.pst[tid];
    if (b == 0 && tid == 0) {
        a.ctl->t = t;
        a.ctl->on_frame = on;
        a.ctl->ntok = ntok;
        a.ctl->rows = rows;
        a.ctl->done = done;
        a.ctl->step = s;
        a.ctl->preds = n;
    }
}

// The hand-over words at the start of a decode: the prediction and each layer's h with tag 0 in
// buffer 0 and no tag in buffer 1; the joint's best-entry words (vocabulary and duration) with the
// low 16 bits of steps -2 and -1, which no step reaches before rewriting them (every step rewrites
// every such word of its buffer).
__global__ void tdt_resident_init_kernel(uint64_t *words, int h, int layers, const float *state, const float *pred) {
    const size_t np = 2 * (size_t)h, nh = (size_t)layers * 2 * h, nb = 2 * (size_t)TDT_ROWS * RES_MAX_GRID,
                 nd = 2 * (size_t)TDT_ROWS * TDT_ROWS, per = np + nh + nb + nd + 2 * RES_DEC;
    for (size_t j = blockIdx.x * (size_t)blockDim.x + threadIdx.x; j < RES_COPIES * per;
         j += (size_t)gridDim.x * blockDim.x) {
        const size_t i = j % per;
        uint64_t v;
        if (i < np) {
            v = i < (size_t)h ? tagged(pred[i], 0) : tagged(0.0f, TAG_NONE);
        } else if (i < np + nh) {
            const size_t k = i - np, l = k / (2 * h), par = (k / h) % 2, u = k % h;
            v = par == 0 ? tagged(state[l * 2 * h + u], 0) : tagged(0.0f, TAG_NONE);
        } else if (i < np + nh + nb) {
            const size_t par = (i - np - nh) / ((size_t)TDT_ROWS * RES_MAX_GRID);
            v = (uint64_t)(par == 0 ? 0xfffeu : 0xffffu) << 48;
        } else if (i < np + nh + nb + nd) {
            const size_t par = (i - np - nh - nb) / ((size_t)TDT_ROWS * TDT_ROWS);
            v = (uint64_t)(par == 0 ? 0xfffeu : 0xffffu) << 48;
        } else {
            v = tagged(0.0f, TAG_NONE);
        }
        words[j] = v;
    }
}


// ------------------------------------------------------------------------ the multi-stream decode
//
// M independent greedy decodes (streams: each its own encoder rows, frames, state, prediction and
// tokens) in one cooperative launch, the matrices held in LDS as in tdt_resident_kernel and the
// same tagged words between workgroups. The streams move in lockstep, one step for all: the joint
// scores the TDT_ROWS row slots, TDT_ROWS / M (the stream's "slots") for each stream's window; the
// decider walks each stream's window on its own and publishes one decision per stream; the streams
// that emitted a token then run the prediction network together, as rows of an MFMA product (row j
// is the j-th emitting stream), so a step costs about what one stream's step costs. Each stream's
// words carry its own prediction count as tag, the step's words the step. int8 matrices.
constexpr int MS_MAX = (int)TDT_MAX_STREAMS;

struct MultiArgs {
    ResMat joint, proj, lstm[TDT_MAX_LAYERS];
    const float *emb;
    const float *enc[MS_MAX];
    size_t lde[MS_MAX];
    int frames[MS_MAX];
    int32_t *tokens[MS_MAX];
    int cap[MS_MAX];
    float *state[MS_MAX], *pred[MS_MAX];
    TdtCtl *ctl;  // ctl[s]: stream s's position; ctl[0].step the steps made, ctl[0].err the error flag
    const int32_t *durations;
    // One copy of the words: predictions [2][M][h], LSTM outputs [layers][2][M][h], the joint's
    // best entries per row slot [2][TDT_ROWS][RES_MAX_GRID] and duration entries
    // [2][TDT_ROWS][TDT_ROWS] (first copy only), decisions [2][M][RES_DEC].
    uint64_t *w_pred, *w_h, *w_part, *w_dur, *w_dec;
    size_t cs;
    int M, slots, h, vocab, ndur, layers, blank, max_symbols;
    int JP, GJ, LP, GL, PP, GP, qoff, grid;
    int steps;
    uint64_t wait_ticks;
};

struct MultiShared {
    float js[RES_MAX_PANELS * PANEL], jbias[RES_MAX_PANELS * PANEL];
    float ps[RES_MAX_PANELS * PANEL], pbias[RES_MAX_PANELS * PANEL];
    float ls[TDT_MAX_LAYERS][RES_MAX_PANELS * PANEL], lbias[TDT_MAX_LAYERS][RES_MAX_PANELS * PANEL];
    Key red[RES_WAVES][TDT_ROWS], dred[RES_WAVES][TDT_ROWS];
    Key cand[RES_THREADS / 16], dcand[RES_THREADS / 16];
    int32_t erow[TDT_ROWS];
    int live[TDT_ROWS];  // row slot holds a frame of a stream's window
    int tok_s[TDT_ROWS], dur_s[TDT_ROWS], durs[TDT_MAX_DURATIONS];
    // The streams' positions (t, on_frame, tokens emitted, window rows, done) and prediction counts.
    int st[MS_MAX][5];
    uint32_t n[MS_MAX], pin_n[MS_MAX];
    int dec[MS_MAX][RES_DEC];
    int emit[MS_MAX], nemit;
    int abort;
};

__device__ __forceinline__ void ms_fail(const MultiArgs &a, MultiShared &sh) {
    sh.abort = 1;
    store_i(&a.ctl[0].err, 1);
}

// Rows j < E of an MFMA product's input from wavefront w = j % 4 (chunk c of 4 inputs in lane c % 64):
// x = [first CA inputs; the rest], each chunk given by ld(j, c), then the row exponent and the digits
// in the 16-row layout (k-block t, digit d at sq + t 2048 + d 1024, lane 16 g + j), zero up to KB
// k-blocks. Returns false when a wait fails.
template <typename LD>
__device__ __forceinline__ bool rows_digits(int E, int CK, int KB, uint8_t *sq, MultiShared &sh, LD ld) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    bool ok = true;
    for (int j = wave; j < E; j += RES_WAVES) {
        v4f x[8];
        uint32_t mx = 0;
#pragma unroll
        for (int q = 0; q < 8; q++) {
            const int c = lane + 64 * q;
            x[q] = v4f{0.0f, 0.0f, 0.0f, 0.0f};
            if (c < CK) {
                ok = ld(j, c, x[q]) && ok;
                mx = max(mx, chunk_max(x[q]));
            }
        }
        const uint32_t m = gemv::wave_max_u(mx);
        const int32_t e = m == 0xffffffffu ? EXP_NONFINITE : row_exponent_of(__uint_as_float(m));
#pragma unroll
        for (int q = 0; q < 8; q++) {
            const int c = lane + 64 * q;
            if (c < KB * 16) {
                uint32_t hi, lo;
                digits4(x[q].x, x[q].y, x[q].z, x[q].w, e, hi, lo);
                uint8_t *d = sq + (c >> 4) * 2048 + ((c & 15) >> 2) * 256 + j * 16 + (c & 3) * 4;
                *reinterpret_cast<uint32_t *>(d) = hi;
                *reinterpret_cast<uint32_t *>(d + 1024) = lo;
            }
        }
        if (lane == 0) sh.erow[j] = e;
    }
    return ok;
}

// The integer sums of the 16 rows in sq with one panel of KB k-blocks in LDS (one wavefront).
__device__ __forceinline__ void rows_sums(const uint8_t *pw, int KB, const uint8_t *sq, gemv::v4i &hi, gemv::v4i &lo) {
    const int lane = threadIdx.x & 63;
    hi = gemv::v4i{0, 0, 0, 0};
    lo = gemv::v4i{0, 0, 0, 0};
    for (int t = 0; t < KB; t++) {
        const gemv::v4i ah = *reinterpret_cast<const gemv::v4i *>(sq + t * 2048 + lane * 16);
        const gemv::v4i al = *reinterpret_cast<const gemv::v4i *>(sq + t * 2048 + 1024 + lane * 16);
        const gemv::v4i wv = *reinterpret_cast<const gemv::v4i *>(pw + (size_t)t * 1024 + lane * 16);
        hi = __builtin_amdgcn_mfma_i32_16x16x64_i8(ah, wv, hi, 0, 0, 0);
        lo = __builtin_amdgcn_mfma_i32_16x16x64_i8(al, wv, lo, 0, 0, 0);
    }
}

// Waits for the four words of chunk c at p (the value of each word its float), tag tg.
__device__ __forceinline__ bool wait_chunk(const uint64_t *p, uint32_t tg, const int32_t *err, uint64_t ticks, v4f &x) {
    const uint64_t *pp[4] = {p, p + 1, p + 2, p + 3};
    const uint32_t tag[4] = {tg, tg, tg, tg};
    uint64_t w[4];
    const bool ok = wait_words<4>(pp, 0xfu, tag, w, err, (uint64_t)wall_clock64() + ticks);
    x = v4f{word_value(w[0]), word_value(w[1]), word_value(w[2]), word_value(w[3])};
    return ok;
}

__global__ __launch_bounds__(RES_THREADS) void tdt_multi_kernel(MultiArgs a) {
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    __shared__ MultiShared sh;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, b = blockIdx.x;
    const size_t rc = (size_t)(b % RES_COPIES) * a.cs;
    const int M = a.M, S = a.slots, h = a.h, NJ = a.joint.n, KBJ = a.joint.KB, KBL = a.lstm[0].KB, KBP = a.proj.KB;
    const int KBJ4 = (KBJ + 3) & ~3;
    const int bq = b - a.qoff;
    const int pj0 = bq * a.JP, npj = bq >= 0 && bq < a.GJ ? min(a.JP, a.joint.P - pj0) : 0;
    const int pl0 = bq * a.LP, npl = bq >= 0 && bq < a.GL ? min(a.LP, a.lstm[0].P - pl0) : 0;
    const int pp0 = b * a.PP, npp = b < a.GP ? min(a.PP, a.proj.P - pp0) : 0;
    const int jd0 = (a.vocab / PANEL) / a.JP, nd = ((NJ - 1) / PANEL) / a.JP - jd0 + 1;
    const int32_t *err = &a.ctl[0].err;
    uint8_t *wj = lds;
    uint8_t *wl = wj + (size_t)a.JP * KBJ * 1024;
    uint8_t *wp = wl + (size_t)a.layers * a.LP * KBL * 1024;
    uint8_t *sq = wp + (size_t)a.PP * KBP * 1024;
    float *pin = reinterpret_cast<float *>(sq + (size_t)max(KBJ4, max(KBL, KBP)) * 2048);  // [M][h]
    float *hst = pin + (size_t)M * h;                                                       // [layers][M][LP 4]
    float *cst = hst + (size_t)a.layers * M * a.LP * 4;
    float *pst = cst + (size_t)a.layers * M * a.LP * 4;  // [M][PP 16]
    const int U = a.LP * 4;

    copy_panels(wj, a.joint, pj0, npj);
    for (int l = 0; l < a.layers; l++) copy_panels(wl + (size_t)l * a.LP * KBL * 1024, a.lstm[l], pl0, npl);
    copy_panels(wp, a.proj, pp0, npp);
    if (tid < npj * PANEL) {
        const int c = min(pj0 * PANEL + tid, NJ - 1);
        sh.js[tid] = a.joint.scales[c];
        sh.jbias[tid] = a.joint.bias[c];
    }
    if (tid < npl * PANEL) {
        for (int l = 0; l < a.layers; l++) {
            sh.ls[l][tid] = a.lstm[l].scales[pl0 * PANEL + tid];
            sh.lbias[l][tid] = a.lstm[l].bias[pl0 * PANEL + tid];
        }
    }
    for (int i = tid; i < a.layers * M * U; i += RES_THREADS) {
        const int l = i / (M * U), s = (i / U) % M, ul = i % U;
        if (ul < npl * 4) {
            hst[i] = a.state[s][(size_t)l * 2 * h + pl0 * 4 + ul];
            cst[i] = a.state[s][(size_t)l * 2 * h + h + pl0 * 4 + ul];
        }
    }
    if (tid < npp * PANEL) {
        const int c = min(pp0 * PANEL + tid, h - 1);
        sh.ps[tid] = a.proj.scales[c];
        sh.pbias[tid] = a.proj.bias[c];
    }
    for (int i = tid; i < M * a.PP * PANEL; i += RES_THREADS) {
        const int s = i / (a.PP * PANEL), ci = i % (a.PP * PANEL);
        if (ci < npp * PANEL) pst[i] = a.pred[s][min(pp0 * PANEL + ci, h - 1)];
    }
    if (tid < a.ndur) sh.durs[tid] = a.durations[tid];
    if (tid < M) {
        const TdtCtl &c = a.ctl[tid];
        sh.st[tid][0] = c.t;
        sh.st[tid][1] = c.on_frame;
        sh.st[tid][2] = c.ntok;
        sh.st[tid][3] = min(c.rows, S);
        sh.st[tid][4] = c.done || c.t >= a.frames[tid];
        sh.n[tid] = c.preds;
        sh.pin_n[tid] = TAG_NONE;
    }
    if (tid == 0) sh.abort = 0;
    uint32_t s = a.ctl[0].step;
    const uint32_t s_end = s + (uint32_t)a.steps;
    const int CH = h >> 2;
    __syncthreads();

    while (s != s_end) {
        bool any = false;
        for (int q = 0; q < M; q++) any = any || !sh.st[q][4];
        if (!any) break;
        const uint32_t par = s & 1;
        if (tid < TDT_ROWS) {
            const int q = tid / S, r = tid % S;
            sh.live[tid] = q < M && !sh.st[q][4] && r < sh.st[q][3];
        }
        // ---- The joint over each stream's window rows.
        if (npj > 0) {
            // The live streams' predictions (waited for only after they change).
            for (int q = 0; q < M; q++) {
                if (sh.st[q][4] || sh.pin_n[q] == sh.n[q]) continue;  // uniform
                const uint32_t nq = sh.n[q];
                for (int i = tid; i < h; i += RES_THREADS) {
                    const uint64_t *p[1] = {a.w_pred + rc + ((size_t)(nq & 1) * M + q) * h + i};
                    const uint32_t tag[1] = {nq};
                    uint64_t w[1];
                    if (!wait_words<1>(p, 1u, tag, w, err, (uint64_t)wall_clock64() + a.wait_ticks)) ms_fail(a, sh);
                    pin[(size_t)q * h + i] = word_value(w[0]);
                }
                __syncthreads();
                if (tid == 0) sh.pin_n[q] = nq;
            }
            __syncthreads();
            if (sh.abort) break;
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const int r = wave + 4 * j;  // the row slot
                if (sh.live[r]) {
                    const int q = r / S, rr = r % S, f = min(sh.st[q][0] + rr, a.frames[q] - 1);
                    const float *er = a.enc[q] + (size_t)f * a.lde[q];
                    const float *pr = pin + (size_t)q * h;
                    v4f z[4];
                    uint32_t mx = 0;
#pragma unroll
                    for (int i = 0; i < 4; i++) {
                        const int c = lane + 64 * i;
                        z[i] = v4f{0.0f, 0.0f, 0.0f, 0.0f};
                        if (c < CH) {
                            const v4f e = *reinterpret_cast<const v4f *>(er + 4 * c);
                            const v4f pv = *reinterpret_cast<const v4f *>(pr + 4 * c);
                            z[i].x = fmaxf(e.x + pv.x, 0.0f);
                            z[i].y = fmaxf(e.y + pv.y, 0.0f);
                            z[i].z = fmaxf(e.z + pv.z, 0.0f);
                            z[i].w = fmaxf(e.w + pv.w, 0.0f);
                            mx = max(mx, chunk_max(z[i]));
                        }
                    }
                    const uint32_t m = gemv::wave_max_u(mx);
                    const int32_t ex = m == 0xffffffffu ? EXP_NONFINITE : row_exponent_of(__uint_as_float(m));
#pragma unroll
                    for (int i = 0; i < 4; i++) {
                        const int c = lane + 64 * i;
                        if (c < KBJ4 * 16) {
                            uint32_t hi, lo;
                            digits4(z[i].x, z[i].y, z[i].z, z[i].w, ex, hi, lo);
                            uint8_t *d = sq + (c >> 4) * 2048 + ((c & 15) >> 2) * 256 + r * 16 + (c & 3) * 4;
                            *reinterpret_cast<uint32_t *>(d) = hi;
                            *reinterpret_cast<uint32_t *>(d + 1024) = lo;
                        }
                    }
                    if (lane == 0) sh.erow[r] = ex;
                }
            }
            __syncthreads();
            Key mine[4], dmine[4];
#pragma unroll
            for (int v = 0; v < 4; v++) mine[v] = dmine[v] = Key{0u, 0xffffffffu};
            const int orow = (lane >> 4) * 4, j16 = lane & 15;
            for (int pi = wave; pi < npj; pi += RES_WAVES) {
                gemv::v4i hi = {0, 0, 0, 0}, lo = {0, 0, 0, 0};
                const uint8_t *wb = wj + (size_t)pi * KBJ * 1024 + lane * 16;
                for (int t0 = 0; t0 < KBJ4; t0 += 4) {
                    gemv::v4i ah[4], al[4], wv[4];
#pragma unroll
                    for (int u = 0; u < 4; u++) {
                        ah[u] = *reinterpret_cast<const gemv::v4i *>(sq + (t0 + u) * 2048 + lane * 16);
                        al[u] = *reinterpret_cast<const gemv::v4i *>(sq + (t0 + u) * 2048 + 1024 + lane * 16);
                        wv[u] = *reinterpret_cast<const gemv::v4i *>(wb + (size_t)min(t0 + u, KBJ - 1) * 1024);
                    }
#pragma unroll
                    for (int u = 0; u < 4; u++) {
                        hi = __builtin_amdgcn_mfma_i32_16x16x64_i8(ah[u], wv[u], hi, 0, 0, 0);
                        lo = __builtin_amdgcn_mfma_i32_16x16x64_i8(al[u], wv[u], lo, 0, 0, 0);
                    }
                }
                const int col = (pj0 + pi) * PANEL + j16;
                const float sc = sh.js[pi * PANEL + j16], bs = sh.jbias[pi * PANEL + j16];
#pragma unroll
                for (int v = 0; v < 4; v++) {
                    const int r = orow + v;
                    if (sh.live[r] && col < NJ) {
                        float val = epilogue_vals(dequant(hi[v], lo[v], sh.erow[r], sc), true, bs, ACT_NONE, 1.0f,
                                                  false, 0.0f);
                        const bool voc = col < a.vocab;
                        const int idx = voc ? col : col - a.vocab;
                        if (idx == 0 && __builtin_isnan(val)) val = __builtin_inff();
                        const uint32_t key = order_key(val);
                        Key &m = voc ? mine[v] : dmine[v];
                        if (key > m.k) m = Key{key, (uint32_t)idx};
                    }
                }
            }
            const bool has_dur = bq >= jd0 && bq < jd0 + nd;
#pragma unroll
            for (int v = 0; v < 4; v++) {
                mine[v] = fold16(mine[v]);
                if (has_dur) dmine[v] = fold16(dmine[v]);
                if (j16 == 0) {
                    sh.red[wave][orow + v] = mine[v];
                    sh.dred[wave][orow + v] = dmine[v];
                }
            }
        }
        __syncthreads();
        if (tid < TDT_ROWS) {
            Key x{0u, 0xffffffffu}, xd{0u, 0xffffffffu};
            if (npj > 0) {
#pragma unroll
                for (int q = 0; q < RES_WAVES; q++) {
                    if (better(sh.red[q][tid], x)) x = sh.red[q][tid];
                    if (better(sh.dred[q][tid], xd)) xd = sh.dred[q][tid];
                }
            }
            word_store(a.w_part + ((size_t)par * TDT_ROWS + tid) * RES_MAX_GRID + b, tagged_key(x, s));
            if (bq >= jd0 && bq < jd0 + nd)
                word_store(a.w_dur + ((size_t)par * TDT_ROWS + tid) * TDT_ROWS + (bq - jd0), tagged_key(xd, s));
        }
        // ---- The decisions: workgroup 0 gathers every slot's words (sixteen threads a slot) and walks
        // each stream's window.
        if (b == 0) {
            const int g = RES_THREADS / TDT_ROWS, r = tid / g, j = tid - r * g;
            const bool live = sh.live[r];
            const uint64_t *pb = a.w_part + ((size_t)par * TDT_ROWS + r) * RES_MAX_GRID + j;
            const uint64_t *pd = a.w_dur + ((size_t)par * TDT_ROWS + r) * TDT_ROWS + min(j, TDT_ROWS - 1);
            uint64_t pw[16], dw = 0;
            uint32_t pneed = 0;
            bool dneed = live && j < nd;
#pragma unroll
            for (int u = 0; u < 16; u++)
                if (live && j + g * u < a.grid) pneed |= 1u << u;
            const uint64_t deadline = (uint64_t)wall_clock64() + a.wait_ticks;
            for (int round = 0;; round++) {
#pragma unroll
                for (int u = 0; u < 16; u++)
                    if (pneed >> u & 1) pw[u] = word_load(pb + g * u);
                if (dneed) dw = word_load(pd);
#pragma unroll
                for (int u = 0; u < 16; u++)
                    if ((pneed >> u & 1) && (uint32_t)(pw[u] >> 48) == (s & 0xffffu)) pneed &= ~(1u << u);
                if (dneed && (uint32_t)(dw >> 48) == (s & 0xffffu)) dneed = false;
                if (!pneed && !dneed) break;
                if ((round & 15) == 15 && ((uint64_t)wall_clock64() > deadline || load_i(err) != 0)) {
                    ms_fail(a, sh);
                    break;
                }
            }
            Key x{0u, 0xffffffffu}, xd{0u, 0xffffffffu};
#pragma unroll
            for (int u = 0; u < 16; u++) {
                if (live && j + g * u < a.grid) {
                    const Key y = key_of(pw[u]);
                    if (better(y, x)) x = y;
                }
            }
            if (live && j < nd) xd = key_of(dw);
            x = fold16(x);
            xd = fold16(xd);
            if ((lane & 15) == 0) {
                sh.cand[tid >> 4] = x;
                sh.dcand[tid >> 4] = xd;
            }
            __syncthreads();
            if (tid < TDT_ROWS) {
                const Key bx = sh.cand[tid], bd = sh.dcand[tid];
                sh.tok_s[tid] = bx.i == 0xffffffffu ? 0 : (int)bx.i;
                sh.dur_s[tid] = sh.durs[bd.i == 0xffffffffu ? 0 : bd.i];
            }
            __syncthreads();
            if (sh.abort) break;
            if (tid < M) {
                int *d = sh.dec[tid];
                if (sh.st[tid][4]) {
                    d[0] = sh.st[tid][0];
                    d[1] = sh.st[tid][1];
                    d[2] = sh.st[tid][2];
                    d[3] = -1;
                    d[4] = sh.st[tid][3];
                    d[5] = 1;
                } else {
                    const Walked wk = walk_window(sh.st[tid][0], sh.st[tid][3], sh.st[tid][1], sh.st[tid][2],
                                                  sh.tok_s + tid * S, sh.dur_s + tid * S, a.blank, a.frames[tid],
                                                  a.max_symbols, a.tokens[tid], a.cap[tid], true);
                    d[0] = wk.t;
                    d[1] = wk.on;
                    d[2] = wk.ntok;
                    d[3] = wk.token;
                    d[4] = min(wk.rows, S);
                    d[5] = wk.done;
                }
            }
            __syncthreads();
            for (int i = tid; i < RES_COPIES * M * RES_DEC; i += RES_THREADS) {
                const int c = i / (M * RES_DEC), k = i % (M * RES_DEC);
                word_store(a.w_dec + (size_t)c * a.cs + (size_t)par * M * RES_DEC + k,
                           tagged(__int_as_float(sh.dec[k / RES_DEC][k % RES_DEC]), s));
            }
        } else {
            if (tid < M * RES_DEC) {
                const uint64_t *p[1] = {a.w_dec + rc + (size_t)par * M * RES_DEC + tid};
                const uint32_t tag[1] = {s};
                uint64_t w[1];
                if (!wait_words<1>(p, 1u, tag, w, err, (uint64_t)wall_clock64() + a.wait_ticks)) ms_fail(a, sh);
                sh.dec[tid / RES_DEC][tid % RES_DEC] = __float_as_int(word_value(w[0]));
            }
            __syncthreads();
            if (sh.abort) break;
        }
        if (tid < M) {
            // A stream ends when its frames are used up, whether a blank or a token's duration took
            // it there (the reference's loop runs while t < frames).
            sh.st[tid][0] = sh.dec[tid][0];
            sh.st[tid][1] = sh.dec[tid][1];
            sh.st[tid][2] = sh.dec[tid][2];
            sh.st[tid][3] = sh.dec[tid][4];
            sh.st[tid][4] = sh.dec[tid][5] || sh.dec[tid][0] >= a.frames[tid];
        }
        if (tid == 0) {
            int e = 0;
            for (int q = 0; q < M; q++)
                if (sh.dec[q][3] >= 0) sh.emit[e++] = q;
            sh.nemit = e;
        }
        __syncthreads();
        s++;
        const int E = sh.nemit;
        if (E == 0) continue;

        // ---- The prediction network for the E emitting streams, row j the j-th of them.
        bool stop = false;
        for (int l = 0; l < a.layers && !stop; l++) {
            if (npl == 0) continue;
            const uint8_t *wlay = wl + (size_t)l * a.LP * KBL * 1024;
            auto ld = [&](int j, int c, v4f &x) -> bool {
                const int q = sh.emit[j];
                const uint32_t nq = sh.n[q];
                if (c < CH) {
                    if (l == 0) {
                        x = *reinterpret_cast<const v4f *>(a.emb + (size_t)sh.dec[q][3] * h + 4 * c);
                        return true;
                    }
                    return wait_chunk(a.w_h + rc + (((size_t)(l - 1) * 2 + ((nq + 1) & 1)) * M + q) * h + 4 * c, nq + 1,
                                      err, a.wait_ticks, x);
                }
                return wait_chunk(a.w_h + rc + (((size_t)l * 2 + (nq & 1)) * M + q) * h + 4 * (c - CH), nq, err,
                                  a.wait_ticks, x);
            };
            if (!rows_digits(E, 2 * CH, KBL, sq, sh, ld)) ms_fail(a, sh);
            __syncthreads();
            if (sh.abort) {
                stop = true;
                break;
            }
            for (int pi = wave; pi < npl; pi += RES_WAVES) {
                gemv::v4i hi, lo;
                rows_sums(wlay + (size_t)pi * KBL * 1024, KBL, sq, hi, lo);
                const int j16 = lane & 15, orow = (lane >> 4) * 4;
                const float sc = sh.ls[l][pi * PANEL + j16], bs = sh.lbias[l][pi * PANEL + j16];
#pragma unroll
                for (int v = 0; v < 4; v++) {
                    const int r = orow + v;
                    const float val = epilogue_vals(dequant(hi[v], lo[v], sh.erow[min(r, E - 1)], sc), true, bs,
                                                    ACT_NONE, 1.0f, false, 0.0f);
                    const float gi = quad_lane<0>(val), gf = quad_lane<1>(val), gg = quad_lane<2>(val),
                                go = quad_lane<3>(val);
                    if (r < E && (j16 & 3) == 0) {
                        const int q = sh.emit[r], ul = pi * 4 + (j16 >> 2), u = pl0 * 4 + ul;
                        const uint32_t nn = sh.n[q] + 1;
                        float *cs_ = cst + ((size_t)l * M + q) * U + ul, *hs_ = hst + ((size_t)l * M + q) * U + ul;
                        const float ig = sigmoid(gi), fg = sigmoid(gf), gt = tanhf(gg), og = sigmoid(go);
                        const float c = fg * *cs_ + ig * gt;
                        const float hn = og * tanhf(c);
                        *cs_ = c;
                        *hs_ = hn;
                        word_store_all(a.w_h + (((size_t)l * 2 + (nn & 1)) * M + q) * h + u, a.cs, tagged(hn, nn));
                    }
                }
            }
            __syncthreads();
        }
        if (stop) break;
        if (npp > 0) {
            auto ld = [&](int j, int c, v4f &x) -> bool {
                const int q = sh.emit[j];
                const uint32_t nn = sh.n[q] + 1;
                return wait_chunk(a.w_h + rc + (((size_t)(a.layers - 1) * 2 + (nn & 1)) * M + q) * h + 4 * c, nn, err,
                                  a.wait_ticks, x);
            };
            if (!rows_digits(E, CH, KBP, sq, sh, ld)) ms_fail(a, sh);
            __syncthreads();
            if (sh.abort) break;
            for (int pi = wave; pi < npp; pi += RES_WAVES) {
                gemv::v4i hi, lo;
                rows_sums(wp + (size_t)pi * KBP * 1024, KBP, sq, hi, lo);
                const int j16 = lane & 15, orow = (lane >> 4) * 4, col = (pp0 + pi) * PANEL + j16;
                const float sc = sh.ps[pi * PANEL + j16], bs = sh.pbias[pi * PANEL + j16];
#pragma unroll
                for (int v = 0; v < 4; v++) {
                    const int r = orow + v;
                    if (r < E && col < h) {
                        const int q = sh.emit[r];
                        const uint32_t nn = sh.n[q] + 1;
                        const float val = epilogue_vals(dequant(hi[v], lo[v], sh.erow[r], sc), true, bs, ACT_NONE,
                                                        1.0f, false, 0.0f);
                        pst[(size_t)q * a.PP * PANEL + pi * PANEL + j16] = val;
                        word_store_all(a.w_pred + ((size_t)(nn & 1) * M + q) * h + col, a.cs, tagged(val, nn));
                    }
                }
            }
            __syncthreads();
        }
        if (tid < E) sh.n[sh.emit[tid]]++;
        __syncthreads();
    }

    // The streams' states, predictions and positions for the caller (or the next launch).
    for (int i = tid; i < a.layers * M * U; i += RES_THREADS) {
        const int l = i / (M * U), q = (i / U) % M, ul = i % U;
        if (ul < npl * 4) {
            a.state[q][(size_t)l * 2 * h + pl0 * 4 + ul] = hst[i];
            a.state[q][(size_t)l * 2 * h + h + pl0 * 4 + ul] = cst[i];
        }
    }
    for (int i = tid; i < M * a.PP * PANEL; i += RES_THREADS) {
        const int q = i / (a.PP * PANEL), ci = i % (a.PP * PANEL);
        if (ci < npp * PANEL && pp0 * PANEL + ci < h) a.pred[q][pp0 * PANEL + ci] = pst[i];
    }
    if (b == 0 && tid < M) {
        TdtCtl &c = a.ctl[tid];
        c.t = sh.st[tid][0];
        c.on_frame = sh.st[tid][1];
        c.ntok = sh.st[tid][2];
        c.rows = sh.st[tid][3];
        c.done = sh.st[tid][4];
        c.preds = sh.n[tid];
        if (tid == 0) c.step = s;
    }
}

// The multi-stream decode's words at its start: each stream's prediction and LSTM outputs with its
// prediction count as tag in buffer count & 1 (none in the other), the joint's words as at the start
// of a single decode, no decisions.
struct MultiInit {
    const float *state[MS_MAX], *pred[MS_MAX];
    uint32_t preds[MS_MAX];
};
__global__ void tdt_multi_init_kernel(uint64_t *words, int h, int layers, int M, MultiInit in) {
    const size_t np = 2 * (size_t)M * h, nh = (size_t)layers * 2 * M * h, nb = 2 * (size_t)TDT_ROWS * RES_MAX_GRID,
                 nd = 2 * (size_t)TDT_ROWS * TDT_ROWS, per = np + nh + nb + nd + 2 * (size_t)M * RES_DEC;
    for (size_t j = blockIdx.x * (size_t)blockDim.x + threadIdx.x; j < RES_COPIES * per;
         j += (size_t)gridDim.x * blockDim.x) {
        const size_t i = j % per;
        uint64_t v;
        if (i < np) {
            const size_t par = i / ((size_t)M * h), q = (i / h) % M, u = i % h;
            v = par == (in.preds[q] & 1) ? tagged(in.pred[q][u], in.preds[q]) : tagged(0.0f, TAG_NONE);
        } else if (i < np + nh) {
            const size_t k = i - np, l = k / (2 * (size_t)M * h), par = (k / ((size_t)M * h)) % 2, q = (k / h) % M,
                         u = k % h;
            v = par == (in.preds[q] & 1) ? tagged(in.state[q][l * 2 * h + u], in.preds[q]) : tagged(0.0f, TAG_NONE);
        } else if (i < np + nh + nb) {
            const size_t par = (i - np - nh) / ((size_t)TDT_ROWS * RES_MAX_GRID);
            v = (uint64_t)(par == 0 ? 0xfffeu : 0xffffu) << 48;
        } else if (i < np + nh + nb + nd) {
            const size_t par = (i - np - nh - nb) / ((size_t)TDT_ROWS * TDT_ROWS);
            v = (uint64_t)(par == 0 ? 0xfffeu : 0xffffu) << 48;
        } else {
            v = tagged(0.0f, TAG_NONE);
        }
        words[j] = v;
    }
}

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

// Words of one copy of the hand-over buffers.
static size_t words_per_copy(const TdtNet &net) {
    return 2 * net.h + net.layers * 2 * net.h + 2 * (size_t)TDT_ROWS * RES_MAX_GRID +
           2 * (size_t)TDT_ROWS * TDT_ROWS + 2 * RES_DEC;
}

size_t tdt_resident_words(const TdtNet &net) { return RES_COPIES * words_per_copy(net); }

bool tdt_resident_plan(const TdtNet &net, TdtPlan &plan) {
    plan = TdtPlan{};
    const uint32_t prec = net.joint->precision;
    if ((prec != INT8 && prec != Q8_0) || net.proj->precision != prec) return false;
    for (size_t l = 0; l < net.layers; l++)
        if (net.lstm[l]->precision != prec) return false;
    const bool q8 = prec == Q8_0;
    if (net.vocab >= 0xffff || net.h > TDT_MAX_H || net.ndur > (size_t)TDT_MAX_DURATIONS) return false;
    int dev = 0, cus = 0, coop = 0, max_lds = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        hipDeviceGetAttribute(&coop, hipDeviceAttributeCooperativeLaunch, dev) != hipSuccess ||
        hipDeviceGetAttribute(&max_lds, hipDeviceAttributeMaxSharedMemoryPerBlock, dev) != hipSuccess)
        return false;
    if (cus < 1 || !coop) return false;
    // Panels spread over at most one workgroup per CU (up to RES_MAX_GRID). The projection's
    // workgroups come first and hold nothing else when the grid has room (their joint would start
    // late, after the projection); the joint and the LSTM share the rest.
    const size_t G = (size_t)std::min(cus, RES_MAX_GRID);
    const size_t PJ = net.joint->panels, PL = net.lstm[0]->panels, PP = net.proj->panels;
    TdtPlan p;
    p.JP = (int)div_ceil(PJ, G);
    p.GJ = (int)div_ceil(PJ, (size_t)p.JP);
    p.LP = (int)div_ceil(PL, G);
    p.GL = (int)div_ceil(PL, (size_t)p.LP);
    p.PP = (int)div_ceil(PP, G);
    p.GP = (int)div_ceil(PP, (size_t)p.PP);
    p.qoff = (size_t)(p.GP + std::max(p.GJ, p.GL)) <= G ? p.GP : 0;
    p.grid = std::max(p.GP, p.qoff + std::max(p.GJ, p.GL));
    if (p.JP > RES_MAX_PANELS || p.LP > RES_MAX_PANELS || p.PP > RES_MAX_PANELS) return false;
    // The joint workgroups holding duration columns write one word each per row: at most TDT_ROWS.
    const size_t nd = (((net.vocab + net.ndur - 1) / PANEL) / p.JP) - ((net.vocab / PANEL) / p.JP) + 1;
    if (nd > (size_t)TDT_ROWS) return false;
    const size_t KBJ = net.joint->kb, KBL = net.lstm[0]->kb, KBP = net.proj->kb;
    p.lds = ((size_t)p.JP * KBJ + net.layers * p.LP * KBL + (size_t)p.PP * KBP) * 1024 +
            std::max(((KBJ + 3) & ~(size_t)3) * 2048, std::max(KBL, KBP) * 128);
    p.q8 = q8;
    if (q8) {
        // The block scales of the workgroup's panels, then a one-row product's block sums.
        const size_t NBJ = net.joint->k / Q8_BLOCK, NBL = net.lstm[0]->k / Q8_BLOCK, NBP = net.proj->k / Q8_BLOCK;
        p.lds += ((size_t)p.JP * NBJ + net.layers * p.LP * NBL + (size_t)p.PP * NBP) * PANEL * sizeof(float) +
                 2 * std::max(KBL, KBP) * PANEL * sizeof(int32_t);
    }
    const void *f = q8 ? reinterpret_cast<const void *>(&tdt_resident_kernel<true>)
                       : reinterpret_cast<const void *>(&tdt_resident_kernel<false>);
    hipFuncAttributes fa;
    if (hipFuncGetAttributes(&fa, f) != hipSuccess || p.lds + fa.sharedSizeBytes > (size_t)max_lds) return false;
    if (hipFuncSetAttribute(f, hipFuncAttributeMaxDynamicSharedMemorySize, (int)p.lds) != hipSuccess) return false;
    int per_cu = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, f, RES_THREADS, p.lds) != hipSuccess || per_cu < 1 ||
        (size_t)p.grid > (size_t)per_cu * cus)
        return false;
    plan = p;
    return true;
}

hipError_t launch_tdt_resident_init(const TdtNet &net, uint64_t *words, const float *state, const float *pred,
                                    hipStream_t s) {
    hipLaunchKernelGGL(tdt_resident_init_kernel, dim3(256), dim3(256), 0, s, words, (int)net.h, (int)net.layers, state,
                       pred);
    return hipGetLastError();
}

hipError_t launch_tdt_resident(TdtCtl *ctl, const TdtNet &net, const TdtPlan &plan, uint64_t *words,
                               const float *enc, size_t lde, int frames, float *state, float *pred, int32_t *tokens,
                               int cap, int steps, uint64_t wait_ticks, hipStream_t s) {
    auto mat = [](const DeviceWeights &d, const float *bias) {
        return ResMat{d.values, d.scales, bias, d.panel_stride, d.blk_stride, (int)d.n, (int)d.kb, (int)d.panels,
                      (int)(d.k / Q8_BLOCK)};
    };
    ResArgs a{};
    a.joint = mat(*net.joint, net.joint_b);
    a.proj = mat(*net.proj, net.proj_b);
    for (size_t l = 0; l < net.layers; l++) a.lstm[l] = mat(*net.lstm[l], net.lstm_b[l]);
    a.emb = net.emb;
    a.enc = enc;
    a.lde = lde;
    a.durations = net.durations;
    a.tokens = tokens;
    a.ctl = ctl;
    a.state = state;
    a.pred = pred;
    a.w_pred = words;
    a.w_h = a.w_pred + 2 * net.h;
    a.w_part = a.w_h + net.layers * 2 * net.h;
    a.w_dur = a.w_part + 2 * (size_t)TDT_ROWS * RES_MAX_GRID;
    a.w_dec = a.w_dur + 2 * (size_t)TDT_ROWS * TDT_ROWS;
    a.cs = words_per_copy(net);
    a.h = (int)net.h;
    a.vocab = (int)net.vocab;
    a.ndur = (int)net.ndur;
    a.layers = (int)net.layers;
    a.blank = (int)net.blank;
    a.max_symbols = (int)net.max_symbols;
    a.frames = frames;
    a.cap = cap;
    a.JP = plan.JP;
    a.GJ = plan.GJ;
    a.LP = plan.LP;
    a.GL = plan.GL;
    a.PP = plan.PP;
    a.GP = plan.GP;
    a.qoff = plan.qoff;
    a.grid = plan.grid;
    a.steps = steps;
    a.wait_ticks = wait_ticks;
    void *args[] = {&a};
    const void *f = plan.q8 ? reinterpret_cast<const void *>(&tdt_resident_kernel<true>)
                            : reinterpret_cast<const void *>(&tdt_resident_kernel<false>);
    return hipLaunchCooperativeKernel(f, dim3((unsigned)plan.grid), dim3(RES_THREADS), args, (unsigned)plan.lds, s);
}

// Words of one copy of the multi-stream decode's hand-over buffers for m streams.
static size_t multi_words_per_copy(const TdtNet &net, size_t m) {
    return 2 * m * net.h + net.layers * 2 * m * net.h + 2 * (size_t)TDT_ROWS * RES_MAX_GRID +
           2 * (size_t)TDT_ROWS * TDT_ROWS + 2 * m * RES_DEC;
}

size_t tdt_multi_words(const TdtNet &net) { return RES_COPIES * multi_words_per_copy(net, TDT_MAX_STREAMS); }

// The multi-stream decode's dynamic LDS: the panels, the 16-row digits of the largest product, the
// streams' predictions for the joint, their cell states and the projection panels' predictions.
static size_t multi_lds(const TdtNet &net, const TdtPlan &p) {
    const size_t KBJ = net.joint->kb, KBL = net.lstm[0]->kb, KBP = net.proj->kb;
    const size_t M = TDT_MAX_STREAMS;
    return ((size_t)p.JP * KBJ + net.layers * p.LP * KBL + (size_t)p.PP * KBP) * 1024 +
           std::max(((KBJ + 3) & ~(size_t)3), std::max(KBL, KBP)) * 2048 +
           (M * net.h + 2 * net.layers * M * p.LP * 4 + M * p.PP * PANEL) * sizeof(float);
}

bool tdt_multi_plan(const TdtNet &net, TdtPlan &plan) {
    plan.multi = false;
    if (plan.grid == 0 || plan.q8) return false;
    int dev = 0, cus = 0, max_lds = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        hipDeviceGetAttribute(&max_lds, hipDeviceAttributeMaxSharedMemoryPerBlock, dev) != hipSuccess)
        return false;
    const size_t lds = multi_lds(net, plan);
    const void *f = reinterpret_cast<const void *>(&tdt_multi_kernel);
    hipFuncAttributes fa;
    if (hipFuncGetAttributes(&fa, f) != hipSuccess || lds + fa.sharedSizeBytes > (size_t)max_lds) return false;
    if (hipFuncSetAttribute(f, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds) != hipSuccess) return false;
    int per_cu = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, f, RES_THREADS, lds) != hipSuccess || per_cu < 1 ||
        (size_t)plan.grid > (size_t)per_cu * cus)
        return false;
    plan.mlds = lds;
    plan.multi = true;
    return true;
}

hipError_t launch_tdt_multi_init(const TdtNet &net, uint64_t *words, size_t m, const TdtStream *streams,
                                 const uint32_t *preds, hipStream_t s) {
    MultiInit in{};
    for (size_t q = 0; q < m; q++) {
        in.state[q] = streams[q].state;
        in.pred[q] = streams[q].pred;
        in.preds[q] = preds[q];
    }
    hipLaunchKernelGGL(tdt_multi_init_kernel, dim3(256), dim3(256), 0, s, words, (int)net.h, (int)net.layers, (int)m,
                       in);
    return hipGetLastError();
}

hipError_t launch_tdt_multi(TdtCtl *ctl, const TdtNet &net, const TdtPlan &plan, uint64_t *words, size_t m,
                            const TdtStream *streams, int steps, uint64_t wait_ticks, hipStream_t s) {
    auto mat = [](const DeviceWeights &d, const float *bias) {
        return ResMat{d.values, d.scales, bias, d.panel_stride, d.blk_stride, (int)d.n, (int)d.kb, (int)d.panels,
                      (int)(d.k / Q8_BLOCK)};
    };
    MultiArgs a{};
    a.joint = mat(*net.joint, net.joint_b);
    a.proj = mat(*net.proj, net.proj_b);
    for (size_t l = 0; l < net.layers; l++) a.lstm[l] = mat(*net.lstm[l], net.lstm_b[l]);
    a.emb = net.emb;
    for (size_t q = 0; q < m; q++) {
        a.enc[q] = streams[q].enc;
        a.lde[q] = streams[q].lde;
        a.frames[q] = streams[q].frames;
        a.tokens[q] = streams[q].tokens;
        a.cap[q] = streams[q].cap;
        a.state[q] = streams[q].state;
        a.pred[q] = streams[q].pred;
    }
    a.ctl = ctl;
    a.durations = net.durations;
    a.cs = multi_words_per_copy(net, m);
    a.w_pred = words;
    a.w_h = a.w_pred + 2 * m * net.h;
    a.w_part = a.w_h + net.layers * 2 * m * net.h;
    a.w_dur = a.w_part + 2 * (size_t)TDT_ROWS * RES_MAX_GRID;
    a.w_dec = a.w_dur + 2 * (size_t)TDT_ROWS * TDT_ROWS;
    a.M = (int)m;
    int slots = TDT_ROWS;
    while (slots * (int)m > TDT_ROWS) slots >>= 1;  // TDT_ROWS / m rounded down to a power of two
    a.slots = slots;
    a.h = (int)net.h;
    a.vocab = (int)net.vocab;
    a.ndur = (int)net.ndur;
    a.layers = (int)net.layers;
    a.blank = (int)net.blank;
    a.max_symbols = (int)net.max_symbols;
    a.JP = plan.JP;
    a.GJ = plan.GJ;
    a.LP = plan.LP;
    a.GL = plan.GL;
    a.PP = plan.PP;
    a.GP = plan.GP;
    a.qoff = plan.qoff;
    a.grid = plan.grid;
    a.steps = steps;
    a.wait_ticks = wait_ticks;
    void *args[] = {&a};
    return hipLaunchCooperativeKernel(reinterpret_cast<const void *>(&tdt_multi_kernel), dim3((unsigned)plan.grid),
                                      dim3(RES_THREADS), args, (unsigned)plan.mlds, s);
}

}  // namespace tg
