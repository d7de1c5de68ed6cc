// The greedy TDT decode of Parakeet (src/parakeet.rs:1412-1577) with every step on the device: the
// joint, both argmaxes, the blank / duration bookkeeping, the prediction network's LSTM layers and
// its projection run as one chain of kernels per step, with no host round trip per token.
//
// Each kernel is the MFMA GEMV of gemv_core.hpp with its own input rows and outputs, followed by a
// finisher: the last workgroup to arrive (an atomic count, nothing waits) does the step's serial
// part (argmax, cell update, bookkeeping). A kernel whose step has nothing to do returns at once.
//
// * tdt_joint_kernel scores TDT_ROWS consecutive frames t, t + 1, ... against the same prediction
//   in one GEMV (z = relu(enc_proj[f] + pred), the joint's bias): a row's logits do not depend on
//   the other rows, so this equals TDT_ROWS separate joints while the prediction is unchanged. The
//   finisher then walks the frames as the reference's loop does (blank: skip max(duration, 1)
//   frames; a token: record it, hand it to the prediction network, move by its duration) until a
//   token is emitted, the window is used up or the frames end.
// * tdt_lstm_kernel runs layer l: gates = W_l [x; h_l] + b_l (x the token's embedding for l = 0,
//   the new h_{l-1} otherwise); its finisher applies the cell update to every row.
// * tdt_proj_kernel writes pred = W_p h_last + b_p and closes the step.
#include "gemv_core.hpp"

namespace tg {

namespace {

using gemv::v4f;

constexpr int TDT_WAVES = 4;
constexpr int TDT_THREADS = TDT_WAVES * 64;

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

// True in every thread of the last workgroup of the grid to get here. Each wavefront's stores are
// released before the count, and the last workgroup acquires everything the others released. The
// count is reset for the next launch.
__device__ __forceinline__ bool last_to_arrive(uint32_t *count, int *flag) {
    __threadfence();
    __syncthreads();
    if (threadIdx.x == 0) {
        const uint32_t prev = __hip_atomic_fetch_add(count, 1u, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT);
        const bool last = prev == gridDim.x - 1;
        if (last) __hip_atomic_store(count, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        *flag = last;
    }
    __syncthreads();
    const bool last = *flag != 0;
    if (last) __threadfence();
    return last;
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

// Joint outputs: the logits, and per lane the best vocabulary entry of its four rows so far.
struct JointOut {
    float *logits;
    int outputs, vocab;
    float bv[4];
    int bi[4];
    __device__ __forceinline__ void store(int r, int col, float v) {
        logits[(size_t)r * outputs + col] = v;
        if (col < vocab && before(v, col, bv[r & 3], bi[r & 3])) {
            bv[r & 3] = v;
            bi[r & 3] = col;
        }
    }
};

// LSTM layer l input row r: [x; h_l] with x = embedding[tok[r]] (l = 0) or the new h_{l-1}. The
// tokens sit in LDS (a register array indexed by row would live in scratch memory).
struct LstmIn {
    const float *emb;
    const float *states;
    size_t width;
    int h, l;
    const int *tok;
    __device__ __forceinline__ v4f load(int r, int i0, int m, int k) const {
        const bool ok = r < m && i0 < k;
        const int rr = ok ? r : 0;
        const float *row = states + (size_t)rr * width;
        const float *src = i0 < h ? (l == 0 ? emb + (size_t)tok[rr] * h + i0 : row + (size_t)(l - 1) * 2 * h + i0)
                                  : row + (size_t)l * 2 * h + (i0 - h);
        return *reinterpret_cast<const v4f *>(ok ? src : gemv::ZERO_CHUNK);
    }
};

struct Weights {
    const uint8_t *values;
    const float *scales;
    int n, k, P, KB, NB;
    size_t panel_stride, blk_stride;
};

__device__ __forceinline__ float sigmoid(float x) { return 1.0f / (1.0f + expf(0.0f - x)); }

template <int KBC, int J, int Q8>
__global__ __launch_bounds__(TDT_THREADS) void tdt_joint_kernel(TdtCtl *ctl, const float *__restrict__ enc, size_t lde,
                                                                const float *__restrict__ pred, int frames, Weights w,
                                                                const float *__restrict__ bias, float *logits,
                                                                int vocab, int blank, const int32_t *durations,
                                                                int ndur, int max_symbols, Best *partials,
                                                                int32_t *tokens, int cap) {
    extern __shared__ __attribute__((aligned(16))) uint8_t sqa[];
    __shared__ uint32_t slot[TDT_WAVES * J];
    __shared__ Best red[TDT_WAVES][TDT_ROWS];
    __shared__ int tok_s[TDT_ROWS], dur_s[TDT_ROWS], flag;
    if (load_i(&ctl->done) || load_i(&ctl->active)) return;
    const int t = load_i(&ctl->t);
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;

    JointOut out{logits, w.n, vocab, {}, {}};
#pragma unroll
    for (int v = 0; v < 4; v++) {
        out.bv[v] = __builtin_nanf("");
        out.bi[v] = INT32_MAX;
    }
    gemv::mfma_body<TDT_WAVES, KBC, J, Q8>(JointIn{enc, lde, pred, t, frames}, out, TDT_ROWS, w.k, w.values, w.scales,
                                           w.n, w.P, w.KB, w.NB, logits, (size_t)w.n, bias, ACT_NONE, 1.0f, 0,
                                           w.panel_stride, w.blk_stride, sqa, slot);
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
    if (!last_to_arrive(&ctl->arrive[0], &flag)) return;

    // Finisher. Row r's best over all workgroups: thread (r, s) takes workgroups s, s + 16, ...
    {
        const int r = tid >> 4, s = tid & 15;
        float bv = __builtin_nanf("");
        int bi = INT32_MAX;
        for (int b = s; b < (int)gridDim.x; b += 16) {
            const Best x = partials[(size_t)b * TDT_ROWS + r];
            if (before(x.v, x.i, bv, bi)) {
                bv = x.v;
                bi = x.i;
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
        if (s == 0) {
            const float *row = logits + (size_t)r * w.n;
            // a NaN first entry is never beaten in the reference's scan
            tok_s[r] = __builtin_isnan(row[0]) || bi == INT32_MAX ? 0 : bi;
            int d = 0;
            for (int i = 1; i < ndur; i++)
                if (row[vocab + i] > row[vocab + d]) d = i;
            dur_s[r] = durations[d];
        }
    }
    __syncthreads();
    if (tid == 0) {
        int tc = t, on = load_i(&ctl->on_frame), ntok = load_i(&ctl->ntok), active = 0, done = 0;
        while (true) {
            const int r = tc - t;
            if (r >= TDT_ROWS) break;  // the next window scores the frames from tc
            const int token = tok_s[r], dur = dur_s[r];
            if (token == blank) {
                tc += max(dur, 1);
                on = 0;
                if (tc >= frames) {
                    done = 1;
                    break;
                }
                continue;
            }
            if (ntok < cap) {
                tokens[3 * ntok] = token;
                tokens[3 * ntok + 1] = tc;
                tokens[3 * ntok + 2] = dur;
            }
            ntok++;
            store_i(&ctl->tok[0], token);
            active = 1;
            if (dur > 0) {
                tc += dur;
                on = 0;
            } else if (++on >= max_symbols) {
                tc += 1;
                on = 0;
            }
            break;
        }
        store_i(&ctl->t, tc);
        store_i(&ctl->on_frame, on);
        store_i(&ctl->ntok, ntok);
        store_i(&ctl->active, active);
        store_i(&ctl->done, done);
    }
}

// The cell update of row r, unit j (src/parakeet.rs:1549-1562): i, f, o = sigmoid, g = tanh of the
// gates, c = f c + i g, h = o tanh(c), each product rounded before the sum.
__device__ __forceinline__ void cell_update(const float *gates, float *state, int h, int j) {
    const float i = sigmoid(gates[j]), f = sigmoid(gates[h + j]), g = tanhf(gates[2 * h + j]),
                o = sigmoid(gates[3 * h + j]);
    const float c = f * state[h + j] + i * g;
    state[h + j] = c;
    state[j] = o * tanhf(c);
}

template <int KBC, int J, int Q8>
__global__ __launch_bounds__(TDT_THREADS) void tdt_lstm_kernel(TdtCtl *ctl, int gated, TdtTokens toks, int m, int l,
                                                               const float *__restrict__ emb, float *states,
                                                               size_t width, Weights w,
                                                               const float *__restrict__ bias, float *gates) {
    extern __shared__ __attribute__((aligned(16))) uint8_t sqa[];
    __shared__ uint32_t slot[TDT_WAVES * J];
    __shared__ int tok_s[TDT_ROWS], flag;
    if (gated && !load_i(&ctl->active)) return;
    const int h = w.k / 2;
    if (threadIdx.x < TDT_ROWS) tok_s[threadIdx.x] = gated ? load_i(&ctl->tok[threadIdx.x]) : toks.tok[threadIdx.x];
    __syncthreads();
    LstmIn in{emb, states, width, h, l, tok_s};
    gemv::StoreC out{gates, (size_t)w.n};
    gemv::mfma_body<TDT_WAVES, KBC, J, Q8>(in, out, m, w.k, w.values, w.scales, w.n, w.P, w.KB, w.NB, gates,
                                           (size_t)w.n, bias, ACT_NONE, 1.0f, 0, w.panel_stride, w.blk_stride, sqa,
                                           slot);
    if (!last_to_arrive(&ctl->arrive[1 + l], &flag)) return;
    for (int x = threadIdx.x; x < m * h; x += TDT_THREADS) {
        const int r = x / h, j = x - r * h;
        cell_update(gates + (size_t)r * w.n, states + (size_t)r * width + (size_t)l * 2 * h, h, j);
    }
}

template <int KBC, int J, int Q8>
__global__ __launch_bounds__(TDT_THREADS) void tdt_proj_kernel(TdtCtl *ctl, int gated, int m, const float *states,
                                                               size_t width, int layers, Weights w,
                                                               const float *__restrict__ bias, float *preds,
                                                               int frames) {
    extern __shared__ __attribute__((aligned(16))) uint8_t sqa[];
    __shared__ uint32_t slot[TDT_WAVES * J];
    __shared__ int flag;
    if (gated && !load_i(&ctl->active)) return;
    const int h = w.k;
    gemv::StoreC out{preds, (size_t)h};
    gemv::mfma_body<TDT_WAVES, KBC, J, Q8>(gemv::RowsIn{states + (size_t)(layers - 1) * 2 * h, width}, out, m, w.k,
                                           w.values, w.scales, w.n, w.P, w.KB, w.NB, preds, (size_t)h, bias, ACT_NONE,
                                           1.0f, 0, w.panel_stride, w.blk_stride, sqa, slot);
    if (!gated) return;
    if (!last_to_arrive(&ctl->arrive[TDT_MAX_LAYERS + 1], &flag)) return;
    if (threadIdx.x == 0) {
        store_i(&ctl->active, 0);
        if (load_i(&ctl->t) >= frames) store_i(&ctl->done, 1);
    }
}

Weights weights_of(const DeviceWeights &d) {
    return Weights{d.values, d.scales, (int)d.n, (int)d.k, (int)d.panels, (int)d.kb, (int)(d.k / Q8_BLOCK),
                   d.panel_stride, d.blk_stride};
}

// Persistent grid as the plain MFMA GEMV sizes it: at most 1024 workgroups walking the panels.
unsigned grid_of(const DeviceWeights &d) {
    const size_t per_wave = div_ceil(d.panels, (size_t)TDT_WAVES * 1024);
    return (unsigned)div_ceil(d.panels, (size_t)TDT_WAVES * per_wave);
}

// Chunk registers per thread for m rows of k inputs: m * ceil(kb / 4) chunk wavefronts over 4.
int j_of(size_t m, const DeviceWeights &d) {
    const size_t j = div_ceil(m * div_ceil(d.kb, (size_t)4), (size_t)TDT_WAVES);
    return j <= 2 ? 2 : j <= 4 ? 4 : j <= 8 ? 8 : j <= 12 ? 12 : j <= 16 ? 16 : 20;
}

#define TG_TDT_DISPATCH(KERNEL, J_, D, ...)                                                                        \
    do {                                                                                                           \
        const bool q8_ = (D).precision == Q8_0;                                                                    \
        const size_t lds_ = (D).kb * 2048;                                                                         \
        const dim3 g_(grid_of(D)), b_(TDT_THREADS);                                                                \
        if ((D).kb <= 10) {                                                                                        \
            switch (J_) {                                                                                          \
            case 2: hipLaunchKernelGGL(q8_ ? (KERNEL<10, 2, 1>) : (KERNEL<10, 2, 0>), g_, b_, lds_, s, __VA_ARGS__); break;     \
            case 4: hipLaunchKernelGGL(q8_ ? (KERNEL<10, 4, 1>) : (KERNEL<10, 4, 0>), g_, b_, lds_, s, __VA_ARGS__); break;     \
            case 8: hipLaunchKernelGGL(q8_ ? (KERNEL<10, 8, 1>) : (KERNEL<10, 8, 0>), g_, b_, lds_, s, __VA_ARGS__); break;     \
            case 12: hipLaunchKernelGGL(q8_ ? (KERNEL<10, 12, 1>) : (KERNEL<10, 12, 0>), g_, b_, lds_, s, __VA_ARGS__); break;  \
            case 16: hipLaunchKernelGGL(q8_ ? (KERNEL<10, 16, 1>) : (KERNEL<10, 16, 0>), g_, b_, lds_, s, __VA_ARGS__); break;  \
            default: hipLaunchKernelGGL(q8_ ? (KERNEL<10, 20, 1>) : (KERNEL<10, 20, 0>), g_, b_, lds_, s, __VA_ARGS__); break; \
            }                                                                                                      \
        } else {                                                                                                   \
            switch (J_) {                                                                                          \
            case 2: hipLaunchKernelGGL(q8_ ? (KERNEL<16, 2, 1>) : (KERNEL<16, 2, 0>), g_, b_, lds_, s, __VA_ARGS__); break;     \
            case 4: hipLaunchKernelGGL(q8_ ? (KERNEL<16, 4, 1>) : (KERNEL<16, 4, 0>), g_, b_, lds_, s, __VA_ARGS__); break;     \
            case 8: hipLaunchKernelGGL(q8_ ? (KERNEL<16, 8, 1>) : (KERNEL<16, 8, 0>), g_, b_, lds_, s, __VA_ARGS__); break;     \
            case 12: hipLaunchKernelGGL(q8_ ? (KERNEL<16, 12, 1>) : (KERNEL<16, 12, 0>), g_, b_, lds_, s, __VA_ARGS__); break;  \
            case 16: hipLaunchKernelGGL(q8_ ? (KERNEL<16, 16, 1>) : (KERNEL<16, 16, 0>), g_, b_, lds_, s, __VA_ARGS__); break;  \
            default: hipLaunchKernelGGL(q8_ ? (KERNEL<16, 20, 1>) : (KERNEL<16, 20, 0>), g_, b_, lds_, s, __VA_ARGS__); break; \
            }                                                                                                      \
        }                                                                                                          \
    } while (0)

}  // namespace

size_t tdt_max_rows(const DeviceWeights &lstm) {
    const size_t spr = div_ceil(lstm.kb, (size_t)4);
    const size_t rows = (size_t)TDT_WAVES * 20 / spr;
    return rows < (size_t)TDT_ROWS ? rows : (size_t)TDT_ROWS;
}

size_t tdt_partials_bytes() { return (size_t)1024 * TDT_ROWS * sizeof(Best); }

hipError_t launch_tdt_predict(TdtCtl *ctl, int gated, const TdtTokens &toks, size_t m, const TdtNet &net,
                              float *states, float *preds, float *gates, int frames, hipStream_t s) {
    const size_t width = net.layers * 2 * net.h;
    for (size_t l = 0; l < net.layers; l++) {
        const DeviceWeights &d = *net.lstm[l];
        TG_TDT_DISPATCH(tdt_lstm_kernel, j_of(m, d), d, ctl, gated, toks, (int)m, (int)l, net.emb, states, width,
                        weights_of(d), net.lstm_b[l], gates);
    }
    const DeviceWeights &p = *net.proj;
    TG_TDT_DISPATCH(tdt_proj_kernel, j_of(m, p), p, ctl, gated, (int)m, states, width, (int)net.layers, weights_of(p),
                    net.proj_b, preds, frames);
    return hipGetLastError();
}

hipError_t launch_tdt_step(TdtCtl *ctl, const TdtNet &net, const float *enc, size_t lde, int frames, float *states,
                           float *pred, float *logits, float *gates, void *partials, int32_t *tokens, int cap,
                           hipStream_t s) {
    const DeviceWeights &d = *net.joint;
    TG_TDT_DISPATCH(tdt_joint_kernel, j_of(TDT_ROWS, d), d, ctl, enc, lde, pred, frames, weights_of(d), net.joint_b,
                    logits, (int)net.vocab, (int)net.blank, net.durations, (int)net.ndur, (int)net.max_symbols,
                    static_cast<Best *>(partials), tokens, cap);
    return launch_tdt_predict(ctl, 1, TdtTokens{}, 1, net, states, pred, gates, frames, s);
}

}  // namespace tg
