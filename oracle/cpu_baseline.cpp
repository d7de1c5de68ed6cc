// CPU baseline: a C++ port of telmo's SIMD + thread-pool matrix product, timed beside the GPU.
// TEST AND BENCHMARK INFRASTRUCTURE ONLY (the bench's cpu_baseline leg and tests/); the product
// never loads it. It must agree bit for bit with the fused oracle (oracle.c, fused = 1).
//
// What it follows (paths relative to the reference repository):
//   tile_rows<R>          src/kernels/avx512.rs:70-105 (8 x 16 register tile), avx2.rs:62-107 (6 x 16)
//   tile_narrow_rows      src/kernels/avx512.rs:156-213, avx2.rs:156-237 (widen in registers, m <= tile rows)
//   widen                 src/kernels/avx512.rs:220-265, avx2.rs:244-301
//   exp / store           src/kernels/avx512.rs:279-343, avx2.rs:305-406
//   gemm_panels / matmul  src/kernels/mod.rs:530-688 (KC = 256, the direct-narrow rule, the
//                         ceil(panels / (4 * threads)) task split)
//   Pool                  src/threads.rs:49-191 (the caller works too, idle workers spin 50 us
//                         and then sleep, a task's failure is raised again after all tasks end)
//   tdt_decode            src/parakeet.rs:1412-1513 (decode_inner) and 1524-1577 (predict_rows):
//                         every product is Kernels::linear on the pool, gate math by the host
//                         libm (sigmoid = 1/(1+exp(-x)), parakeet.rs:1678-1680), argmax the first
//                         largest value (parakeet.rs:1682-1691)
#include <immintrin.h>

#include <atomic>
#include <chrono>
#include <cmath>
#include <condition_variable>
#include <cstdint>
#include <cstring>
#include <functional>
#include <mutex>
#include <thread>
#include <vector>

namespace {

constexpr size_t PANEL = 16;
constexpr size_t Q8_BLOCK = 32;
constexpr size_t KC = 256;
enum { P_F32 = 0, P_F16 = 1, P_BF16 = 2, P_INT8 = 3, P_Q8_0 = 4 };
enum { ACT_NONE = 0, ACT_RELU = 1, ACT_SILU = 2 };
enum Isa { ISA_NONE = 0, ISA_AVX2 = 1, ISA_AVX512 = 2 };

size_t div_ceil(size_t a, size_t b) { return (a + b - 1) / b; }
size_t value_bytes(int p) { return p == P_F32 ? 4 : (p == P_F16 || p == P_BF16) ? 2 : 1; }

// ------------------------------------------------------------------ the pool

constexpr auto SPIN = std::chrono::microseconds(50);

class Pool {
  public:
    explicit Pool(size_t threads) : threads_(threads < 1 ? 1 : threads) {
        for (size_t i = 1; i < threads_; i++) workers_.emplace_back([this] { worker(); });
    }
    ~Pool() {
        {
            std::lock_guard<std::mutex> g(state_);
            shutdown_ = true;
        }
        wake_.notify_all();
        for (auto &w : workers_) w.join();
    }
    size_t threads() const { return threads_; }

    // Calls f(i) for every i in 0..tasks and waits for all. Returns false if a task threw.
    bool run(size_t tasks, const std::function<void(size_t)> &f) {
        if (tasks == 0) return true;
        if (threads_ == 1 || tasks == 1) {
            bool ok = true;
            for (size_t i = 0; i < tasks; i++) {
                try {
                    f(i);
                } catch (...) {
                    ok = false;
                }
            }
            return ok;
        }
        std::lock_guard<std::mutex> running(running_);
        {
            std::lock_guard<std::mutex> g(state_);
            next_.store(0, std::memory_order_relaxed);
            remaining_.store(tasks, std::memory_order_relaxed);
            job_ = &f;
            tasks_ = tasks;
            epoch_.store(epoch_.load(std::memory_order_relaxed) + 1, std::memory_order_release);
        }
        wake_.notify_all();
        run_tasks(f, tasks);
        auto start = std::chrono::steady_clock::now();
        while (remaining_.load(std::memory_order_acquire) != 0) {
            if (std::chrono::steady_clock::now() - start < SPIN) {
                _mm_pause();
            } else {
                std::this_thread::yield();
            }
        }
        {
            std::lock_guard<std::mutex> g(state_);
            job_ = nullptr;
        }
        while (active_.load(std::memory_order_acquire) != 0) std::this_thread::yield();
        return !failed_.exchange(false);
    }

  private:
    void run_tasks(const std::function<void(size_t)> &f, size_t tasks) {
        for (;;) {
            size_t i = next_.fetch_add(1, std::memory_order_relaxed);
            if (i >= tasks) return;
            try {
                f(i);
            } catch (...) {
                failed_.store(true, std::memory_order_relaxed);
            }
            remaining_.fetch_sub(1, std::memory_order_release);
        }
    }

    void worker() {
        uint64_t seen = 0;
        for (;;) {
            auto start = std::chrono::steady_clock::now();
            while (epoch_.load(std::memory_order_acquire) == seen &&
                   std::chrono::steady_clock::now() - start < SPIN)
                _mm_pause();
            const std::function<void(size_t)> *f;
            size_t tasks;
            {
                std::unique_lock<std::mutex> g(state_);
                wake_.wait(g, [&] { return epoch_.load(std::memory_order_relaxed) != seen || shutdown_; });
                if (shutdown_) return;
                seen = epoch_.load(std::memory_order_relaxed);
                if (!job_) continue;  // the job finished before this worker woke
                active_.fetch_add(1, std::memory_order_acq_rel);
                f = job_;
                tasks = tasks_;
            }
            run_tasks(*f, tasks);
            active_.fetch_sub(1, std::memory_order_acq_rel);
        }
    }

    size_t threads_;
    std::vector<std::thread> workers_;
    std::mutex state_, running_;
    std::condition_variable wake_;
    std::atomic<uint64_t> epoch_{0};
    std::atomic<size_t> next_{0}, remaining_{0}, active_{0};
    std::atomic<bool> failed_{false};
    const std::function<void(size_t)> *job_ = nullptr;
    size_t tasks_ = 0;
    bool shutdown_ = false;
};

// ------------------------------------------------------------------ AVX-512 kernels

#define T512 __attribute__((target("avx512f,fma,f16c")))
#define T256 __attribute__((target("avx2,fma,f16c")))

template <int R>
T512 void tile512(size_t k, const float *a, size_t lda, const float *b, size_t ks, float *out, bool load) {
    __m512 acc[R];
    for (int r = 0; r < R; r++) acc[r] = load ? _mm512_loadu_ps(out + r * PANEL) : _mm512_setzero_ps();
    for (size_t i = 0; i < k; i++) {
        __m512 bv = _mm512_loadu_ps(b + i * ks);
        for (int r = 0; r < R; r++) acc[r] = _mm512_fmadd_ps(_mm512_set1_ps(a[r * lda + i]), bv, acc[r]);
    }
    for (int r = 0; r < R; r++) _mm512_storeu_ps(out + r * PANEL, acc[r]);
}

T512 inline __m512 wide512(int p, const uint8_t *src, __m512 s) {
    if (p == P_F16) return _mm512_cvtph_ps(_mm256_loadu_si256((const __m256i *)src));
    if (p == P_BF16)
        return _mm512_castsi512_ps(
            _mm512_slli_epi32(_mm512_cvtepu16_epi32(_mm256_loadu_si256((const __m256i *)src)), 16));
    __m512 q = _mm512_cvtepi32_ps(_mm512_cvtepi8_epi32(_mm_loadu_si128((const __m128i *)src)));
    return _mm512_mul_ps(q, s);
}

template <int R>
T512 void tile_narrow512(int p, size_t k, const float *a, size_t lda, const uint8_t *b, const float *scales,
                         float *out, bool load) {
    __m512 acc[R];
    for (int r = 0; r < R; r++) acc[r] = load ? _mm512_loadu_ps(out + r * PANEL) : _mm512_setzero_ps();
    size_t step = (p == P_F16 || p == P_BF16) ? 32 : 16;
    __m512 s = p == P_INT8 ? _mm512_loadu_ps(scales) : _mm512_set1_ps(1.0f);
    size_t i = 0;
    while (i < k) {
        size_t end = k;
        if (p == P_Q8_0) {
            s = _mm512_loadu_ps(scales + i / Q8_BLOCK * PANEL);
            end = i + Q8_BLOCK < k ? i + Q8_BLOCK : k;
        }
        for (; i < end; i++) {
            __m512 w = wide512(p, b + i * step, s);
            for (int r = 0; r < R; r++) acc[r] = _mm512_fmadd_ps(_mm512_set1_ps(a[r * lda + i]), w, acc[r]);
        }
    }
    for (int r = 0; r < R; r++) _mm512_storeu_ps(out + r * PANEL, acc[r]);
}

T512 void widen512(int p, size_t k, const uint8_t *src, const float *scales, float *out) {
    if (p == P_F32) {
        std::memcpy(out, src, k * PANEL * 4);
        return;
    }
    size_t step = (p == P_F16 || p == P_BF16) ? 32 : 16;
    __m512 s = p == P_INT8 ? _mm512_loadu_ps(scales) : _mm512_set1_ps(1.0f);
    for (size_t i = 0; i < k; i++) {
        if (p == P_Q8_0 && i % Q8_BLOCK == 0) s = _mm512_loadu_ps(scales + i / Q8_BLOCK * PANEL);
        _mm512_storeu_ps(out + i * PANEL, wide512(p, src + i * step, s));
    }
}

// e^x in the reference's SIMD steps: clamp, n = rint(x log2 e), two-part reduction,
// degree-6 fused polynomial, times 2^n built from the exponent bits.
T512 __m512 exp512(__m512 x) {
    x = _mm512_min_ps(_mm512_max_ps(x, _mm512_set1_ps(-87.33654f)), _mm512_set1_ps(88.37626f));
    __m512 n = _mm512_roundscale_ps(_mm512_mul_ps(x, _mm512_set1_ps(1.44269504088896340736f)),
                                    _MM_FROUND_TO_NEAREST_INT | _MM_FROUND_NO_EXC);
    __m512 r = _mm512_fnmadd_ps(n, _mm512_set1_ps(0.6933594f), x);
    r = _mm512_fnmadd_ps(n, _mm512_set1_ps(-2.1219444e-4f), r);
    __m512 p = _mm512_set1_ps(1.9875691e-4f);
    p = _mm512_fmadd_ps(p, r, _mm512_set1_ps(1.3982e-3f));
    p = _mm512_fmadd_ps(p, r, _mm512_set1_ps(8.333452e-3f));
    p = _mm512_fmadd_ps(p, r, _mm512_set1_ps(4.1665796e-2f));
    p = _mm512_fmadd_ps(p, r, _mm512_set1_ps(0.16666665f));
    p = _mm512_fmadd_ps(p, r, _mm512_set1_ps(0.5f));
    p = _mm512_fmadd_ps(p, _mm512_mul_ps(r, r), r);
    p = _mm512_add_ps(p, _mm512_set1_ps(1.0f));
    __m512i e = _mm512_slli_epi32(_mm512_add_epi32(_mm512_cvtps_epi32(n), _mm512_set1_epi32(127)), 23);
    return _mm512_mul_ps(p, _mm512_castsi512_ps(e));
}

T512 void store512(const float *acc, float *c, size_t cols, const float *bias, int act, float scale, bool accumulate) {
    __mmask16 m = cols >= 16 ? (__mmask16)0xffff : (__mmask16)((1u << cols) - 1);
    __m512 v = _mm512_maskz_loadu_ps(m, acc);
    if (bias) v = _mm512_add_ps(v, _mm512_maskz_loadu_ps(m, bias));
    if (act == ACT_RELU) v = _mm512_max_ps(v, _mm512_setzero_ps());
    if (act == ACT_SILU) {
        __m512 e = exp512(_mm512_sub_ps(_mm512_setzero_ps(), v));
        v = _mm512_div_ps(v, _mm512_add_ps(_mm512_set1_ps(1.0f), e));
    }
    v = _mm512_mul_ps(v, _mm512_set1_ps(scale));
    if (accumulate) v = _mm512_add_ps(_mm512_maskz_loadu_ps(m, c), v);
    _mm512_mask_storeu_ps(c, m, v);
}

// ------------------------------------------------------------------ AVX2 kernels

template <int R>
T256 void tile256(size_t k, const float *a, size_t lda, const float *b, size_t ks, float *out, bool load) {
    __m256 acc0[R], acc1[R];
    for (int r = 0; r < R; r++) {
        acc0[r] = load ? _mm256_loadu_ps(out + r * PANEL) : _mm256_setzero_ps();
        acc1[r] = load ? _mm256_loadu_ps(out + r * PANEL + 8) : _mm256_setzero_ps();
    }
    for (size_t i = 0; i < k; i++) {
        __m256 b0 = _mm256_loadu_ps(b + i * ks), b1 = _mm256_loadu_ps(b + i * ks + 8);
        for (int r = 0; r < R; r++) {
            __m256 av = _mm256_broadcast_ss(a + r * lda + i);
            acc0[r] = _mm256_fmadd_ps(av, b0, acc0[r]);
            acc1[r] = _mm256_fmadd_ps(av, b1, acc1[r]);
        }
    }
    for (int r = 0; r < R; r++) {
        _mm256_storeu_ps(out + r * PANEL, acc0[r]);
        _mm256_storeu_ps(out + r * PANEL + 8, acc1[r]);
    }
}

T256 inline void wide256(int p, const uint8_t *src, __m256 s0, __m256 s1, __m256 &w0, __m256 &w1) {
    if (p == P_F16) {
        w0 = _mm256_cvtph_ps(_mm_loadu_si128((const __m128i *)src));
        w1 = _mm256_cvtph_ps(_mm_loadu_si128((const __m128i *)src + 1));
    } else if (p == P_BF16) {
        w0 = _mm256_castsi256_ps(_mm256_slli_epi32(_mm256_cvtepu16_epi32(_mm_loadu_si128((const __m128i *)src)), 16));
        w1 = _mm256_castsi256_ps(
            _mm256_slli_epi32(_mm256_cvtepu16_epi32(_mm_loadu_si128((const __m128i *)src + 1)), 16));
    } else {
        w0 = _mm256_mul_ps(_mm256_cvtepi32_ps(_mm256_cvtepi8_epi32(_mm_loadl_epi64((const __m128i *)src))), s0);
        w1 = _mm256_mul_ps(_mm256_cvtepi32_ps(_mm256_cvtepi8_epi32(_mm_loadl_epi64((const __m128i *)(src + 8)))),
                           s1);
    }
}

template <int R>
T256 void tile_narrow256(int p, size_t k, const float *a, size_t lda, const uint8_t *b, const float *scales,
                         float *out, bool load) {
    __m256 acc0[R], acc1[R];
    for (int r = 0; r < R; r++) {
        acc0[r] = load ? _mm256_loadu_ps(out + r * PANEL) : _mm256_setzero_ps();
        acc1[r] = load ? _mm256_loadu_ps(out + r * PANEL + 8) : _mm256_setzero_ps();
    }
    size_t step = (p == P_F16 || p == P_BF16) ? 32 : 16;
    __m256 s0 = _mm256_set1_ps(1.0f), s1 = s0;
    if (p == P_INT8) {
        s0 = _mm256_loadu_ps(scales);
        s1 = _mm256_loadu_ps(scales + 8);
    }
    size_t i = 0;
    while (i < k) {
        size_t end = k;
        if (p == P_Q8_0) {
            s0 = _mm256_loadu_ps(scales + i / Q8_BLOCK * PANEL);
            s1 = _mm256_loadu_ps(scales + i / Q8_BLOCK * PANEL + 8);
            end = i + Q8_BLOCK < k ? i + Q8_BLOCK : k;
        }
        for (; i < end; i++) {
            __m256 w0, w1;
            wide256(p, b + i * step, s0, s1, w0, w1);
            for (int r = 0; r < R; r++) {
                __m256 av = _mm256_broadcast_ss(a + r * lda + i);
                acc0[r] = _mm256_fmadd_ps(av, w0, acc0[r]);
                acc1[r] = _mm256_fmadd_ps(av, w1, acc1[r]);
            }
        }
    }
    for (int r = 0; r < R; r++) {
        _mm256_storeu_ps(out + r * PANEL, acc0[r]);
        _mm256_storeu_ps(out + r * PANEL + 8, acc1[r]);
    }
}

T256 void widen256(int p, size_t k, const uint8_t *src, const float *scales, float *out) {
    if (p == P_F32) {
        std::memcpy(out, src, k * PANEL * 4);
        return;
    }
    size_t step = (p == P_F16 || p == P_BF16) ? 32 : 16;
    __m256 s0 = _mm256_set1_ps(1.0f), s1 = s0;
    if (p == P_INT8) {
        s0 = _mm256_loadu_ps(scales);
        s1 = _mm256_loadu_ps(scales + 8);
    }
    for (size_t i = 0; i < k; i++) {
        if (p == P_Q8_0 && i % Q8_BLOCK == 0) {
            s0 = _mm256_loadu_ps(scales + i / Q8_BLOCK * PANEL);
            s1 = _mm256_loadu_ps(scales + i / Q8_BLOCK * PANEL + 8);
        }
        __m256 w0, w1;
        wide256(p, src + i * step, s0, s1, w0, w1);
        _mm256_storeu_ps(out + i * PANEL, w0);
        _mm256_storeu_ps(out + i * PANEL + 8, w1);
    }
}

T256 __m256 exp256(__m256 x) {
    x = _mm256_min_ps(_mm256_max_ps(x, _mm256_set1_ps(-87.33654f)), _mm256_set1_ps(88.37626f));
    __m256 n = _mm256_round_ps(_mm256_mul_ps(x, _mm256_set1_ps(1.44269504088896340736f)),
                               _MM_FROUND_TO_NEAREST_INT | _MM_FROUND_NO_EXC);
    __m256 r = _mm256_fnmadd_ps(n, _mm256_set1_ps(0.6933594f), x);
    r = _mm256_fnmadd_ps(n, _mm256_set1_ps(-2.1219444e-4f), r);
    __m256 p = _mm256_set1_ps(1.9875691e-4f);
    p = _mm256_fmadd_ps(p, r, _mm256_set1_ps(1.3982e-3f));
    p = _mm256_fmadd_ps(p, r, _mm256_set1_ps(8.333452e-3f));
    p = _mm256_fmadd_ps(p, r, _mm256_set1_ps(4.1665796e-2f));
    p = _mm256_fmadd_ps(p, r, _mm256_set1_ps(0.16666665f));
    p = _mm256_fmadd_ps(p, r, _mm256_set1_ps(0.5f));
    p = _mm256_fmadd_ps(p, _mm256_mul_ps(r, r), r);
    p = _mm256_add_ps(p, _mm256_set1_ps(1.0f));
    __m256i e = _mm256_slli_epi32(_mm256_add_epi32(_mm256_cvtps_epi32(n), _mm256_set1_epi32(127)), 23);
    return _mm256_mul_ps(p, _mm256_castsi256_ps(e));
}

T256 void store256(const float *acc, float *c, size_t cols, const float *bias, int act, float scale, bool accumulate) {
    // Whole 8-lane halves where the panel is full; lane by lane (the same operations) otherwise.
    float lane_acc[16] = {0}, lane_bias[16] = {0}, lane_c[16] = {0};
    std::memcpy(lane_acc, acc, cols * 4);
    if (bias) std::memcpy(lane_bias, bias, cols * 4);
    if (accumulate) std::memcpy(lane_c, c, cols * 4);
    for (int h = 0; h < 2; h++) {
        __m256 v = _mm256_loadu_ps(lane_acc + 8 * h);
        if (bias) v = _mm256_add_ps(v, _mm256_loadu_ps(lane_bias + 8 * h));
        if (act == ACT_RELU) v = _mm256_max_ps(v, _mm256_setzero_ps());
        if (act == ACT_SILU) {
            __m256 e = exp256(_mm256_sub_ps(_mm256_setzero_ps(), v));
            v = _mm256_div_ps(v, _mm256_add_ps(_mm256_set1_ps(1.0f), e));
        }
        v = _mm256_mul_ps(v, _mm256_set1_ps(scale));
        if (accumulate) v = _mm256_add_ps(_mm256_loadu_ps(lane_c + 8 * h), v);
        _mm256_storeu_ps(lane_c + 8 * h, v);
    }
    std::memcpy(c, lane_c, cols * 4);
}

// ------------------------------------------------------------------ the driver

struct Kernels {
    Isa isa;
    size_t tile_rows;
    void (*tile)(size_t rows, size_t k, const float *a, size_t lda, const float *b, size_t ks, float *out, bool load);
    void (*tile_narrow)(size_t rows, int p, size_t k, const float *a, size_t lda, const uint8_t *b,
                        const float *scales, float *out, bool load);
    void (*widen)(int p, size_t k, const uint8_t *src, const float *scales, float *out);
    void (*store)(const float *acc, float *c, size_t cols, const float *bias, int act, float scale, bool accumulate);
};

template <template <int> class F, int MAXR>
struct Dispatch;

#define ROWS_SWITCH(MAXR, CALL)                                                                                  \
    switch (rows) {                                                                                              \
    case 1: CALL(1); break;                                                                                      \
    case 2: CALL(2); break;                                                                                      \
    case 3: CALL(3); break;                                                                                      \
    case 4: CALL(4); break;                                                                                      \
    case 5: CALL(5); break;                                                                                      \
    case 6: CALL(6); break;                                                                                      \
    case 7: if (MAXR >= 7) CALL(7); break;                                                                       \
    case 8: if (MAXR >= 8) CALL(8); break;                                                                       \
    default: break;                                                                                              \
    }

void tile_512(size_t rows, size_t k, const float *a, size_t lda, const float *b, size_t ks, float *out, bool load) {
#define C512(R) tile512<R>(k, a, lda, b, ks, out, load)
    ROWS_SWITCH(8, C512)
#undef C512
}
void narrow_512(size_t rows, int p, size_t k, const float *a, size_t lda, const uint8_t *b, const float *s, float *out,
                bool load) {
#define N512(R) tile_narrow512<R>(p, k, a, lda, b, s, out, load)
    ROWS_SWITCH(8, N512)
#undef N512
}
void tile_256(size_t rows, size_t k, const float *a, size_t lda, const float *b, size_t ks, float *out, bool load) {
#define C256(R) tile256<(R > 6 ? 6 : R)>(k, a, lda, b, ks, out, load)
    ROWS_SWITCH(6, C256)
#undef C256
}
void narrow_256(size_t rows, int p, size_t k, const float *a, size_t lda, const uint8_t *b, const float *s, float *out,
                bool load) {
#define N256(R) tile_narrow256<(R > 6 ? 6 : R)>(p, k, a, lda, b, s, out, load)
    ROWS_SWITCH(6, N256)
#undef N256
}

Isa detect_isa() {
    __builtin_cpu_init();
    if (__builtin_cpu_supports("avx512f") && __builtin_cpu_supports("fma") && __builtin_cpu_supports("f16c"))
        return ISA_AVX512;
    if (__builtin_cpu_supports("avx2") && __builtin_cpu_supports("fma") && __builtin_cpu_supports("f16c"))
        return ISA_AVX2;
    return ISA_NONE;
}

bool make_kernels(int isa, Kernels &k) {
    if (isa == ISA_AVX512) {
        k = {ISA_AVX512, 8, tile_512, narrow_512, widen512, store512};
        return true;
    }
    if (isa == ISA_AVX2) {
        k = {ISA_AVX2, 6, tile_256, narrow_256, widen256, store256};
        return true;
    }
    return false;
}

// gemm_panels for the panels in [p0, p1).
void gemm_panels(const Kernels &kn, const float *a, size_t lda, size_t m, const uint8_t *values, const float *scales,
                 int p, size_t n, size_t k, size_t p0, size_t p1, float *c, size_t ldc, const float *bias, int act,
                 float scale, bool accumulate) {
    bool narrow = p != P_F32;
    size_t vb = value_bytes(p), blocks = div_ceil(k, Q8_BLOCK);
    bool direct = narrow && m <= kn.tile_rows;
    std::vector<float> wide(narrow && !direct ? KC * PANEL : 0);
    std::vector<float> partial(m * PANEL, 0.0f);
    for (size_t pp = p0; pp < p1; pp++) {
        size_t col = pp * PANEL, cols = n - col < PANEL ? n - col : PANEL;
        for (size_t k0 = 0; k0 < k; k0 += KC) {
            size_t kc = k - k0 < KC ? k - k0 : KC;
            const float *sc = nullptr;
            if (p == P_INT8) sc = scales + pp * PANEL;
            if (p == P_Q8_0) sc = scales + (pp * blocks + k0 / Q8_BLOCK) * PANEL;
            const uint8_t *src = values + (pp * k + k0) * PANEL * vb;
            if (direct) {
                kn.tile_narrow(m, p, kc, a + k0, lda, src, sc, partial.data(), k0 > 0);
                continue;
            }
            const float *bp = reinterpret_cast<const float *>(src);
            if (narrow) {
                kn.widen(p, kc, src, sc, wide.data());
                bp = wide.data();
            }
            for (size_t row = 0; row < m; row += kn.tile_rows) {
                size_t rows = m - row < kn.tile_rows ? m - row : kn.tile_rows;
                kn.tile(rows, kc, a + row * lda + k0, lda, bp, PANEL, partial.data() + row * PANEL, k0 > 0);
            }
        }
        for (size_t r = 0; r < m; r++)
            kn.store(partial.data() + r * PANEL, c + r * ldc + col, cols, bias ? bias + col : nullptr, act, scale,
                     accumulate);
    }
}

// Kernels::matmul: the pool splits the panels, a few tasks per thread. False if a task threw.
bool pool_matmul(Pool *pl, const Kernels &kn, const float *a, size_t lda, size_t m, const uint8_t *values,
                 const float *scales, int p, size_t n, size_t k, float *c, size_t ldc, const float *bias, int act,
                 float scale, bool accumulate) {
    size_t panels = div_ceil(n, PANEL);
    size_t per_task = div_ceil(panels, pl->threads() * 4);
    if (per_task < 1) per_task = 1;
    size_t tasks = div_ceil(panels, per_task);
    return pl->run(tasks, [&](size_t t) {
        size_t p0 = t * per_task, p1 = (t + 1) * per_task < panels ? (t + 1) * per_task : panels;
        gemm_panels(kn, a, lda, m, values, scales, p, n, k, p0, p1, c, ldc, bias, act, scale, accumulate);
    });
}

// ------------------------------------------------------------------ the TDT decoder

float sigmoid(float x) { return 1.0f / (1.0f + std::exp(-x)); }

size_t argmax(const float *v, size_t n) {
    size_t best = 0;
    for (size_t i = 0; i < n; i++)
        if (v[i] > v[best]) best = i;
    return best;
}

struct Tdt {
    Pool *pool;
    Kernels kn;
    int p;
    size_t h, layers;
    const float *emb;
    const uint8_t *const *lstm_v;
    const float *const *lstm_s, *const *lstm_b;
    const uint8_t *proj_v;
    const float *proj_s, *proj_b;
    std::vector<float> input, gates;

    bool linear(const float *a, const uint8_t *v, const float *s, size_t n, size_t k, const float *bias, float *c) {
        return pool_matmul(pool, kn, a, k, 1, v, s, p, n, k, c, n, bias, ACT_NONE, 1.0f, false);
    }

    // predict_rows for one token: state is layers x [h, c], pred h floats.
    bool predict(size_t token, float *state, float *pred) {
        std::memcpy(input.data(), emb + token * h, h * sizeof(float));
        for (size_t l = 0; l < layers; l++) {
            float *hs = state + l * 2 * h, *cs = hs + h;
            std::memcpy(input.data() + h, hs, h * sizeof(float));
            if (!linear(input.data(), lstm_v[l], lstm_s[l], 4 * h, 2 * h, lstm_b[l], gates.data())) return false;
            const float *g = gates.data();
            for (size_t j = 0; j < h; j++) {
                float i = sigmoid(g[j]), f = sigmoid(g[h + j]), gg = std::tanh(g[2 * h + j]),
                      o = sigmoid(g[3 * h + j]);
                cs[j] = f * cs[j] + i * gg;
                hs[j] = o * std::tanh(cs[j]);
            }
            std::memcpy(input.data(), hs, h * sizeof(float));
        }
        return linear(input.data(), proj_v, proj_s, h, h, proj_b, pred);
    }
};

}  // namespace

extern "C" {

// 2 = AVX-512F+FMA+F16C, 1 = AVX2+FMA+F16C, 0 = neither (the baseline cannot run).
int cb_isa(void) { return detect_isa(); }

void *cb_pool_new(size_t threads) { return new Pool(threads); }
void cb_pool_free(void *pool) { delete static_cast<Pool *>(pool); }
size_t cb_pool_threads(void *pool) { return static_cast<Pool *>(pool)->threads(); }

// Pool test hook: runs `tasks` tasks; task i increments counts[i] and throws if i == fail_at.
// Returns 0, or -1 if a task threw (raised again after every task finished).
int cb_pool_test(void *pool, size_t tasks, uint32_t *counts, long fail_at) {
    bool ok = static_cast<Pool *>(pool)->run(tasks, [&](size_t i) {
        __atomic_fetch_add(&counts[i], 1u, __ATOMIC_RELAXED);
        if ((long)i == fail_at) throw 1;
    });
    return ok ? 0 : -1;
}

// Kernels::matmul on the pool with the ISA `isa` (2 or 1; 0 picks the fastest). Returns 0,
// -2 for a shape the reference rejects, -5 if the ISA is not available.
int cb_matmul(void *pool, int isa, const float *a, size_t a_len, size_t lda, size_t m, const uint8_t *values,
              const float *scales, int p, size_t n, size_t k, float *c, size_t c_len, size_t ldc, const float *bias,
              size_t bias_len, int act, float scale, int accumulate) {
    if (m == 0 || n == 0) return 0;
    if (lda < k || ldc < n || a_len < (m - 1) * lda + k || c_len < (m - 1) * ldc + n) return -2;
    if (bias && bias_len < n) return -2;
    if (p == P_Q8_0 && k % Q8_BLOCK) return -7;
    Kernels kn;
    if (!make_kernels(isa == 0 ? detect_isa() : isa, kn) || (isa != 0 && detect_isa() < isa)) return -5;
    bool ok = pool_matmul(static_cast<Pool *>(pool), kn, a, lda, m, values, scales, p, n, k, c, ldc, bias, act,
                          scale, accumulate != 0);
    return ok ? 0 : -4;
}

// decode_inner from frame *t_io with *on_frame_io tokens on it, every product on the pool with the
// ISA `isa` (0 picks the fastest). Weights are int8 (p = 3) or Q8_0 (p = 4) in the panel layout:
// the joint (vocab + ndur) x h, `layers` LSTM matrices 4h x 2h, the projection h x h. enc holds
// frames rows of h floats (stride lde); state is layers x [h, c] and pred h floats, both updated.
// Tokens get (id, frame, duration) triples, at most cap of them. Returns the number emitted, -5 if
// the ISA is not available, -4 if a task failed.
long cb_tdt_decode(void *pool, int isa, int p, size_t h, size_t layers, size_t vocab, const int32_t *durations,
                   size_t ndur, size_t max_symbols, const uint8_t *joint_v, const float *joint_s,
                   const float *joint_b, const float *emb, const uint8_t *const *lstm_v,
                   const float *const *lstm_s, const float *const *lstm_b, const uint8_t *proj_v,
                   const float *proj_s, const float *proj_b, const float *enc, size_t lde, size_t frames,
                   float *state, float *pred, size_t *t_io, size_t *on_frame_io, int32_t *tokens, size_t cap) {
    Tdt d{static_cast<Pool *>(pool), {}, p, h, layers, emb, lstm_v, lstm_s, lstm_b, proj_v, proj_s, proj_b,
          std::vector<float>(2 * h), std::vector<float>(4 * h)};
    if (!make_kernels(isa == 0 ? detect_isa() : isa, d.kn) || (isa != 0 && detect_isa() < isa)) return -5;
    const size_t outputs = vocab + ndur, blank = vocab - 1;
    std::vector<float> z(h), logits(outputs);
    size_t t = *t_io, on_frame = *on_frame_io;
    long count = 0;
    while (t < frames) {
        for (size_t i = 0; i < h; i++) z[i] = std::fmax(enc[t * lde + i] + pred[i], 0.0f);
        if (!d.linear(z.data(), joint_v, joint_s, outputs, h, joint_b, logits.data())) return -4;
        const size_t token = argmax(logits.data(), vocab);
        const size_t duration = (size_t)durations[argmax(logits.data() + vocab, ndur)];
        if (token == blank) {
            t += duration > 1 ? duration : 1;
            on_frame = 0;
            continue;
        }
        if ((size_t)count < cap) {
            tokens[3 * count] = (int32_t)token;
            tokens[3 * count + 1] = (int32_t)t;
            tokens[3 * count + 2] = (int32_t)duration;
        }
        count++;
        if (!d.predict(token, state, pred)) return -4;
        if (duration > 0) {
            t += duration;
            on_frame = 0;
        } else if (++on_frame >= max_symbols) {
            t += 1;
            on_frame = 0;
        }
    }
    *t_io = t;
    *on_frame_io = on_frame;
    return count;
}

}  // extern "C"
