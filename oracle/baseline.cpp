// baseline.cpp — ingot's amd64 CPU algorithm for the hot path, restated in
// C++ ("port": the Go reference cannot be built here), used ONLY as the
// cpu_baseline leg of bench.py and as a second checker in tests. Never part
// of the product.
//
// f32 / bf16-weight GEMM: the Goto/BLIS packed-B sweep of
// kernels/gemm/gemm.go:280-334,431-490,849-913 with the amd64 blocking of
// kernels/gemm/params_amd64.go:8-14 (MR=6, NR=16, MC=144, KC=384), B packed
// once as [kBlock][nPanel][KC·NR] (PackB, kernels/gemm/gemm.go:860-885;
// bf16 panels widened per task like PackBBF16/widenPanel :920-962), A packed
// per MC block as [kBlock][mPanel][KC·MR], the 6×16 FMA micro-kernel of
// kernels/gemm/ukernel_amd64.s (zeroed accumulators, C added at the store,
// bias after: kernels/gemm/ukernel_generic.go:15-46), and par.Run's dynamic
// chunked parallel-for over N-panels (kernels/par/par.go:172-241).
// bf16 GEMV: GemvBF16 (kernels/gemm/bgemm.go:201-206) parallel over rows
// with a widening dot. int8: QgemmRef-exact u8·s8 products (s8 path of
// ops/quant.go:831-900): AVX-512 VNNI (VPDPBUSD) on 4×4 blocks of rows when
// the CPU has F+VL+VNNI, as the reference picks its VNNI kernel
// (kernels/gemm/qkernel_pick_amd64.go:18-30), else AVX2 int16 madd;
// parallel over row blocks.
//
// Micro-kernel choice (kernels/gemm/ukernel_amd64.go:33-93): the AVX-512
// 6×16 kernel only when the CPU has AVX-512F and a start-up probe (best of 3
// tight loops of 24 calls on a cache-hot 6×16 tile, kc = 384) finds it more
// than 5% faster than the AVX2 one; INGOT_GEMM_KERNEL=avx2 / avx512 pins it.

#include <immintrin.h>

#include <algorithm>
#include <atomic>
#include <cmath>
#include <cstdint>
#include <cstring>
#include <chrono>
#include <cstdlib>
#include <condition_variable>
#include <functional>
#include <mutex>
#include <thread>
#include <vector>

namespace {

constexpr int MR = 6, NR = 16, MC = 144, KC = 384;

inline float bf16f(uint16_t h) {
    uint32_t b = (uint32_t)h << 16;
    float f;
    memcpy(&f, &b, 4);
    return f;
}

// par.Run: tasks [0, n) handed out in chunks of `grain` from an atomic counter to the caller (worker 0)
// and up to threads-1 helpers of a pool that lives for the process (kernels/par/par.go:1-25,172-241).
// Each helper has its own mailbox (a generation number): the caller fills in the region, then bumps the
// mailboxes of the helpers it enlists and waits until each of them has finished, so a helper never reads a
// region that is not its own. Helpers spin on their mailbox for about 50 µs, then sleep on a condition
// variable, so back-to-back regions start without a thread wake-up. One region runs at a time, and a
// region's task must not start another (the pool would wait on itself).
class Pool {
public:
    static constexpr int kMaxHelpers = 255;

    void run(int64_t n, int64_t grain, int threads, const std::function<void(int64_t, int)>& fn) {
        std::lock_guard<std::mutex> region(region_);
        const int helpers = std::min(threads - 1, kMaxHelpers);
        grow(helpers);
        fn_ = &fn;
        n_ = n;
        grain_ = grain;
        next_.store(0, std::memory_order_relaxed);
        pending_.store(helpers, std::memory_order_relaxed);
        {
            std::lock_guard<std::mutex> l(mu_);
            for (int id = 1; id <= helpers; ++id) box_[id].fetch_add(1, std::memory_order_release);
        }
        wake_.notify_all();
        claim(0);
        while (pending_.load(std::memory_order_acquire) != 0) _mm_pause();
    }
    ~Pool() {
        {
            std::lock_guard<std::mutex> l(mu_);
            stop_.store(true, std::memory_order_relaxed);
            for (size_t id = 1; id <= helpers_.size(); ++id) box_[id].fetch_add(1, std::memory_order_release);
        }
        wake_.notify_all();
        for (auto& t : helpers_) t.join();
    }

private:
    void claim(int w) {
        for (;;) {
            const int64_t i0 = next_.fetch_add(grain_, std::memory_order_relaxed);
            if (i0 >= n_) return;
            const int64_t i1 = std::min(n_, i0 + grain_);
            for (int64_t i = i0; i < i1; ++i) (*fn_)(i, w);
        }
    }
    void grow(int helpers) {
        while ((int)helpers_.size() < helpers) {
            const int id = (int)helpers_.size() + 1;
            const uint64_t seen = box_[id].load(std::memory_order_acquire);
            helpers_.emplace_back([this, id, seen] { loop(id, seen); });
        }
    }
    void loop(int id, uint64_t seen) {
        std::atomic<uint64_t>& box = box_[id];
        for (;;) {
            uint64_t g;
            const auto until = std::chrono::steady_clock::now() + std::chrono::microseconds(50);
            int spins = 0;
            while ((g = box.load(std::memory_order_acquire)) == seen) {
                _mm_pause();
                if (++spins % 1024 == 0 && std::chrono::steady_clock::now() > until) {
                    std::unique_lock<std::mutex> l(mu_);
                    wake_.wait(l, [&] { return box.load(std::memory_order_acquire) != seen; });
                }
            }
            seen = g;
            if (stop_.load(std::memory_order_relaxed)) return;
            claim(id);
            pending_.fetch_sub(1, std::memory_order_acq_rel);
        }
    }

    std::mutex region_, mu_;
    std::condition_variable wake_;
    std::vector<std::thread> helpers_;
    std::atomic<uint64_t> box_[kMaxHelpers + 1] = {};
    std::atomic<int64_t> next_{0};
    std::atomic<int> pending_{0};
    std::atomic<bool> stop_{false};
    const std::function<void(int64_t, int)>* fn_ = nullptr;
    int64_t n_ = 0, grain_ = 1;
};

Pool& pool() {
    static Pool p;
    return p;
}

void par_run(int64_t n, int64_t grain, int threads, const std::function<void(int64_t, int)>& fn) {
    if (threads <= 1 || n <= grain) {
        for (int64_t i = 0; i < n; ++i) fn(i, 0);
        return;
    }
    // no more helpers than there are chunks to hand out
    threads = (int)std::min<int64_t>(threads, (n + grain - 1) / grain);
    pool().run(n, grain, threads, fn);
}

struct Packed {
    int64_t k, n, np, nkb;
    std::vector<float> f32;     // [kb][jp][KC*NR]
    std::vector<uint16_t> b16;  // same layout as bf16 bits
};

// C[MR×NR] (+)= Ap[kc×MR]ᵀ·Bp[kc×NR]; then + bias (the fused Linear bias).
inline void micro_kernel(int kc, const float* ap, const float* bp, float* c, int64_t ldc, bool accumulate,
                         const float* bias, int mr, int nr) {
    __m256 acc[MR][2];
    for (int i = 0; i < MR; ++i) acc[i][0] = acc[i][1] = _mm256_setzero_ps();
    for (int p = 0; p < kc; ++p) {
        const __m256 b0 = _mm256_loadu_ps(bp + p * NR);
        const __m256 b1 = _mm256_loadu_ps(bp + p * NR + 8);
        for (int i = 0; i < MR; ++i) {
            const __m256 a = _mm256_broadcast_ss(ap + p * MR + i);
            acc[i][0] = _mm256_fmadd_ps(a, b0, acc[i][0]);
            acc[i][1] = _mm256_fmadd_ps(a, b1, acc[i][1]);
        }
    }
    alignas(32) float t[MR][NR];
    for (int i = 0; i < MR; ++i) {
        _mm256_store_ps(t[i], acc[i][0]);
        _mm256_store_ps(t[i] + 8, acc[i][1]);
    }
    for (int i = 0; i < mr; ++i) {
        float* row = c + i * ldc;
        for (int j = 0; j < nr; ++j) {
            float v = accumulate ? row[j] + t[i][j] : t[i][j];
            if (bias) v += bias[j];
            row[j] = v;
        }
    }
}

// The same tile with one 16-wide AVX-512 accumulator per row
// (microKernelAVX512, kernels/gemm/ukernel_amd64_avx512.s:9).
__attribute__((target("avx512f"))) void micro_kernel_512(int kc, const float* ap, const float* bp, float* c,
                                                         int64_t ldc, bool accumulate, const float* bias, int mr,
                                                         int nr) {
    __m512 acc[MR];
    for (int i = 0; i < MR; ++i) acc[i] = _mm512_setzero_ps();
    for (int p = 0; p < kc; ++p) {
        const __m512 b = _mm512_loadu_ps(bp + p * NR);
        for (int i = 0; i < MR; ++i) acc[i] = _mm512_fmadd_ps(_mm512_set1_ps(ap[p * MR + i]), b, acc[i]);
    }
    alignas(64) float t[MR][NR];
    for (int i = 0; i < MR; ++i) _mm512_store_ps(t[i], acc[i]);
    for (int i = 0; i < mr; ++i) {
        float* row = c + i * ldc;
        for (int j = 0; j < nr; ++j) {
            float v = accumulate ? row[j] + t[i][j] : t[i][j];
            if (bias) v += bias[j];
            row[j] = v;
        }
    }
}

typedef void (*MicroKernel)(int, const float*, const float*, float*, int64_t, bool, const float*, int, int);

// avx512Faster (kernels/gemm/ukernel_amd64.go:65-93).
bool avx512_faster() {
    constexpr int kc = 384;
    std::vector<float> ap(kc * MR), bp(kc * NR), c(MR * NR);
    for (size_t i = 0; i < ap.size(); ++i) ap[i] = (float)(i % 7) * 0.5f;
    for (size_t i = 0; i < bp.size(); ++i) bp[i] = (float)(i % 5) * 0.25f;
    auto bench = [&](MicroKernel k) {
        k(kc, ap.data(), bp.data(), c.data(), NR, false, nullptr, MR, NR);
        double best = 1e30;
        for (int r = 0; r < 3; ++r) {
            const auto t0 = std::chrono::steady_clock::now();
            for (int i = 0; i < 24; ++i) k(kc, ap.data(), bp.data(), c.data(), NR, false, nullptr, MR, NR);
            best = std::min(best, std::chrono::duration<double>(std::chrono::steady_clock::now() - t0).count());
        }
        return best;
    };
    const double a2 = bench(micro_kernel), a5 = bench(micro_kernel_512);
    return a5 * 100 < a2 * 95;
}

struct KernelPick {
    MicroKernel fn = micro_kernel;
    const char* name = "avx2";
    bool vnni = false;
    KernelPick() {
        __builtin_cpu_init();
        const bool has512 = __builtin_cpu_supports("avx512f");
        vnni = has512 && __builtin_cpu_supports("avx512vl") && __builtin_cpu_supports("avx512vnni");
        const char* force = getenv("INGOT_GEMM_KERNEL");
        const bool want512 = force && !strcmp(force, "avx512");
        const bool want2 = force && !strcmp(force, "avx2");
        if (has512 && (want512 || (!want2 && avx512_faster()))) {
            fn = micro_kernel_512;
            name = "avx512";
        }
    }
};

const KernelPick& pick() {
    static const KernelPick k;
    return k;
}

// Σ_p a[p]·b[p] over k bytes, u8 × s8, for 4 rows of A × 4 rows of Bᵀ
// (VPDPBUSD: exact int32 sums of four u8·s8 products per lane).
__attribute__((target("avx512f,avx512vl,avx512bw,avx512vnni"))) void qdot4x4_vnni(const uint8_t* const* ar,
                                                                                  const int8_t* const* br, int64_t k,
                                                                                  uint32_t out[4][4]) {
    __m512i acc[4][4];
    for (int i = 0; i < 4; ++i)
        for (int j = 0; j < 4; ++j) acc[i][j] = _mm512_setzero_si512();
    int64_t p = 0;
    for (; p + 64 <= k; p += 64) {
        __m512i av[4], bv[4];
        for (int i = 0; i < 4; ++i) av[i] = _mm512_loadu_si512(ar[i] + p);
        for (int j = 0; j < 4; ++j) bv[j] = _mm512_loadu_si512(br[j] + p);
        for (int i = 0; i < 4; ++i)
            for (int j = 0; j < 4; ++j) acc[i][j] = _mm512_dpbusd_epi32(acc[i][j], av[i], bv[j]);
    }
    for (int i = 0; i < 4; ++i)
        for (int j = 0; j < 4; ++j) {
            uint32_t s = (uint32_t)_mm512_reduce_add_epi32(acc[i][j]);
            for (int64_t q = p; q < k; ++q) s += (uint32_t)((int32_t)ar[i][q] * (int32_t)br[j][q]);
            out[i][j] = s;
        }
}

}  // namespace

extern "C" {

// Which micro-kernel and int8 kernel the probe picked ("avx512" / "avx2",
// vnni 1 / 0).
const char* base_active_kernel(int* vnni) {
    if (vnni) *vnni = pick().vnni ? 1 : 0;
    return pick().name;
}

// PackB (kernels/gemm/gemm.go:860-885): B[k×n] (transB: stored [n×k]).
void* base_pack_b_f32(int64_t k, int64_t n, const float* b, int64_t ldb, int transB) {
    auto* p = new Packed();
    p->k = k;
    p->n = n;
    p->np = (n + NR - 1) / NR;
    p->nkb = (k + KC - 1) / KC;
    p->f32.assign((size_t)(p->nkb * p->np * KC * NR), 0.f);
    for (int64_t kb = 0; kb < p->nkb; ++kb)
        for (int64_t jp = 0; jp < p->np; ++jp) {
            float* dst = &p->f32[(size_t)((kb * p->np + jp) * KC * NR)];
            for (int64_t pp = 0; pp < std::min<int64_t>(KC, k - kb * KC); ++pp)
                for (int64_t j = 0; j < std::min<int64_t>(NR, n - jp * NR); ++j) {
                    const int64_t kk = kb * KC + pp, nn = jp * NR + j;
                    dst[pp * NR + j] = transB ? b[nn * ldb + kk] : b[kk * ldb + nn];
                }
        }
    return p;
}

// PackBBF16 (kernels/gemm/gemm.go:920-954): the same panels as bf16 bits.
void* base_pack_b_bf16(int64_t k, int64_t n, const uint16_t* b, int64_t ldb, int transB) {
    auto* p = new Packed();
    p->k = k;
    p->n = n;
    p->np = (n + NR - 1) / NR;
    p->nkb = (k + KC - 1) / KC;
    p->b16.assign((size_t)(p->nkb * p->np * KC * NR), 0);
    for (int64_t kb = 0; kb < p->nkb; ++kb)
        for (int64_t jp = 0; jp < p->np; ++jp) {
            uint16_t* dst = &p->b16[(size_t)((kb * p->np + jp) * KC * NR)];
            for (int64_t pp = 0; pp < std::min<int64_t>(KC, k - kb * KC); ++pp)
                for (int64_t j = 0; j < std::min<int64_t>(NR, n - jp * NR); ++j) {
                    const int64_t kk = kb * KC + pp, nn = jp * NR + j;
                    dst[pp * NR + j] = transB ? b[nn * ldb + kk] : b[kk * ldb + nn];
                }
        }
    return p;
}

void base_free_packed(void* h) { delete (Packed*)h; }

// SgemmPackedB / SgemmPackedBEpi (kernels/gemm/gemm.go:521-597, 887-913):
// C[m×n] = A·B (+ bias), optional GELU(erf) over each finished row strip.
void base_sgemm_packed(int64_t m, const float* a, int64_t lda, const void* handle, float* c, int64_t ldc,
                       const float* bias, int gelu, int threads) {
    const Packed* p = (const Packed*)handle;
    const int64_t k = p->k, n = p->n, np = p->np, nkb = p->nkb;
    std::vector<std::vector<float>> widen(std::max(threads, 1), std::vector<float>(KC * NR));
    std::vector<float> ap;
    for (int64_t i0 = 0; i0 < m; i0 += MC) {
        const int64_t mc = std::min<int64_t>(MC, m - i0);
        const int64_t mp = (mc + MR - 1) / MR;
        ap.assign((size_t)(nkb * mp * KC * MR), 0.f);
        // smallPackA: [kb][ip][KC*MR]
        par_run(nkb * mp, 4, threads, [&](int64_t t, int) {
            const int64_t kb = t / mp, ip = t % mp;
            float* dst = &ap[(size_t)((kb * mp + ip) * KC * MR)];
            const int64_t kc = std::min<int64_t>(KC, k - kb * KC);
            const int64_t mr = std::min<int64_t>(MR, mc - ip * MR);
            for (int64_t pp = 0; pp < kc; ++pp)
                for (int64_t r = 0; r < MR; ++r)
                    dst[pp * MR + r] = r < mr ? a[(i0 + ip * MR + r) * lda + kb * KC + pp] : 0.f;
        });
        // smallMSweep: one task per N-panel
        par_run(np, 1, threads, [&](int64_t jp, int w) {
            const int64_t nr = std::min<int64_t>(NR, n - jp * NR);
            for (int64_t kb = 0; kb < nkb; ++kb) {
                const int64_t kc = std::min<int64_t>(KC, k - kb * KC);
                const float* bp;
                if (!p->b16.empty()) {
                    const uint16_t* src = &p->b16[(size_t)((kb * np + jp) * KC * NR)];
                    float* dst = widen[w].data();
                    for (int64_t i = 0; i < kc * NR; ++i) dst[i] = bf16f(src[i]);
                    bp = dst;
                } else {
                    bp = &p->f32[(size_t)((kb * np + jp) * KC * NR)];
                }
                const bool last = kb == nkb - 1;
                const MicroKernel mk = pick().fn;
                for (int64_t ip = 0; ip < mp; ++ip) {
                    const int64_t mr = std::min<int64_t>(MR, mc - ip * MR);
                    mk((int)kc, &ap[(size_t)((kb * mp + ip) * KC * MR)], bp,
                                 c + (i0 + ip * MR) * ldc + jp * NR, ldc, kb > 0, last && bias ? bias + jp * NR : nullptr,
                                 (int)mr, (int)nr);
                }
            }
            if (gelu) {
                for (int64_t i = 0; i < mc; ++i) {
                    float* row = c + (i0 + i) * ldc + jp * NR;
                    for (int64_t j = 0; j < nr; ++j) {
                        const float x = row[j];
                        row[j] = 0.5f * x * (1.f + (float)std::erf((double)x / std::sqrt(2.0)));
                    }
                }
            }
        });
    }
}

// GemvBF16 per activation row (kernels/gemm/bgemm.go:201-206; ops/matmul.go:86-96).
void base_gemv_bf16(int64_t m, int64_t k, int64_t n, const float* x, const uint16_t* w, float* y, int threads) {
    for (int64_t i = 0; i < m; ++i) {
        const float* xr = x + i * k;
        float* yr = y + i * n;
        par_run(n, std::max<int64_t>(1, 65536 / std::max<int64_t>(k, 1)), threads, [&](int64_t j, int) {
            const uint16_t* wr = w + j * k;
            __m256 s0 = _mm256_setzero_ps(), s1 = _mm256_setzero_ps();
            int64_t p = 0;
            for (; p + 16 <= k; p += 16) {
                const __m128i h0 = _mm_loadu_si128((const __m128i*)(wr + p));
                const __m128i h1 = _mm_loadu_si128((const __m128i*)(wr + p + 8));
                const __m256 w0 = _mm256_castsi256_ps(_mm256_slli_epi32(_mm256_cvtepu16_epi32(h0), 16));
                const __m256 w1 = _mm256_castsi256_ps(_mm256_slli_epi32(_mm256_cvtepu16_epi32(h1), 16));
                s0 = _mm256_fmadd_ps(_mm256_loadu_ps(xr + p), w0, s0);
                s1 = _mm256_fmadd_ps(_mm256_loadu_ps(xr + p + 8), w1, s1);
            }
            alignas(32) float t[8];
            _mm256_store_ps(t, _mm256_add_ps(s0, s1));
            float s = 0;
            for (int e = 0; e < 8; ++e) s += t[e];
            for (; p < k; ++p) s += xr[p] * bf16f(wr[p]);
            yr[j] = s;
        });
    }
}

// MatMulInteger core: Y[m×n] = Σ_p (A[i,p] − za)·B[p,j], B given transposed
// ([n×k] s8, like bWeights' Bᵀ), exact int32.
void base_qgemm(int64_t m, int64_t n, int64_t k, const uint8_t* a, int32_t za, const int8_t* bt, int32_t* y,
                int threads) {
    std::vector<uint32_t> cs((size_t)n, 0);
    for (int64_t j = 0; j < n; ++j)
        for (int64_t q = 0; q < k; ++q) cs[j] += (uint32_t)(int32_t)bt[j * k + q];
    if (pick().vnni && m % 4 == 0 && n % 4 == 0) {
        par_run(m / 4, 1, threads, [&](int64_t ib, int) {
            const uint8_t* ar[4];
            for (int i = 0; i < 4; ++i) ar[i] = a + (ib * 4 + i) * k;
            for (int64_t jb = 0; jb < n / 4; ++jb) {
                const int8_t* br[4];
                for (int j = 0; j < 4; ++j) br[j] = bt + (jb * 4 + j) * k;
                uint32_t t[4][4];
                qdot4x4_vnni(ar, br, k, t);
                for (int i = 0; i < 4; ++i)
                    for (int j = 0; j < 4; ++j)
                        y[(ib * 4 + i) * n + jb * 4 + j] = (int32_t)(t[i][j] - (uint32_t)za * cs[jb * 4 + j]);
            }
        });
        return;
    }
    par_run(m, 1, threads, [&](int64_t i, int) {
        const uint8_t* ar = a + i * k;
        for (int64_t j = 0; j < n; ++j) {
            const int8_t* br = bt + j * k;
            __m256i acc = _mm256_setzero_si256();
            int64_t p = 0;
            for (; p + 16 <= k; p += 16) {
                const __m256i av = _mm256_cvtepu8_epi16(_mm_loadu_si128((const __m128i*)(ar + p)));
                const __m256i bv = _mm256_cvtepi8_epi16(_mm_loadu_si128((const __m128i*)(br + p)));
                acc = _mm256_add_epi32(acc, _mm256_madd_epi16(av, bv));
            }
            alignas(32) int32_t t[8];
            _mm256_store_si256((__m256i*)t, acc);
            uint32_t s = 0;
            for (int e = 0; e < 8; ++e) s += (uint32_t)t[e];
            for (; p < k; ++p) s += (uint32_t)((int32_t)ar[p] * (int32_t)br[p]);
            y[i * n + j] = (int32_t)(s - (uint32_t)za * cs[j]);
        }
    });
}

}  // extern "C"
