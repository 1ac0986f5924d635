// Oracle (test infrastructure only; never linked into the product library).
//
// The dense product every Linear / LinearBackward of the oracle runs on. It restates the
// semantics of the reference's panel GEMM (src/StructuredDecisions.Base/Numerics/PackedMatrix.cs:109-162:
// y = x·Wᵀ, with the same kernel reused for dX and dW through FromInputMajor packing,
// src/StructuredDecisions.Laya.Training/Ops.cs:33-62) as a register-tiled, cache-blocked CPU GEMM:
// C[m, n] (+)= Σ_k A(m, k) · B(k, n) with arbitrary element strides for A and B, so the three
// backprop layouts need no transposed copies. Summation order inside a dot product differs from
// the reference's (any exact fp32 GEMM is acceptable there; parity is at tolerance level).
//
// Compiled with -ffp-contract=fast so the micro-kernel uses FMA, as the reference GEMM does.
#include <immintrin.h>

#include <algorithm>
#include <cstdint>
#include <cstring>
#include <type_traits>
#include <vector>
#include <omp.h>

namespace oracle {

template <typename R> struct VecTraits;
template <> struct VecTraits<float> {
    typedef float V __attribute__((vector_size(32), aligned(4)));
    static constexpr int W = 8;
};
template <> struct VecTraits<double> {
    typedef double V __attribute__((vector_size(32), aligned(8)));
    static constexpr int W = 4;
};

// 6 × (2 vectors) register tile with AVX2 FMA: 12 named accumulators stay in ymm registers.
#define OGEMM_MICRO(NAME, R, V, LOAD, STORE, BCAST, FMA, ZERO, ADD, W)                                        \
    static inline void NAME(int kc, const R* __restrict ap, const R* __restrict bp, R* c, long ldc, int mr,    \
                            int nr) {                                                                        \
        V c00 = ZERO(), c01 = ZERO(), c10 = ZERO(), c11 = ZERO(), c20 = ZERO(), c21 = ZERO();                 \
        V c30 = ZERO(), c31 = ZERO(), c40 = ZERO(), c41 = ZERO(), c50 = ZERO(), c51 = ZERO();                 \
        for (int k = 0; k < kc; ++k) {                                                                        \
            const R* b = bp + (long)k * 2 * W;                                                                \
            const R* a = ap + (long)k * 6;                                                                    \
            const V b0 = LOAD(b), b1 = LOAD(b + W);                                                           \
            V x = BCAST(a + 0);                                                                               \
            c00 = FMA(x, b0, c00);                                                                            \
            c01 = FMA(x, b1, c01);                                                                            \
            x = BCAST(a + 1);                                                                                 \
            c10 = FMA(x, b0, c10);                                                                            \
            c11 = FMA(x, b1, c11);                                                                            \
            x = BCAST(a + 2);                                                                                 \
            c20 = FMA(x, b0, c20);                                                                            \
            c21 = FMA(x, b1, c21);                                                                            \
            x = BCAST(a + 3);                                                                                 \
            c30 = FMA(x, b0, c30);                                                                            \
            c31 = FMA(x, b1, c31);                                                                            \
            x = BCAST(a + 4);                                                                                 \
            c40 = FMA(x, b0, c40);                                                                            \
            c41 = FMA(x, b1, c41);                                                                            \
            x = BCAST(a + 5);                                                                                 \
            c50 = FMA(x, b0, c50);                                                                            \
            c51 = FMA(x, b1, c51);                                                                            \
        }                                                                                                     \
        V acc[12] = {c00, c01, c10, c11, c20, c21, c30, c31, c40, c41, c50, c51};                             \
        if (mr == 6 && nr == 2 * W) {                                                                         \
            for (int i = 0; i < 6; ++i) {                                                                     \
                STORE(c + i * ldc, ADD(LOAD(c + i * ldc), acc[2 * i]));                                       \
                STORE(c + i * ldc + W, ADD(LOAD(c + i * ldc + W), acc[2 * i + 1]));                           \
            }                                                                                                 \
        } else {                                                                                              \
            for (int i = 0; i < mr; ++i) {                                                                    \
                R tmp[2 * W];                                                                                 \
                STORE(tmp, acc[2 * i]);                                                                       \
                STORE(tmp + W, acc[2 * i + 1]);                                                               \
                for (int j = 0; j < nr; ++j) c[i * ldc + j] += tmp[j];                                        \
            }                                                                                                 \
        }                                                                                                     \
    }

OGEMM_MICRO(micro_f32, float, __m256, _mm256_loadu_ps, _mm256_storeu_ps, _mm256_broadcast_ss, _mm256_fmadd_ps,
            _mm256_setzero_ps, _mm256_add_ps, 8)
OGEMM_MICRO(micro_f64, double, __m256d, _mm256_loadu_pd, _mm256_storeu_pd, _mm256_broadcast_sd, _mm256_fmadd_pd,
            _mm256_setzero_pd, _mm256_add_pd, 4)

template <typename R>
static inline void micro_kernel(int kc, const R* ap, const R* bp, R* c, long ldc, int mr, int nr) {
    if constexpr (std::is_same<R, float>::value)
        micro_f32(kc, ap, bp, c, ldc, mr, nr);
    else
        micro_f64(kc, ap, bp, c, ldc, mr, nr);
}

// C[m*ldc + n] = (accumulate ? C : 0) + Σ_k A[m*sam + k*sak] · B[k*sbk + n*sbn]
template <typename R>
void gemm(int M, int N, int K, const R* A, long sam, long sak, const R* B, long sbk, long sbn, R* C, long ldc,
          bool accumulate) {
    using T = VecTraits<R>;
    constexpr int W = T::W, NR = 2 * W, MR = 6, KC = 256, MC = 48;
    if (M <= 0 || N <= 0) return;
    if (!accumulate) {
#pragma omp parallel for schedule(static)
        for (int m = 0; m < M; ++m) std::memset(C + (long)m * ldc, 0, sizeof(R) * N);
    }
    if (K <= 0) return;
    const int panels = (N + NR - 1) / NR;
    std::vector<R> bpack((size_t)panels * NR * KC);
    const int mblocks = (M + MC - 1) / MC;
    for (int k0 = 0; k0 < K; k0 += KC) {
        const int kc = std::min(KC, K - k0);
#pragma omp parallel for schedule(static)
        for (int p = 0; p < panels; ++p) {
            R* dst = bpack.data() + (size_t)p * kc * NR;
            for (int kk = 0; kk < kc; ++kk) {
                for (int j = 0; j < NR; ++j) {
                    int n = p * NR + j;
                    dst[kk * NR + j] = n < N ? B[(long)(k0 + kk) * sbk + (long)n * sbn] : R(0);
                }
            }
        }
#pragma omp parallel
        {
            std::vector<R> apack((size_t)MC * KC);
#pragma omp for schedule(dynamic, 1)
            for (int mb = 0; mb < mblocks; ++mb) {
                const int m0 = mb * MC;
                const int mc = std::min(MC, M - m0);
                const int micro = (mc + MR - 1) / MR;
                for (int u = 0; u < micro; ++u) {
                    R* dst = apack.data() + (size_t)u * kc * MR;
                    for (int kk = 0; kk < kc; ++kk) {
                        for (int i = 0; i < MR; ++i) {
                            int m = m0 + u * MR + i;
                            dst[kk * MR + i] = m < M ? A[(long)m * sam + (long)(k0 + kk) * sak] : R(0);
                        }
                    }
                }
                for (int p = 0; p < panels; ++p) {
                    const R* bp = bpack.data() + (size_t)p * kc * NR;
                    const int nr = std::min(NR, N - p * NR);
                    for (int u = 0; u < micro; ++u) {
                        const int mr = std::min(MR, mc - u * MR);
                        micro_kernel<R>(kc, apack.data() + (size_t)u * kc * MR, bp,
                                        C + (long)(m0 + u * MR) * ldc + p * NR, ldc, mr, nr);
                    }
                }
            }
        }
    }
}

template void gemm<float>(int, int, int, const float*, long, long, const float*, long, long, float*, long, bool);
template void gemm<double>(int, int, int, const double*, long, long, const double*, long, long, double*, long, bool);

}  // namespace oracle
