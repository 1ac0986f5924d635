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
#include <algorithm>
#include <cstdint>
#include <cstring>
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

template <typename R>
static inline void micro_kernel(int kc, const R* __restrict ap, const R* __restrict bp, R* c, long ldc, int mr, int nr) {
    using T = VecTraits<R>;
    using V = typename T::V;
    constexpr int W = T::W, NR = 2 * W, MR = 6;
    V acc[MR][2];
    for (int i = 0; i < MR; ++i) acc[i][0] = acc[i][1] = V{} ;
    for (int k = 0; k < kc; ++k) {
        V b0, b1;
        std::memcpy(&b0, bp + (long)k * NR, sizeof(V));
        std::memcpy(&b1, bp + (long)k * NR + W, sizeof(V));
        const R* a = ap + (long)k * MR;
        for (int i = 0; i < MR; ++i) {
            V av = V{} + a[i];
            acc[i][0] += av * b0;
            acc[i][1] += av * b1;
        }
    }
    if (mr == MR && nr == NR) {
        for (int i = 0; i < MR; ++i) {
            V c0, c1;
            std::memcpy(&c0, c + i * ldc, sizeof(V));
            std::memcpy(&c1, c + i * ldc + W, sizeof(V));
            c0 += acc[i][0];
            c1 += acc[i][1];
            std::memcpy(c + i * ldc, &c0, sizeof(V));
            std::memcpy(c + i * ldc + W, &c1, sizeof(V));
        }
    } else {
        for (int i = 0; i < mr; ++i) {
            R tmp[2 * W];
            std::memcpy(tmp, &acc[i][0], sizeof(V));
            std::memcpy(tmp + W, &acc[i][1], sizeof(V));
            for (int j = 0; j < nr; ++j) c[i * ldc + j] += tmp[j];
        }
    }
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
