// fp32 GEMM on CDNA4 matrix cores for the three products of backpropagation.
//
// Replaces the reference's panel GEMM (src/StructuredDecisions.Base/Numerics/PackedMatrix.cs:109-428)
// and the transposes/copies LinearBackward wraps around it (Ops.cs:47-61): each layout reads its
// operands in place, so no packed or transposed copy of a weight or activation is ever made.
//
//   NT  C = A·Bᵀ   y  = x·Wᵀ      A k-contiguous, B k-contiguous
//   NN  C = A·B    dx = dy·W      A k-contiguous, B n-contiguous
//   TN  C = Aᵀ·B   dW += dyᵀ·x    A m-contiguous, B n-contiguous  (K = tokens, split-K)
//
// Block tile 128×128×32, 256 threads = 4 waves in 2×2, each wave 64×64 = 2×2 tiles of
// v_mfma_f32_32x32x2_f32. Operand tiles are staged through LDS in their global orientation
// (k-contiguous rows read as b128 fragments; mn-contiguous rows read as 4 conflict-free b32),
// double-buffered with a register prefetch of the next K tile. Split-K partials are reduced in a
// fixed order, so results never depend on timing.
#include "common.hpp"

namespace laya {
namespace {

constexpr int BM = 128, BN = 128, BK = 32, THREADS = 256;
constexpr int KPAD = BK + 4;   // row stride of a k-contiguous tile [mn][k]: b128 reads hit all 64 banks once
constexpr int MNPAD = BM + 8;  // row stride of an mn-contiguous tile [k][mn]: rows k and k+4 land 32 banks apart
constexpr int STAGE = BM * KPAD;  // ≥ BK * MNPAD

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

struct GemmParams {
    const float* A;
    const float* B;
    float* C;
    const float* bias;
    const float* R;
    long lda, ldb, ldc, ldr;
    int M, N, K;
    int tiles_m, tiles_n, splits, k_per_split;
    int mode;  // 0 store, 1 accumulate in place (one writer per element), 2 split-K partial
    int vec_a, vec_b;
};

// Loads one 128×32 operand tile into 4 float4 registers per thread (zero outside the matrix).
template <bool KCONTIG>
__device__ __forceinline__ void load_tile(const float* __restrict__ src, long ld, int mn0, int MN, int k0, int kend,
                                          bool vec, f32x4 (&reg)[4], int tid) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        int idx = tid + THREADS * i;
        if (KCONTIG) {
            int mn = mn0 + (idx >> 3);
            int k = k0 + ((idx & 7) << 2);
            if (vec && mn < MN && k + 3 < kend) {
                reg[i] = *reinterpret_cast<const f32x4*>(src + (long)mn * ld + k);
            } else {
#pragma unroll
                for (int e = 0; e < 4; ++e) reg[i][e] = (mn < MN && k + e < kend) ? src[(long)mn * ld + k + e] : 0.0f;
            }
        } else {
            int k = k0 + (idx >> 5);
            int mn = mn0 + ((idx & 31) << 2);
            if (vec && k < kend && mn + 3 < MN) {
                reg[i] = *reinterpret_cast<const f32x4*>(src + (long)k * ld + mn);
            } else {
#pragma unroll
                for (int e = 0; e < 4; ++e) reg[i][e] = (k < kend && mn + e < MN) ? src[(long)k * ld + mn + e] : 0.0f;
            }
        }
    }
}

template <bool KCONTIG>
__device__ __forceinline__ void store_tile(float* lds, const f32x4 (&reg)[4], int tid) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        int idx = tid + THREADS * i;
        if (KCONTIG)
            *reinterpret_cast<f32x4*>(lds + (idx >> 3) * KPAD + ((idx & 7) << 2)) = reg[i];
        else
            *reinterpret_cast<f32x4*>(lds + (idx >> 5) * MNPAD + ((idx & 31) << 2)) = reg[i];
    }
}

// The 4 consecutive-k values lane (mn, k..k+3) contributes to 4 successive MFMAs.
template <bool KCONTIG>
__device__ __forceinline__ f32x4 read_frag(const float* lds, int mn, int k) {
    if (KCONTIG) return *reinterpret_cast<const f32x4*>(lds + mn * KPAD + k);
    return f32x4{lds[k * MNPAD + mn], lds[(k + 1) * MNPAD + mn], lds[(k + 2) * MNPAD + mn], lds[(k + 3) * MNPAD + mn]};
}

template <bool AK, bool BKC>
__global__ __launch_bounds__(THREADS, 2) void gemm_kernel(GemmParams p) {
    __shared__ __attribute__((aligned(16))) float smem[2][2][STAGE];

    // XCD-aware order: workgroups are dealt round-robin to the 8 XCDs, so give each XCD a contiguous
    // run of logical tiles (n fastest); tiles sharing an A row-panel then share one XCD's L2.
    const int nblocks = gridDim.x, bid = blockIdx.x;
    const int xcd = bid & 7, local = bid >> 3, per = nblocks >> 3, rem = nblocks & 7;
    const int logical = (xcd < rem ? xcd * (per + 1) : rem * (per + 1) + (xcd - rem) * per) + local;
    const int tiles = p.tiles_m * p.tiles_n;
    const int split = logical / tiles, t = logical - split * tiles;
    const int tile_m = t / p.tiles_n, tile_n = t - tile_m * p.tiles_n;
    const int m0 = tile_m * BM, n0 = tile_n * BN;
    const int kb = split * p.k_per_split;
    const int ke = min(p.K, kb + p.k_per_split);
    const int nk = ke > kb ? (ke - kb + BK - 1) / BK : 0;

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    const int lr = lane & 31, kh = (lane >> 5) << 2;

    f32x16 acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) acc[i][j] = f32x16{};

    f32x4 ra[4], rb[4];
    if (nk > 0) {
        load_tile<AK>(p.A, p.lda, m0, p.M, kb, ke, p.vec_a, ra, tid);
        load_tile<BKC>(p.B, p.ldb, n0, p.N, kb, ke, p.vec_b, rb, tid);
        store_tile<AK>(smem[0][0], ra, tid);
        store_tile<BKC>(smem[0][1], rb, tid);
    }
    __syncthreads();

    for (int kt = 0; kt < nk; ++kt) {
        const int cur = kt & 1;
        if (kt + 1 < nk) {
            const int k0 = kb + (kt + 1) * BK;
            load_tile<AK>(p.A, p.lda, m0, p.M, k0, ke, p.vec_a, ra, tid);
            load_tile<BKC>(p.B, p.ldb, n0, p.N, k0, ke, p.vec_b, rb, tid);
        }
        const float* As = smem[cur][0];
        const float* Bs = smem[cur][1];
#pragma unroll
        for (int kk = 0; kk < BK; kk += 8) {
            const int k = kk + kh;
            f32x4 a0 = read_frag<AK>(As, wm * 64 + lr, k);
            f32x4 a1 = read_frag<AK>(As, wm * 64 + 32 + lr, k);
            f32x4 b0 = read_frag<BKC>(Bs, wn * 64 + lr, k);
            f32x4 b1 = read_frag<BKC>(Bs, wn * 64 + 32 + lr, k);
#pragma unroll
            for (int c = 0; c < 4; ++c) {
                acc[0][0] = __builtin_amdgcn_mfma_f32_32x32x2f32(a0[c], b0[c], acc[0][0], 0, 0, 0);
                acc[0][1] = __builtin_amdgcn_mfma_f32_32x32x2f32(a0[c], b1[c], acc[0][1], 0, 0, 0);
                acc[1][0] = __builtin_amdgcn_mfma_f32_32x32x2f32(a1[c], b0[c], acc[1][0], 0, 0, 0);
                acc[1][1] = __builtin_amdgcn_mfma_f32_32x32x2f32(a1[c], b1[c], acc[1][1], 0, 0, 0);
            }
        }
        if (kt + 1 < nk) {
            store_tile<AK>(smem[cur ^ 1][0], ra, tid);
            store_tile<BKC>(smem[cur ^ 1][1], rb, tid);
        }
        __syncthreads();
    }

    // Accumulator layout of a 32×32 tile: lane holds column lane%32, rows 8(r/4) + 4(lane/32) + r%4.
#pragma unroll
    for (int i = 0; i < 2; ++i) {
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const int n = n0 + wn * 64 + j * 32 + lr;
            if (n >= p.N) continue;
            const float bn = (p.mode == 0 && p.bias) ? p.bias[n] : 0.0f;
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int m = m0 + wm * 64 + i * 32 + 8 * (r >> 2) + kh + (r & 3);
                if (m >= p.M) continue;
                float v = acc[i][j][r];
                if (p.mode == 0) {
                    v += bn;
                    if (p.R) v += p.R[(long)m * p.ldr + n];
                    p.C[(long)m * p.ldc + n] = v;
                } else if (p.mode == 1) {
                    p.C[(long)m * p.ldc + n] += v;
                } else {
                    p.C[(long)split * p.M * p.N + (long)m * p.N + n] = v;
                }
            }
        }
    }
}

// C[m, n] += Σ_s P[s][m][n], s in order.
__global__ void splitk_reduce_kernel(const float* __restrict__ P, int splits, int M, int N, float* C, long ldc) {
    const long total = (long)M * N;
    for (long i = blockIdx.x * (long)blockDim.x + threadIdx.x; i < total; i += (long)gridDim.x * blockDim.x) {
        float s = 0.0f;
        for (int k = 0; k < splits; ++k) s += P[(long)k * total + i];
        const long m = i / N, n = i - m * N;
        C[m * ldc + n] += s;
    }
}

__global__ void column_sum_kernel(const float* __restrict__ x, int rows, int n, float* out) {
    // One thread per column; rows summed in order (bias gradients are small: n ≤ a few thousand).
    const int c = blockIdx.x * blockDim.x + threadIdx.x;
    if (c >= n) return;
    float s = 0.0f;
    for (int r = 0; r < rows; ++r) s += x[(long)r * n + c];
    out[c] += s;
}

__global__ void column_partial_kernel(const float* __restrict__ x, int rows, int n, int rows_per, float* part) {
    const int c = blockIdx.x * blockDim.x + threadIdx.x;
    const int chunk = blockIdx.y;
    if (c >= n) return;
    const int r0 = chunk * rows_per, r1 = min(rows, r0 + rows_per);
    float s = 0.0f;
    for (int r = r0; r < r1; ++r) s += x[(long)r * n + c];
    part[(long)chunk * n + c] = s;
}

__global__ void column_reduce_kernel(const float* __restrict__ part, int chunks, int n, float* out) {
    const int c = blockIdx.x * blockDim.x + threadIdx.x;
    if (c >= n) return;
    float s = 0.0f;
    for (int k = 0; k < chunks; ++k) s += part[(long)k * n + c];
    out[c] += s;
}

template <bool AK, bool BKC> void launch(laya_ctx* ctx, const GemmParams& p, int blocks) {
    hipLaunchKernelGGL((gemm_kernel<AK, BKC>), dim3(blocks), dim3(THREADS), 0, ctx->stream, p);
    check_launch("gemm_kernel");
}

inline bool aligned16(const void* ptr) { return ((uintptr_t)ptr & 15u) == 0; }

}  // namespace

void gemm(laya_ctx* ctx, GemmLayout layout, GemmEpilogue ep, int M, int N, int K, const float* A, long lda,
          const float* B, long ldb, float* C, long ldc, const float* bias, const float* R, long ldr) {
    LAYA_REQUIRE(M >= 0 && N >= 0 && K >= 0, "gemm: negative size");
    if (M == 0 || N == 0) return;
    GemmParams p{};
    p.A = A;
    p.B = B;
    p.C = C;
    p.bias = bias;
    p.R = R;
    p.lda = lda;
    p.ldb = ldb;
    p.ldc = ldc;
    p.ldr = ldr;
    p.M = M;
    p.N = N;
    p.K = K;
    p.tiles_m = (M + BM - 1) / BM;
    p.tiles_n = (N + BN - 1) / BN;
    p.vec_a = (lda % 4 == 0) && aligned16(A);
    p.vec_b = (ldb % 4 == 0) && aligned16(B);
    const int tiles = p.tiles_m * p.tiles_n;

    int splits = 1;
    if (ep == GemmEpilogue::Accumulate) {
        // Fill the chip: aim for ≥ 2 workgroups per CU, but keep ≥ 512 of K per split.
        const int want = (2 * ctx->cu_count + tiles - 1) / tiles;
        const int max_by_k = std::max(1, K / 512);
        splits = std::max(1, std::min(want, max_by_k));
    }
    int kps = (K + splits - 1) / splits;
    kps = (kps + BK - 1) / BK * BK;
    if (kps == 0) kps = BK;
    splits = std::max(1, (K + kps - 1) / kps);
    p.splits = splits;
    p.k_per_split = kps;

    float* partial = nullptr;
    if (ep == GemmEpilogue::Store) {
        p.mode = 0;
    } else if (splits == 1) {
        p.mode = 1;
    } else {
        p.mode = 2;
        partial = static_cast<float*>(ctx->workspace(0, sizeof(float) * (size_t)splits * M * N));
        p.C = partial;
    }
    const int blocks = tiles * splits;
    {
        static const char* names[3] = {"gemm_nt", "gemm_nn", "gemm_tn"};
        ProfileScope scope(ctx, names[(int)layout], 2.0 * M * N * (double)K, 0.0);
        switch (layout) {
            case GemmLayout::NT: launch<true, true>(ctx, p, blocks); break;
            case GemmLayout::NN: launch<true, false>(ctx, p, blocks); break;
            case GemmLayout::TN: launch<false, false>(ctx, p, blocks); break;
        }
    }
    if (p.mode == 2) {
        const long total = (long)M * N;
        ProfileScope scope(ctx, "gemm_splitk_reduce", 0.0, 4.0 * total * (splits + 2));
        hipLaunchKernelGGL(splitk_reduce_kernel, dim3(blocks_for(total, 256, 4096)), dim3(256), 0, ctx->stream,
                           partial, splits, M, N, C, ldc);
        check_launch("splitk_reduce_kernel");
    }
}

void column_sum_add(laya_ctx* ctx, const float* x, int rows, int n, float* out) {
    if (rows <= 0 || n <= 0) return;
    const int rows_per = 256;
    const int chunks = (rows + rows_per - 1) / rows_per;
    if (chunks <= 1) {
        hipLaunchKernelGGL(column_sum_kernel, dim3((n + 255) / 256), dim3(256), 0, ctx->stream, x, rows, n, out);
        check_launch("column_sum_kernel");
        return;
    }
    float* part = static_cast<float*>(ctx->workspace(1, sizeof(float) * (size_t)chunks * n));
    hipLaunchKernelGGL(column_partial_kernel, dim3((n + 255) / 256, chunks), dim3(256), 0, ctx->stream, x, rows, n,
                       rows_per, part);
    check_launch("column_partial_kernel");
    hipLaunchKernelGGL(column_reduce_kernel, dim3((n + 255) / 256), dim3(256), 0, ctx->stream, part, chunks, n, out);
    check_launch("column_reduce_kernel");
}

}  // namespace laya
