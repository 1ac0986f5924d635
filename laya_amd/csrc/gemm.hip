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

// XCD-aware order: workgroups are dealt round-robin to the 8 XCDs, so give each XCD a contiguous run
// of logical tiles (n fastest); tiles sharing an A row-panel then share one XCD's L2.
__device__ __forceinline__ int xcd_logical_block() {
    const int nblocks = gridDim.x, bid = blockIdx.x;
    const int xcd = bid & 7, local = bid >> 3, per = nblocks >> 3, rem = nblocks & 7;
    return (xcd < rem ? xcd * (per + 1) : rem * (per + 1) + (xcd - rem) * per) + local;
}

// One 128×128 output tile (or one split-K slice of it) of C = op(A)·op(B).
template <bool AK, bool BKC>
__device__ __forceinline__ void gemm_tile(const GemmParams& p, int logical, float (*smem)[2][STAGE]) {
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

template <bool AK, bool BKC>
__global__ __launch_bounds__(THREADS, 2) void gemm_kernel(GemmParams p) {
    __shared__ __attribute__((aligned(16))) float smem[2][2][STAGE];
    gemm_tile<AK, BKC>(p, xcd_logical_block(), smem);
}

// dX = dY·W (NN) and dW += dYᵀ·X (TN, split-K partials) in one grid: the first `blocks0` logical
// blocks are dX tiles, the rest dW slices. The two products are independent, and one grid lets their
// tiles fill the CUs together instead of each leaving a partial last wave.
__global__ __launch_bounds__(THREADS, 2) void gemm_pair_kernel(GemmParams nn, GemmParams tn, int blocks0) {
    __shared__ __attribute__((aligned(16))) float smem[2][2][STAGE];
    const int logical = xcd_logical_block();
    if (logical < blocks0)
        gemm_tile<true, false>(nn, logical, smem);
    else
        gemm_tile<false, false>(tn, logical - blocks0, smem);
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

GemmParams make_params(int M, int N, int K, const float* A, long lda, const float* B, long ldb, float* C, long ldc,
                       const float* bias, const float* R, long ldr) {
    LAYA_REQUIRE(M >= 0 && N >= 0 && K >= 0, "gemm: negative size");
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
    p.splits = 1;
    p.k_per_split = std::max(BK, (K + BK - 1) / BK * BK);
    return p;
}

// Splits K into `splits` slices of a multiple of BK; returns the realised split count.
int set_splits(GemmParams& p, int splits) {
    int kps = (p.K + splits - 1) / splits;
    kps = std::max(BK, (kps + BK - 1) / BK * BK);
    p.k_per_split = kps;
    p.splits = std::max(1, (p.K + kps - 1) / kps);
    return p.splits;
}

// An accumulating product: one writer per element (mode 1), or split-K partials into workspace slot 0
// (mode 2) to be reduced by finish_accumulate.
float* prepare_accumulate(laya_ctx* ctx, GemmParams& p) {
    if (p.splits == 1) {
        p.mode = 1;
        return nullptr;
    }
    p.mode = 2;
    float* partial = static_cast<float*>(ctx->workspace(0, sizeof(float) * (size_t)p.splits * p.M * p.N));
    float* out = p.C;
    p.C = partial;
    return out;
}

void finish_accumulate(laya_ctx* ctx, const GemmParams& p, float* out, long ldc) {
    if (p.mode != 2) return;
    const long total = (long)p.M * p.N;
    ProfileScope scope(ctx, "gemm_splitk_reduce", 0.0, 4.0 * total * (p.splits + 2));
    hipLaunchKernelGGL(splitk_reduce_kernel, dim3(blocks_for(total, 256, 4096)), dim3(256), 0, ctx->stream, p.C,
                       p.splits, p.M, p.N, out, ldc);
    check_launch("splitk_reduce_kernel");
}

}  // namespace

void gemm(laya_ctx* ctx, GemmLayout layout, GemmEpilogue ep, int M, int N, int K, const float* A, long lda,
          const float* B, long ldb, float* C, long ldc, const float* bias, const float* R, long ldr) {
    if (M == 0 || N == 0) return;
    GemmParams p = make_params(M, N, K, A, lda, B, ldb, C, ldc, bias, R, ldr);
    const int tiles = p.tiles_m * p.tiles_n;
    float* out = C;
    if (ep == GemmEpilogue::Accumulate) {
        // Fill the chip: aim for ≥ 2 workgroups per CU, but keep ≥ 512 of K per split.
        const int want = (2 * ctx->cu_count + tiles - 1) / tiles;
        set_splits(p, std::max(1, std::min(want, std::max(1, K / 512))));
        out = prepare_accumulate(ctx, p);
    } else {
        p.mode = 0;
    }
    const int blocks = tiles * p.splits;
    {
        static const char* names[3] = {"gemm_nt", "gemm_nn", "gemm_tn"};
        ProfileScope scope(ctx, names[(int)layout], 2.0 * M * N * (double)K, 0.0);
        switch (layout) {
            case GemmLayout::NT: launch<true, true>(ctx, p, blocks); break;
            case GemmLayout::NN: launch<true, false>(ctx, p, blocks); break;
            case GemmLayout::TN: launch<false, false>(ctx, p, blocks); break;
        }
    }
    finish_accumulate(ctx, p, out, ldc);
}

void gemm_backward_pair(laya_ctx* ctx, int rows, int in, int out, const float* dy, const float* W, const float* x,
                        float* dx, const float* dx_residual, float* dW) {
    if (rows == 0) return;
    // dx[rows, in] = dy[rows, out] · W[out, in]       (NN, K = out)
    GemmParams nn = make_params(rows, in, out, dy, out, W, in, dx, in, nullptr, dx_residual, in);
    nn.mode = 0;
    // dW[out, in] += dy[rows, out]ᵀ · x[rows, in]     (TN, K = rows)
    GemmParams tn = make_params(out, in, rows, dy, out, x, in, dW, in, nullptr, nullptr, 0);
    const int n0 = nn.tiles_m * nn.tiles_n, n1 = tn.tiles_m * tn.tiles_n;
    // Choose the dW split so its slices are as long as a dX tile's K loop, then minimise the rounds of
    // 2-blocks-per-CU the combined grid needs times the longest block.
    const long slots = 2L * ctx->cu_count;
    const long knn = std::max(BK, (out + BK - 1) / BK * BK);
    int best_s = 1;
    double best = 1e300;
    for (int s = 1; s <= 64; ++s) {
        GemmParams t = tn;
        const int real = set_splits(t, s);
        if (real != s) continue;
        const long total = n0 + (long)n1 * s;
        // Rounds × the longest block's K, plus the split-K reduce traffic in the same K units (a round
        // of two 128×128 blocks per CU costs ≈ 1.2e-7 s per unit of K; the reduce moves 4·out·in·s bytes).
        const double est = (double)((total + slots - 1) / slots) * std::max<long>(knn, t.k_per_split) +
                           6.8e-6 * s * (double)out * in;
        if (est < best) {
            best = est;
            best_s = s;
        }
    }
    set_splits(tn, best_s);
    float* dW_out = prepare_accumulate(ctx, tn);
    const int blocks = n0 + n1 * tn.splits;
    {
        ProfileScope scope(ctx, "gemm_bwd_pair", 2.0 * 2.0 * rows * (double)in * out, 0.0);
        hipLaunchKernelGGL(gemm_pair_kernel, dim3(blocks), dim3(THREADS), 0, ctx->stream, nn, tn, n0);
        check_launch("gemm_pair_kernel");
    }
    finish_accumulate(ctx, tn, dW_out, in);
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
