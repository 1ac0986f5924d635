// Memory-bound kernels of the step: activations, dropout, residual adds, row gathers/scatters,
// embedding and type-embedding gradients, the decision-head cross-entropy gradient, and synthetic
// initialisation. All are coalesced float4 streams where the shape allows; every reduction over
// rows runs in a fixed order.
#include "elementwise.hpp"

namespace laya {
namespace {

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ f32x4 ld4(const float* p) { return *reinterpret_cast<const f32x4*>(p); }
__device__ __forceinline__ void st4(float* p, f32x4 v) { *reinterpret_cast<f32x4*>(p) = v; }

#define GRID_STRIDE(i, n) for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < (n); i += (size_t)gridDim.x * blockDim.x)

__global__ void fill_kernel(float* dst, float v, size_t n) {
    GRID_STRIDE(i, n) dst[i] = v;
}

__global__ void add_kernel(float* dst, const float* src, size_t n) {
    GRID_STRIDE(i, n) dst[i] += src[i];
}

__global__ void scale_kernel(float* dst, float s, size_t n) {
    GRID_STRIDE(i, n) dst[i] *= s;
}

__global__ void fill4_kernel(f32x4* dst, float v, size_t n4) {
    GRID_STRIDE(i, n4) dst[i] = f32x4{v, v, v, v};
}

__global__ void add4_kernel(f32x4* dst, const f32x4* src, size_t n4) {
    GRID_STRIDE(i, n4) dst[i] += src[i];
}

__global__ void gelu_fwd_kernel(const float* x, size_t n, float* y) {
    GRID_STRIDE(i, n) y[i] = gelu_f(x[i]);
}

__global__ void gelu_bwd_kernel(const float* u, float* g, size_t n) {
    GRID_STRIDE(i, n) g[i] *= gelu_grad_f(u[i]);
}

// GeGLU, 4 columns per thread: act[t, i] = gelu(wide[t, i]) · wide[t, I + i].
// amax (optional): max|act| folded in (the output's magnitude word).
__global__ void geglu_fwd_kernel(const float* __restrict__ wide, int rows, int inter, float* __restrict__ act,
                                 __bf16* __restrict__ act16, unsigned* amax) {
    const int q = inter >> 2;
    const size_t n = (size_t)rows * q;
    unsigned m = 0;
    GRID_STRIDE(i, n) {
        const size_t t = i / q;
        const int c = (int)(i - t * q) * 4;
        const float* w = wide + t * 2 * inter;
        const f32x4 x = ld4(w + c), g = ld4(w + inter + c);
        const f32x4 o = {gelu_f(x[0]) * g[0], gelu_f(x[1]) * g[1], gelu_f(x[2]) * g[2], gelu_f(x[3]) * g[3]};
        st4(act + t * inter + c, o);
        if (act16) *reinterpret_cast<bf16x4*>(act16 + t * inter + c) = __builtin_convertvector(o, bf16x4);
        m = max(m, amax_bits4(o));
    }
    block_amax_fold(m, amax);
}

// dwide[t] = [dact·gate·gelu'(input) | dact·gelu(input)] (TrainableDecisionModel.cs:573-578).
// amax (optional): max|dwide| folded in.
__global__ void geglu_bwd_kernel(const float* __restrict__ wide, const float* __restrict__ dact, int rows, int inter,
                                 float* __restrict__ dwide, unsigned* amax) {
    const int q = inter >> 2;
    const size_t n = (size_t)rows * q;
    unsigned m = 0;
    GRID_STRIDE(i, n) {
        const size_t t = i / q;
        const int c = (int)(i - t * q) * 4;
        const float* w = wide + t * 2 * inter;
        const f32x4 x = ld4(w + c), g = ld4(w + inter + c), up = ld4(dact + t * inter + c);
        f32x4 di, dg;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            dg[e] = gelu_f(x[e]) * up[e];
            di[e] = up[e] * g[e] * gelu_grad_f(x[e]);
        }
        st4(dwide + t * 2 * inter + c, di);
        st4(dwide + t * 2 * inter + inter + c, dg);
        m = max(m, max(amax_bits4(di), amax_bits4(dg)));
    }
    block_amax_fold(m, amax);
}

__global__ void geglu_fwd_scalar_kernel(const float* wide, int rows, int inter, float* act) {
    const size_t n = (size_t)rows * inter;
    GRID_STRIDE(i, n) {
        const size_t t = i / inter, c = i - t * inter;
        act[i] = gelu_f(wide[t * 2 * inter + c]) * wide[t * 2 * inter + inter + c];
    }
}

__global__ void geglu_bwd_scalar_kernel(const float* wide, const float* dact, int rows, int inter, float* dwide) {
    const size_t n = (size_t)rows * inter;
    GRID_STRIDE(i, n) {
        const size_t t = i / inter, c = i - t * inter;
        const float x = wide[t * 2 * inter + c], g = wide[t * 2 * inter + inter + c], up = dact[i];
        dwide[t * 2 * inter + inter + c] = gelu_f(x) * up;
        dwide[t * 2 * inter + c] = up * g * gelu_grad_f(x);
    }
}

// Ops.Dropout (Ops.cs:244-258): element i is dropped when Uniform(seed, i) < p.
__global__ void dropout_kernel(float* v, size_t n, float p, float keep, uint64_t seed) {
    GRID_STRIDE(i, n) v[i] = uniform01(seed, i) < p ? 0.0f : v[i] * keep;
}

__global__ void relu_dropout_fwd_kernel(const float* wide, size_t n, float p, float keep, uint64_t seed,
                                        float* dropped) {
    GRID_STRIDE(i, n) {
        const float r = fmaxf(wide[i], 0.0f);
        dropped[i] = (p > 0.0f && uniform01(seed, i) < p) ? 0.0f : (p > 0.0f ? r * keep : r);
    }
}

__global__ void relu_dropout_bwd_kernel(const float* wide, float* g, size_t n, float p, float keep, uint64_t seed) {
    GRID_STRIDE(i, n) {
        float v = g[i];
        if (p > 0.0f) v = uniform01(seed, i) < p ? 0.0f : v * keep;
        g[i] = wide[i] <= 0.0f ? 0.0f : v;
    }
}

// Four elements per thread; the mask of element i is still Uniform(seed, i) < p.
__global__ void dropout4_kernel(f32x4* v, size_t n4, float p, float keep, uint64_t seed) {
    GRID_STRIDE(i, n4) {
        f32x4 x = v[i];
#pragma unroll
        for (int e = 0; e < 4; ++e) x[e] = uniform01(seed, 4 * i + e) < p ? 0.0f : x[e] * keep;
        v[i] = x;
    }
}

// v = Dropout(v) + r in one pass (the same two operations as dropout4_kernel then add4_kernel).
__global__ void dropout_add4_kernel(f32x4* v, const f32x4* r, size_t n4, float p, float keep, uint64_t seed) {
    GRID_STRIDE(i, n4) {
        f32x4 x = v[i];
        const f32x4 y = r[i];
#pragma unroll
        for (int e = 0; e < 4; ++e) x[e] = uniform01(seed, 4 * i + e) < p ? 0.0f : x[e] * keep;
        v[i] = x + y;
    }
}

__global__ void dropout_copy4_kernel(const f32x4* src, f32x4* dst, size_t n4, float p, float keep, uint64_t seed) {
    GRID_STRIDE(i, n4) {
        f32x4 x = src[i];
#pragma unroll
        for (int e = 0; e < 4; ++e) x[e] = uniform01(seed, 4 * i + e) < p ? 0.0f : x[e] * keep;
        dst[i] = x;
    }
}

// amax (optional): max|dropped| folded in (its magnitude word).
__global__ void relu_dropout_fwd4_kernel(const f32x4* wide, size_t n4, float p, float keep, uint64_t seed,
                                         f32x4* dropped, bf16x4* dropped16, unsigned* amax) {
    unsigned m = 0;
    GRID_STRIDE(i, n4) {
        const f32x4 w = wide[i];
        f32x4 o;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const float r = fmaxf(w[e], 0.0f);
            o[e] = (p > 0.0f && uniform01(seed, 4 * i + e) < p) ? 0.0f : (p > 0.0f ? r * keep : r);
        }
        dropped[i] = o;
        if (dropped16) dropped16[i] = __builtin_convertvector(o, bf16x4);
        m = max(m, amax_bits4(o));
    }
    block_amax_fold(m, amax);
}

// dst = bf16(src), nearest even: the bf16 copies of weights and activations the bf16 products read.
__global__ void to_bf16_kernel(const f32x4* __restrict__ src, bf16x4* __restrict__ dst, size_t n4) {
    GRID_STRIDE(i, n4) dst[i] = __builtin_convertvector(src[i], bf16x4);
}
__global__ void to_bf16_scalar_kernel(const float* __restrict__ src, __bf16* __restrict__ dst, size_t n) {
    GRID_STRIDE(i, n) dst[i] = (__bf16)src[i];
}
// dst = float(bf16(src)), rounded to nearest even: the bf16 value widened back to fp32 (exact).
__global__ void round_bf16_kernel(const f32x4* __restrict__ src, f32x4* __restrict__ dst, size_t n4) {
    GRID_STRIDE(i, n4) dst[i] = __builtin_convertvector(__builtin_convertvector(src[i], bf16x4), f32x4);
}
__global__ void round_bf16_scalar_kernel(const float* __restrict__ src, float* __restrict__ dst, size_t n) {
    GRID_STRIDE(i, n) dst[i] = (float)(__bf16)src[i];
}

// The backward from the forward's output: an element passes its gradient (times 1/(1 − p)) exactly when
// it was kept and its pre-activation was positive, i.e. when its output is positive. Same product as
// recomputing the mask from the pre-activation, without the per-element hash.
// amax (optional): max|g| (after) folded in (its magnitude word).
__global__ void relu_dropout_bwd_out4_kernel(const f32x4* dropped, f32x4* g, size_t n4, float keep, unsigned* amax) {
    unsigned m = 0;
    GRID_STRIDE(i, n4) {
        const f32x4 d = dropped[i];
        f32x4 v = g[i];
#pragma unroll
        for (int e = 0; e < 4; ++e) v[e] = d[e] > 0.0f ? v[e] * keep : 0.0f;
        g[i] = v;
        m = max(m, amax_bits4(v));
    }
    block_amax_fold(m, amax);
}

// Rotary.Apply (Ops.cs:489-503) over rows of [rows, head_dim].
__global__ void rotary_kernel(const float* cos_t, const float* sin_t, int half, float* vec, int rows, const int* pos,
                              int inverse) {
    const size_t n = (size_t)rows * half;
    GRID_STRIDE(i, n) {
        const size_t r = i / half;
        const int k = (int)(i - r * half);
        const int t = pos[r];
        const float c = cos_t[(size_t)t * half + k];
        const float s = inverse ? -sin_t[(size_t)t * half + k] : sin_t[(size_t)t * half + k];
        float* v = vec + r * 2 * half;
        const float a = v[k], b = v[k + half];
        v[k] = a * c - b * s;
        v[k + half] = b * c + a * s;
    }
}

__global__ void embedding_fwd_kernel(const int* ids, int n, const float* E, int vocab, int hidden, float* out,
                                     int* bad) {
    const size_t total = (size_t)n * hidden;
    GRID_STRIDE(i, total) {
        const size_t t = i / hidden, c = i - t * hidden;
        const int id = ids[t];
        const bool ok = (unsigned)id < (unsigned)vocab;
        out[i] = ok ? E[(size_t)id * hidden + c] : 0.0f;
        if (!ok && c == 0 && bad) atomicAdd(bad, 1);
    }
}

// One block per unique id: grad[id] += Σ d[t] over the id's token positions, in token order.
__global__ void embedding_bwd_kernel(const int* __restrict__ sorted_pos, const int* __restrict__ unique_ids,
                                     const int* __restrict__ offsets, const float* __restrict__ d, int hidden,
                                     float* __restrict__ grad) {
    const int u = blockIdx.x;
    const int b = offsets[u], e = offsets[u + 1];
    float* g = grad + (size_t)unique_ids[u] * hidden;
    for (int c = threadIdx.x; c < hidden; c += blockDim.x) {
        float s = g[c];
        for (int k = b; k < e; ++k) s += d[(size_t)sorted_pos[k] * hidden + c];
        g[c] = s;
    }
}

// The same sums four columns per thread with the loads of 16 token rows in flight before they are added
// (in token order, so each column's sum is the serial one): a frequent id's long run of tokens is no longer
// one load latency per token.
__global__ void embedding_bwd4_kernel(const int* __restrict__ sorted_pos, const int* __restrict__ unique_ids,
                                      const int* __restrict__ offsets, const f32x4* __restrict__ d, int hidden4,
                                      f32x4* __restrict__ grad) {
    const int u = blockIdx.x;
    const int b = offsets[u], e = offsets[u + 1];
    f32x4* g = grad + (size_t)unique_ids[u] * hidden4;
    for (int c = threadIdx.x; c < hidden4; c += blockDim.x) {
        f32x4 s = g[c];
        int k = b;
        for (; k + 16 <= e; k += 16) {
            f32x4 v[16];
#pragma unroll
            for (int j = 0; j < 16; ++j) v[j] = d[(size_t)sorted_pos[k + j] * hidden4 + c];
#pragma unroll
            for (int j = 0; j < 16; ++j) s += v[j];
        }
        for (; k < e; ++k) s += d[(size_t)sorted_pos[k] * hidden4 + c];
        g[c] = s;
    }
}

__global__ void gather_rows_kernel(const float* src, const int* rows, int n, int width, float* dst) {
    const size_t total = (size_t)n * width;
    GRID_STRIDE(i, total) {
        const size_t r = i / width, c = i - r * width;
        dst[i] = src[(size_t)rows[r] * width + c];
    }
}

// dst[r] += table[idx[r]] over [rows, width] (float4 columns).
__global__ void add_indexed_rows4_kernel(f32x4* __restrict__ dst, const int* __restrict__ idx, int rows, int w4,
                                         const f32x4* __restrict__ table) {
    const size_t total = (size_t)rows * w4;
    GRID_STRIDE(i, total) {
        const size_t r = i / w4, c = i - r * w4;
        dst[i] += table[(size_t)idx[r] * w4 + c];
    }
}

// dst[rows[r]] += src[r] for r in order (one thread per column; rows may repeat).
__global__ void scatter_add_rows_kernel(const float* src, const int* rows, int n, int width, float* dst) {
    const int c = blockIdx.x * blockDim.x + threadIdx.x;
    if (c >= width) return;
    for (int r = 0; r < n; ++r) dst[(size_t)rows[r] * width + c] += src[(size_t)r * width + c];
}

// Column sums in two deterministic stages (bias gradients, the type-embedding gradient, LayerNorm γ/β
// partials). Stage 1: part[chunk][type][c] = Σ over the chunk's rows r with row_type[r] == type of x[r][c]
// (one type when row_type is null); a block is 64 float4 columns × 4 row phases, phase k summing rows
// k, k + 4, … in order, the phases combined in LDS in order. AMAX: max|x| over the values read folded into
// the word group amax as well (the operand magnitude a two-piece product of x needs, in the same pass).
template <int TYPES, bool AMAX = false>
__global__ __launch_bounds__(256) void colsum_partial4_kernel(const f32x4* __restrict__ x, int rows, int n4,
                                                              int rows_per, const int* __restrict__ row_type,
                                                              f32x4* __restrict__ part, unsigned* amax) {
    static_assert(TYPES == 1 || !AMAX, "the magnitude rides on the one-type sums");
    __shared__ f32x4 red[TYPES][4][64];
    const int lc = threadIdx.x & 63, ph = threadIdx.x >> 6;
    const int c = blockIdx.x * 64 + lc;
    const int r0 = blockIdx.y * rows_per, r1 = min(rows, r0 + rows_per);
    f32x4 acc[TYPES];
#pragma unroll
    for (int t = 0; t < TYPES; ++t) acc[t] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    unsigned m = 0;
    if (c < n4) {
#pragma unroll 4
        for (int r = r0 + ph; r < r1; r += 4) {
            const f32x4 v = x[(long)r * n4 + c];
            if (TYPES == 1) {
                acc[0] += v;
                if constexpr (AMAX) m = max(m, amax_bits4(v));
            } else {
                const int ty = row_type[r];
#pragma unroll
                for (int t = 0; t < TYPES; ++t)
                    if (ty == t) acc[t] += v;
            }
        }
    }
#pragma unroll
    for (int t = 0; t < TYPES; ++t) red[t][ph][lc] = acc[t];
    __syncthreads();
    if (ph == 0 && c < n4)
#pragma unroll
        for (int t = 0; t < TYPES; ++t)
            part[((long)blockIdx.y * TYPES + t) * n4 + c] =
                ((red[t][0][lc] + red[t][1][lc]) + red[t][2][lc]) + red[t][3][lc];
    if constexpr (AMAX) block_amax_fold(m, amax);
}

// Stage 2: out[c] += Σ_k part[k][c] over `count` partials; a block is 16 float4 columns × 16 phases,
// phase q summing partials q, q + 16, … in order, the phases combined in order.
__global__ __launch_bounds__(256) void colsum_reduce4_kernel(const f32x4* __restrict__ part, int count, int w4,
                                                             f32x4* __restrict__ out) {
    __shared__ f32x4 red[16][16];
    const int lc = threadIdx.x & 15, ph = threadIdx.x >> 4;
    const int c = blockIdx.x * 16 + lc;
    f32x4 s = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    if (c < w4) {
#pragma unroll 4
        for (int k = ph; k < count; k += 16) s += part[(long)k * w4 + c];
    }
    red[ph][lc] = s;
    __syncthreads();
    if (ph == 0 && c < w4) {
        f32x4 t = red[0][lc];
#pragma unroll
        for (int q = 1; q < 16; ++q) t += red[q][lc];
        out[c] += t;
    }
}

// The same reduction for a batch of independent column sums in one launch: blockIdx.y picks the job.
__global__ __launch_bounds__(256) void colsum_reduce4_multi_kernel(ColumnSumJobs jobs) {
    const ColumnSumJob j = jobs.job[blockIdx.y];
    const int w4 = j.n / 4;
    if ((int)blockIdx.x * 16 >= w4) return;  // block-uniform
    __shared__ f32x4 red[16][16];
    const f32x4* part = reinterpret_cast<const f32x4*>(j.part);
    const int lc = threadIdx.x & 15, ph = threadIdx.x >> 4;
    const int c = blockIdx.x * 16 + lc;
    f32x4 s = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    if (c < w4) {
#pragma unroll 4
        for (int k = ph; k < j.count; k += 16) s += part[(long)k * w4 + c];
    }
    red[ph][lc] = s;
    __syncthreads();
    if (ph == 0 && c < w4) {
        f32x4 t = red[0][lc];
#pragma unroll
        for (int q = 1; q < 16; ++q) t += red[q][lc];
        reinterpret_cast<f32x4*>(j.out)[c] += t;
    }
}

// Soft cross-entropy gradient (RlcdObjective.cs:139-150): one thread per item computes its options'
// gradient and its loss term; the terms are then added in item order by one thread (a fixed order).
constexpr int CE_THREADS = 256;
__global__ __launch_bounds__(CE_THREADS) void softmax_ce_kernel(const float* logits, const float* targets,
                                                                const int* offsets, int n_items, float ce_weight,
                                                                float scale, float* grad, float* loss,
                                                                double* terms) {
    for (int i = threadIdx.x; i < n_items; i += CE_THREADS) {
        const int b = offsets[i], k = offsets[i + 1] - offsets[i];
        float mx = -__builtin_huge_valf();
        for (int o = 0; o < k; ++o) mx = fmaxf(mx, logits[b + o]);
        float total = 0.0f;
        for (int o = 0; o < k; ++o) total += expf(logits[b + o] - mx);
        const float inv = total > 0.0f ? 1.0f / total : 0.0f;
        double mass = 0.0;
        for (int o = 0; o < k; ++o) mass += targets[b + o];
        double ce = 0.0;
        for (int o = 0; o < k; ++o) {
            const float p = expf(logits[b + o] - mx) * inv;
            ce -= targets[b + o] * log(fmax((double)p, 1e-30)) / n_items;
            const double g = (double)ce_weight * (p * mass - targets[b + o]) / n_items;
            grad[b + o] = (float)(g * scale);
        }
        terms[i] = ce;
    }
    if (!loss) return;
    __syncthreads();
    if (threadIdx.x != 0) return;
    double ce = 0.0;
    for (int i = 0; i < n_items; ++i) ce += terms[i];
    *loss = (float)ce;
}

// N(0, std) by Box–Muller over two counter-RNG draws; kind 0 normal, 1 ones, 2 zeros.
__global__ void init_kernel(float* dst, size_t n, int kind, float std, uint64_t seed) {
    GRID_STRIDE(i, n) {
        float v;
        if (kind == 1) {
            v = 1.0f;
        } else if (kind == 2) {
            v = 0.0f;
        } else {
            const float u1 = uniform01(seed, 2 * i), u2 = uniform01(seed, 2 * i + 1);
            v = std * sqrtf(-2.0f * logf(1.0f - u1)) * cospif(2.0f * u2);
        }
        dst[i] = v;
    }
}

unsigned grid_for(size_t n) { return blocks_for(n, 256, 8192); }

}  // namespace

bool vec4(const void* p) { return ((uintptr_t)p & 15u) == 0; }

void fill(laya_ctx* ctx, float* dst, float v, size_t n) {
    if (!n) return;
    ProfileScope scope(ctx, "fill", 0.0, 4.0 * n);
    if (n % 4 == 0 && vec4(dst)) {
        LAYA_LAUNCH(fill4_kernel, dim3(grid_for(n / 4)), dim3(256), 0, ctx->stream,
                           reinterpret_cast<f32x4*>(dst), v, n / 4);
        check_launch("fill4_kernel");
        return;
    }
    LAYA_LAUNCH(fill_kernel, dim3(grid_for(n)), dim3(256), 0, ctx->stream, dst, v, n);
    check_launch("fill_kernel");
}
void add(laya_ctx* ctx, float* dst, const float* src, size_t n) {
    if (!n) return;
    ProfileScope scope(ctx, "add", 0.0, 12.0 * n);
    if (n % 4 == 0 && vec4(dst) && vec4(src)) {
        LAYA_LAUNCH(add4_kernel, dim3(grid_for(n / 4)), dim3(256), 0, ctx->stream,
                           reinterpret_cast<f32x4*>(dst), reinterpret_cast<const f32x4*>(src), n / 4);
        check_launch("add4_kernel");
        return;
    }
    LAYA_LAUNCH(add_kernel, dim3(grid_for(n)), dim3(256), 0, ctx->stream, dst, src, n);
    check_launch("add_kernel");
}
void scale(laya_ctx* ctx, float* dst, float s, size_t n) {
    if (!n) return;
    LAYA_LAUNCH(scale_kernel, dim3(grid_for(n)), dim3(256), 0, ctx->stream, dst, s, n);
    check_launch("scale_kernel");
}
void gelu_fwd(laya_ctx* ctx, const float* x, size_t n, float* y) {
    if (!n) return;
    LAYA_LAUNCH(gelu_fwd_kernel, dim3(grid_for(n)), dim3(256), 0, ctx->stream, x, n, y);
    check_launch("gelu_fwd_kernel");
}
void gelu_bwd(laya_ctx* ctx, const float* u, float* g, size_t n) {
    if (!n) return;
    LAYA_LAUNCH(gelu_bwd_kernel, dim3(grid_for(n)), dim3(256), 0, ctx->stream, u, g, n);
    check_launch("gelu_bwd_kernel");
}
void geglu_fwd(laya_ctx* ctx, const float* wide, int rows, int inter, float* act, __bf16* act16, unsigned* amax) {
    if (rows <= 0 || inter <= 0) return;
    ProfileScope scope(ctx, "geglu_fwd", 0.0, (12.0 + (act16 ? 2.0 : 0.0)) * rows * (double)inter);
    if (inter % 4 == 0) {
        LAYA_LAUNCH(geglu_fwd_kernel, dim3(grid_for((size_t)rows * inter / 4)), dim3(256), 0, ctx->stream,
                           wide, rows, inter, act, act16, amax);
    } else {
        LAYA_LAUNCH(geglu_fwd_scalar_kernel, dim3(grid_for((size_t)rows * inter)), dim3(256), 0, ctx->stream,
                           wide, rows, inter, act);
        if (act16) to_bf16(ctx, act, (size_t)rows * inter, act16);
        if (amax) absmax_into(ctx, act, rows, inter, inter, amax);
    }
    check_launch("geglu_fwd_kernel");
}

void to_bf16(laya_ctx* ctx, const float* src, size_t n, __bf16* dst) {
    if (!n) return;
    ProfileScope scope(ctx, "to_bf16", 0.0, 6.0 * n);
    if (n % 4 == 0 && vec4(src) && ((uintptr_t)dst & 7u) == 0) {
        LAYA_LAUNCH(to_bf16_kernel, dim3(grid_for(n / 4)), dim3(256), 0, ctx->stream,
                           reinterpret_cast<const f32x4*>(src), reinterpret_cast<bf16x4*>(dst), n / 4);
        check_launch("to_bf16_kernel");
        return;
    }
    LAYA_LAUNCH(to_bf16_scalar_kernel, dim3(grid_for(n)), dim3(256), 0, ctx->stream, src, dst, n);
    check_launch("to_bf16_scalar_kernel");
}
void round_bf16(laya_ctx* ctx, const float* src, size_t n, float* dst) {
    if (!n) return;
    ProfileScope scope(ctx, "round_bf16", 0.0, 8.0 * n);
    if (n % 4 == 0 && vec4(src) && vec4(dst)) {
        LAYA_LAUNCH(round_bf16_kernel, dim3(grid_for(n / 4)), dim3(256), 0, ctx->stream,
                           reinterpret_cast<const f32x4*>(src), reinterpret_cast<f32x4*>(dst), n / 4);
        check_launch("round_bf16_kernel");
        return;
    }
    LAYA_LAUNCH(round_bf16_scalar_kernel, dim3(grid_for(n)), dim3(256), 0, ctx->stream, src, dst, n);
    check_launch("round_bf16_scalar_kernel");
}
void geglu_bwd(laya_ctx* ctx, const float* wide, const float* dact, int rows, int inter, float* dwide,
               unsigned* amax) {
    if (rows <= 0 || inter <= 0) return;
    ProfileScope scope(ctx, "geglu_bwd", 0.0, 20.0 * rows * (double)inter);
    if (inter % 4 == 0) {
        LAYA_LAUNCH(geglu_bwd_kernel, dim3(grid_for((size_t)rows * inter / 4)), dim3(256), 0, ctx->stream,
                           wide, dact, rows, inter, dwide, amax);
    } else {
        LAYA_LAUNCH(geglu_bwd_scalar_kernel, dim3(grid_for((size_t)rows * inter)), dim3(256), 0, ctx->stream,
                           wide, dact, rows, inter, dwide);
        if (amax) absmax_into(ctx, dwide, rows, 2 * inter, 2 * inter, amax);
    }
    check_launch("geglu_bwd_kernel");
}
void dropout(laya_ctx* ctx, float* v, size_t n, float p, uint64_t seed) {
    if (!n || p <= 0.0f) return;
    ProfileScope scope(ctx, "dropout", 0.0, 8.0 * n);
    if (n % 4 == 0 && vec4(v)) {
        LAYA_LAUNCH(dropout4_kernel, dim3(grid_for(n / 4)), dim3(256), 0, ctx->stream,
                           reinterpret_cast<f32x4*>(v), n / 4, p, 1.0f / (1.0f - p), seed);
        check_launch("dropout4_kernel");
        return;
    }
    LAYA_LAUNCH(dropout_kernel, dim3(grid_for(n)), dim3(256), 0, ctx->stream, v, n, p, 1.0f / (1.0f - p),
                       seed);
    check_launch("dropout_kernel");
}
void dropout_add(laya_ctx* ctx, float* v, const float* r, size_t n, float p, uint64_t seed) {
    if (!n) return;
    if (p > 0.0f && n % 4 == 0 && vec4(v) && vec4(r)) {
        ProfileScope scope(ctx, "dropout_add", 0.0, 12.0 * n);
        LAYA_LAUNCH(dropout_add4_kernel, dim3(grid_for(n / 4)), dim3(256), 0, ctx->stream,
                    reinterpret_cast<f32x4*>(v), reinterpret_cast<const f32x4*>(r), n / 4, p, 1.0f / (1.0f - p), seed);
        check_launch("dropout_add4_kernel");
        return;
    }
    dropout(ctx, v, n, p, seed);
    add(ctx, v, r, n);
}
void dropout_copy(laya_ctx* ctx, const float* src, float* dst, size_t n, float p, uint64_t seed) {
    if (!n) return;
    if (p <= 0.0f || n % 4 != 0 || !vec4(src) || !vec4(dst)) {
        LAYA_HIP(hipMemcpyAsync(dst, src, n * sizeof(float), hipMemcpyDeviceToDevice, ctx->stream));
        dropout(ctx, dst, n, p, seed);
        return;
    }
    ProfileScope scope(ctx, "dropout", 0.0, 8.0 * n);
    LAYA_LAUNCH(dropout_copy4_kernel, dim3(grid_for(n / 4)), dim3(256), 0, ctx->stream,
                       reinterpret_cast<const f32x4*>(src), reinterpret_cast<f32x4*>(dst), n / 4, p,
                       1.0f / (1.0f - p), seed);
    check_launch("dropout_copy4_kernel");
}
void relu_dropout_fwd(laya_ctx* ctx, const float* wide, size_t n, float p, uint64_t seed, float* dropped,
                      __bf16* dropped16, unsigned* amax) {
    if (!n) return;
    const float keep = p > 0.0f ? 1.0f / (1.0f - p) : 1.0f;
    ProfileScope scope(ctx, "relu_dropout_fwd", 0.0, (8.0 + (dropped16 ? 2.0 : 0.0)) * n);
    if (n % 4 == 0 && vec4(wide) && vec4(dropped) && ((uintptr_t)dropped16 & 7u) == 0) {
        LAYA_LAUNCH(relu_dropout_fwd4_kernel, dim3(grid_for(n / 4)), dim3(256), 0, ctx->stream,
                           reinterpret_cast<const f32x4*>(wide), n / 4, p, keep, seed,
                           reinterpret_cast<f32x4*>(dropped), reinterpret_cast<bf16x4*>(dropped16), amax);
        check_launch("relu_dropout_fwd4_kernel");
        return;
    }
    LAYA_LAUNCH(relu_dropout_fwd_kernel, dim3(grid_for(n)), dim3(256), 0, ctx->stream, wide, n, p, keep, seed,
                       dropped);
    check_launch("relu_dropout_fwd_kernel");
    if (dropped16) to_bf16(ctx, dropped, n, dropped16);
    if (amax) {
        LAYA_REQUIRE(n <= (size_t)INT32_MAX, "relu_dropout_fwd: too many elements to measure");
        absmax_into(ctx, dropped, 1, (int)n, (long)n, amax);
    }
}
void relu_dropout_bwd(laya_ctx* ctx, const float* wide, float* g, size_t n, float p, uint64_t seed) {
    if (!n) return;
    const float keep = p > 0.0f ? 1.0f / (1.0f - p) : 1.0f;
    ProfileScope scope(ctx, "relu_dropout_bwd", 0.0, 12.0 * n);
    LAYA_LAUNCH(relu_dropout_bwd_kernel, dim3(grid_for(n)), dim3(256), 0, ctx->stream, wide, g, n, p, keep,
                       seed);
    check_launch("relu_dropout_bwd_kernel");
}
void relu_dropout_bwd_from_output(laya_ctx* ctx, const float* dropped, float* g, size_t n, float p, unsigned* amax) {
    if (!n) return;
    LAYA_REQUIRE(n % 4 == 0 && vec4(dropped) && vec4(g), "relu_dropout_bwd: 16-byte aligned multiples of 4");
    const float keep = p > 0.0f ? 1.0f / (1.0f - p) : 1.0f;
    ProfileScope scope(ctx, "relu_dropout_bwd", 0.0, 12.0 * n);
    LAYA_LAUNCH(relu_dropout_bwd_out4_kernel, dim3(grid_for(n / 4)), dim3(256), 0, ctx->stream,
                       reinterpret_cast<const f32x4*>(dropped), reinterpret_cast<f32x4*>(g), n / 4, keep, amax);
    check_launch("relu_dropout_bwd_out4_kernel");
}
void column_sums(laya_ctx* ctx, const float* x, int rows, int n, const int* row_type, int types, float* out,
                 int slot, unsigned* amax) {
    LAYA_REQUIRE(types == 1 || types == 3, "column_sums: one or three row types");
    LAYA_REQUIRE(!amax || types == 1, "column_sums: the magnitude rides on the one-type sums");
    LAYA_REQUIRE(n % 4 == 0 && vec4(x) && vec4(out), "column_sums: 16-byte aligned rows of a multiple of 4");
    if (rows <= 0 || n <= 0) return;
    const int n4 = n / 4, cblocks = (n4 + 63) / 64;
    // About 2048 workgroups in stage 1, at least 16 rows each.
    const int want = std::max(1, 2048 / cblocks);
    const int rows_per = std::max(16, ((rows + want - 1) / want + 15) / 16 * 16);
    const int chunks = (rows + rows_per - 1) / rows_per;
    f32x4* part = static_cast<f32x4*>(ctx->workspace(slot, sizeof(f32x4) * (size_t)chunks * types * n4));
    ProfileScope scope(ctx, "column_sums", 0.0, 4.0 * (double)rows * n);
    if (amax)
        LAYA_LAUNCH((colsum_partial4_kernel<1, true>), dim3(cblocks, chunks), dim3(256), 0, ctx->stream,
                    reinterpret_cast<const f32x4*>(x), rows, n4, rows_per, nullptr, part, amax);
    else if (types == 1)
        LAYA_LAUNCH(colsum_partial4_kernel<1>, dim3(cblocks, chunks), dim3(256), 0, ctx->stream,
                           reinterpret_cast<const f32x4*>(x), rows, n4, rows_per, nullptr, part, nullptr);
    else
        LAYA_LAUNCH(colsum_partial4_kernel<3>, dim3(cblocks, chunks), dim3(256), 0, ctx->stream,
                           reinterpret_cast<const f32x4*>(x), rows, n4, rows_per, row_type, part, nullptr);
    check_launch("colsum_partial4_kernel");
    column_reduce(ctx, reinterpret_cast<const float*>(part), chunks, types * n, out);
}
void column_reduce(laya_ctx* ctx, const float* part, int count, int n, float* out) {
    LAYA_REQUIRE(n % 4 == 0 && vec4(part) && vec4(out), "column_reduce: 16-byte aligned rows of a multiple of 4");
    if (count <= 0 || n <= 0) return;
    const int w4 = n / 4;
    LAYA_LAUNCH(colsum_reduce4_kernel, dim3((w4 + 15) / 16), dim3(256), 0, ctx->stream,
                       reinterpret_cast<const f32x4*>(part), count, w4, reinterpret_cast<f32x4*>(out));
    check_launch("colsum_reduce4_kernel");
}
void column_reduce_batch(laya_ctx* ctx, const ColumnSumJobs& jobs) {
    if (jobs.n <= 0) return;
    int max_w4 = 0;
    for (int i = 0; i < jobs.n; ++i) {
        const ColumnSumJob& j = jobs.job[i];
        LAYA_REQUIRE(j.n % 4 == 0 && vec4(j.part) && vec4(j.out) && j.count > 0,
                     "column_reduce_batch: 16-byte aligned rows of a multiple of 4");
        max_w4 = std::max(max_w4, j.n / 4);
    }
    double bytes = 0;
    for (int i = 0; i < jobs.n; ++i) bytes += 4.0 * jobs.job[i].n * (jobs.job[i].count + 2);
    ProfileScope scope(ctx, "column_sums_deferred", 0.0, bytes);
    LAYA_LAUNCH(colsum_reduce4_multi_kernel, dim3((max_w4 + 15) / 16, jobs.n), dim3(256), 0, ctx->stream, jobs);
    check_launch("colsum_reduce4_multi_kernel");
}
void rotary_apply(laya_ctx* ctx, const float* cos_t, const float* sin_t, int head_dim, float* vec, int rows,
                  const int* pos, int inverse) {
    if (rows <= 0) return;
    const int half = head_dim / 2;
    LAYA_LAUNCH(rotary_kernel, dim3(grid_for((size_t)rows * half)), dim3(256), 0, ctx->stream, cos_t, sin_t,
                       half, vec, rows, pos, inverse);
    check_launch("rotary_kernel");
}
void embedding_fwd(laya_ctx* ctx, const int* ids, int n, const float* E, int vocab, int hidden, float* out,
                   int* bad) {
    if (n <= 0) return;
    LAYA_LAUNCH(embedding_fwd_kernel, dim3(grid_for((size_t)n * hidden)), dim3(256), 0, ctx->stream, ids, n,
                       E, vocab, hidden, out, bad);
    check_launch("embedding_fwd_kernel");
}
void embedding_bwd(laya_ctx* ctx, const int* sorted_pos, const int* unique_ids, const int* offsets, int n_unique,
                   const float* d, int hidden, float* grad) {
    if (n_unique <= 0) return;
    ProfileScope scope(ctx, "embedding_bwd", 0.0, 0.0);
    if (hidden % 4 == 0 && vec4(d) && vec4(grad)) {
        const int h4 = hidden / 4;
        LAYA_LAUNCH(embedding_bwd4_kernel, dim3(n_unique), dim3(std::min(256, (h4 + 63) / 64 * 64)), 0,
                           ctx->stream, sorted_pos, unique_ids, offsets, reinterpret_cast<const f32x4*>(d), h4,
                           reinterpret_cast<f32x4*>(grad));
        check_launch("embedding_bwd4_kernel");
        return;
    }
    LAYA_LAUNCH(embedding_bwd_kernel, dim3(n_unique), dim3(256), 0, ctx->stream, sorted_pos, unique_ids,
                       offsets, d, hidden, grad);
    check_launch("embedding_bwd_kernel");
}
void gather_rows(laya_ctx* ctx, const float* src, const int* rows, int n, int width, float* dst) {
    if (n <= 0) return;
    LAYA_LAUNCH(gather_rows_kernel, dim3(grid_for((size_t)n * width)), dim3(256), 0, ctx->stream, src, rows, n,
                       width, dst);
    check_launch("gather_rows_kernel");
}
void scatter_add_rows(laya_ctx* ctx, const float* src, const int* rows, int n, int width, float* dst) {
    if (n <= 0) return;
    LAYA_LAUNCH(scatter_add_rows_kernel, dim3((width + 255) / 256), dim3(256), 0, ctx->stream, src, rows, n,
                       width, dst);
    check_launch("scatter_add_rows_kernel");
}
void add_indexed_rows(laya_ctx* ctx, float* dst, const int* idx, int rows, int width, const float* table) {
    if (rows <= 0 || width <= 0) return;
    LAYA_REQUIRE(width % 4 == 0 && vec4(dst) && vec4(table), "add_indexed_rows: 16-byte aligned rows of a multiple of 4");
    ProfileScope scope(ctx, "add_indexed_rows", 0.0, 8.0 * rows * (double)width);
    LAYA_LAUNCH(add_indexed_rows4_kernel, dim3(grid_for((size_t)rows * width / 4)), dim3(256), 0, ctx->stream,
                       reinterpret_cast<f32x4*>(dst), idx, rows, width / 4, reinterpret_cast<const f32x4*>(table));
    check_launch("add_indexed_rows4_kernel");
}
void type_embedding_bwd(laya_ctx* ctx, const float* d, const int* row_type, int rows, int width, float* grad) {
    if (rows <= 0) return;
    if (width % 4 == 0 && vec4(d) && vec4(grad)) {
        column_sums(ctx, d, rows, width, row_type, 3, grad, 1);
        return;
    }
    LAYA_REQUIRE(false, "type_embedding_bwd: rows must be 16-byte aligned multiples of 4 floats");
}
void softmax_ce_bwd(laya_ctx* ctx, const float* logits, const float* targets, const int* offsets, int n_items,
                    float ce_weight, float s, float* grad, float* loss) {
    if (n_items <= 0) return;
    double* terms = static_cast<double*>(ctx->workspace(1, sizeof(double) * (size_t)n_items));
    LAYA_LAUNCH(softmax_ce_kernel, dim3(1), dim3(CE_THREADS), 0, ctx->stream, logits, targets, offsets, n_items,
                       ce_weight, s, grad, loss, terms);
    check_launch("softmax_ce_kernel");
}
void init_param(laya_ctx* ctx, float* dst, size_t n, int kind, float std, uint64_t seed) {
    if (!n) return;
    LAYA_LAUNCH(init_kernel, dim3(grid_for(n)), dim3(256), 0, ctx->stream, dst, n, kind, std, seed);
    check_launch("init_kernel");
}

}  // namespace laya
