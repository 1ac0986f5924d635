// Memory-bound kernels of the step: activations, dropout, residual adds, row gathers/scatters,
// embedding and type-embedding gradients, the decision-head cross-entropy gradient, and synthetic
// initialisation. All are coalesced float4 streams where the shape allows; every reduction over
// rows runs in a fixed order.
#include "elementwise.hpp"

namespace laya {
namespace {

typedef float f32x4 __attribute__((ext_vector_type(4)));
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

__global__ void gelu_fwd_kernel(const float* x, size_t n, float* y) {
    GRID_STRIDE(i, n) y[i] = gelu_f(x[i]);
}

__global__ void gelu_bwd_kernel(const float* u, float* g, size_t n) {
    GRID_STRIDE(i, n) g[i] *= gelu_grad_f(u[i]);
}

// GeGLU, 4 columns per thread: act[t, i] = gelu(wide[t, i]) · wide[t, I + i].
__global__ void geglu_fwd_kernel(const float* __restrict__ wide, int rows, int inter, float* __restrict__ act) {
    const int q = inter >> 2;
    const size_t n = (size_t)rows * q;
    GRID_STRIDE(i, n) {
        const size_t t = i / q;
        const int c = (int)(i - t * q) * 4;
        const float* w = wide + t * 2 * inter;
        const f32x4 x = ld4(w + c), g = ld4(w + inter + c);
        st4(act + t * inter + c, f32x4{gelu_f(x[0]) * g[0], gelu_f(x[1]) * g[1], gelu_f(x[2]) * g[2],
                                       gelu_f(x[3]) * g[3]});
    }
}

// dwide[t] = [dact·gate·gelu'(input) | dact·gelu(input)] (TrainableDecisionModel.cs:573-578).
__global__ void geglu_bwd_kernel(const float* __restrict__ wide, const float* __restrict__ dact, int rows, int inter,
                                 float* __restrict__ dwide) {
    const int q = inter >> 2;
    const size_t n = (size_t)rows * q;
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
    }
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

__global__ void gather_rows_kernel(const float* src, const int* rows, int n, int width, float* dst) {
    const size_t total = (size_t)n * width;
    GRID_STRIDE(i, total) {
        const size_t r = i / width, c = i - r * width;
        dst[i] = src[(size_t)rows[r] * width + c];
    }
}

// dst[rows[r]] += src[r] for r in order (one thread per column; rows may repeat).
__global__ void scatter_add_rows_kernel(const float* src, const int* rows, int n, int width, float* dst) {
    const int c = blockIdx.x * blockDim.x + threadIdx.x;
    if (c >= width) return;
    for (int r = 0; r < n; ++r) dst[(size_t)rows[r] * width + c] += src[(size_t)r * width + c];
}

// Per-segment column sums, then per-type accumulation in segment order (TrainableDecisionModel.cs:512-521).
__global__ void segment_sum_kernel(const float* d, const int* seg_start, const int* seg_len, int width,
                                   float* part) {
    const int s = blockIdx.y;
    const int c = blockIdx.x * blockDim.x + threadIdx.x;
    if (c >= width) return;
    const int b = seg_start[s], L = seg_len[s];
    float acc = 0.0f;
    for (int t = 0; t < L; ++t) acc += d[(size_t)(b + t) * width + c];
    part[(size_t)s * width + c] = acc;
}

__global__ void type_accumulate_kernel(const float* part, const int* qtypes, int nseg, int width, float* grad) {
    const int c = blockIdx.x * blockDim.x + threadIdx.x;
    if (c >= width) return;
    for (int s = 0; s < nseg; ++s) grad[(size_t)qtypes[s] * width + c] += part[(size_t)s * width + c];
}

// Soft cross-entropy gradient (RlcdObjective.cs:139-150), one thread, items in order.
__global__ void softmax_ce_kernel(const float* logits, const float* targets, const int* offsets, int n_items,
                                  float ce_weight, float scale, float* grad, float* loss) {
    if (threadIdx.x != 0 || blockIdx.x != 0) return;
    double ce = 0.0;
    for (int i = 0; i < n_items; ++i) {
        const int b = offsets[i], k = offsets[i + 1] - offsets[i];
        float mx = -__builtin_huge_valf();
        for (int o = 0; o < k; ++o) mx = fmaxf(mx, logits[b + o]);
        float total = 0.0f;
        for (int o = 0; o < k; ++o) total += expf(logits[b + o] - mx);
        const float inv = total > 0.0f ? 1.0f / total : 0.0f;
        double mass = 0.0;
        for (int o = 0; o < k; ++o) mass += targets[b + o];
        for (int o = 0; o < k; ++o) {
            const float p = expf(logits[b + o] - mx) * inv;
            ce -= targets[b + o] * log(fmax((double)p, 1e-30)) / n_items;
            const double g = (double)ce_weight * (p * mass - targets[b + o]) / n_items;
            grad[b + o] = (float)(g * scale);
        }
    }
    if (loss) *loss = (float)ce;
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

void fill(laya_ctx* ctx, float* dst, float v, size_t n) {
    if (!n) return;
    ProfileScope scope(ctx, "fill", 0.0, 4.0 * n);
    hipLaunchKernelGGL(fill_kernel, dim3(grid_for(n)), dim3(256), 0, ctx->stream, dst, v, n);
    check_launch("fill_kernel");
}
void add(laya_ctx* ctx, float* dst, const float* src, size_t n) {
    if (!n) return;
    ProfileScope scope(ctx, "add", 0.0, 12.0 * n);
    hipLaunchKernelGGL(add_kernel, dim3(grid_for(n)), dim3(256), 0, ctx->stream, dst, src, n);
    check_launch("add_kernel");
}
void scale(laya_ctx* ctx, float* dst, float s, size_t n) {
    if (!n) return;
    hipLaunchKernelGGL(scale_kernel, dim3(grid_for(n)), dim3(256), 0, ctx->stream, dst, s, n);
    check_launch("scale_kernel");
}
void gelu_fwd(laya_ctx* ctx, const float* x, size_t n, float* y) {
    if (!n) return;
    hipLaunchKernelGGL(gelu_fwd_kernel, dim3(grid_for(n)), dim3(256), 0, ctx->stream, x, n, y);
    check_launch("gelu_fwd_kernel");
}
void gelu_bwd(laya_ctx* ctx, const float* u, float* g, size_t n) {
    if (!n) return;
    hipLaunchKernelGGL(gelu_bwd_kernel, dim3(grid_for(n)), dim3(256), 0, ctx->stream, u, g, n);
    check_launch("gelu_bwd_kernel");
}
void geglu_fwd(laya_ctx* ctx, const float* wide, int rows, int inter, float* act) {
    if (rows <= 0 || inter <= 0) return;
    ProfileScope scope(ctx, "geglu_fwd", 0.0, 12.0 * rows * (double)inter);
    if (inter % 4 == 0) {
        hipLaunchKernelGGL(geglu_fwd_kernel, dim3(grid_for((size_t)rows * inter / 4)), dim3(256), 0, ctx->stream,
                           wide, rows, inter, act);
    } else {
        hipLaunchKernelGGL(geglu_fwd_scalar_kernel, dim3(grid_for((size_t)rows * inter)), dim3(256), 0, ctx->stream,
                           wide, rows, inter, act);
    }
    check_launch("geglu_fwd_kernel");
}
void geglu_bwd(laya_ctx* ctx, const float* wide, const float* dact, int rows, int inter, float* dwide) {
    if (rows <= 0 || inter <= 0) return;
    ProfileScope scope(ctx, "geglu_bwd", 0.0, 20.0 * rows * (double)inter);
    if (inter % 4 == 0) {
        hipLaunchKernelGGL(geglu_bwd_kernel, dim3(grid_for((size_t)rows * inter / 4)), dim3(256), 0, ctx->stream,
                           wide, dact, rows, inter, dwide);
    } else {
        hipLaunchKernelGGL(geglu_bwd_scalar_kernel, dim3(grid_for((size_t)rows * inter)), dim3(256), 0, ctx->stream,
                           wide, dact, rows, inter, dwide);
    }
    check_launch("geglu_bwd_kernel");
}
void dropout(laya_ctx* ctx, float* v, size_t n, float p, uint64_t seed) {
    if (!n || p <= 0.0f) return;
    ProfileScope scope(ctx, "dropout", 0.0, 8.0 * n);
    hipLaunchKernelGGL(dropout_kernel, dim3(grid_for(n)), dim3(256), 0, ctx->stream, v, n, p, 1.0f / (1.0f - p),
                       seed);
    check_launch("dropout_kernel");
}
void relu_dropout_fwd(laya_ctx* ctx, const float* wide, size_t n, float p, uint64_t seed, float* dropped) {
    if (!n) return;
    const float keep = p > 0.0f ? 1.0f / (1.0f - p) : 1.0f;
    ProfileScope scope(ctx, "relu_dropout_fwd", 0.0, 8.0 * n);
    hipLaunchKernelGGL(relu_dropout_fwd_kernel, dim3(grid_for(n)), dim3(256), 0, ctx->stream, wide, n, p, keep, seed,
                       dropped);
    check_launch("relu_dropout_fwd_kernel");
}
void relu_dropout_bwd(laya_ctx* ctx, const float* wide, float* g, size_t n, float p, uint64_t seed) {
    if (!n) return;
    const float keep = p > 0.0f ? 1.0f / (1.0f - p) : 1.0f;
    ProfileScope scope(ctx, "relu_dropout_bwd", 0.0, 12.0 * n);
    hipLaunchKernelGGL(relu_dropout_bwd_kernel, dim3(grid_for(n)), dim3(256), 0, ctx->stream, wide, g, n, p, keep,
                       seed);
    check_launch("relu_dropout_bwd_kernel");
}
void rotary_apply(laya_ctx* ctx, const float* cos_t, const float* sin_t, int head_dim, float* vec, int rows,
                  const int* pos, int inverse) {
    if (rows <= 0) return;
    const int half = head_dim / 2;
    hipLaunchKernelGGL(rotary_kernel, dim3(grid_for((size_t)rows * half)), dim3(256), 0, ctx->stream, cos_t, sin_t,
                       half, vec, rows, pos, inverse);
    check_launch("rotary_kernel");
}
void embedding_fwd(laya_ctx* ctx, const int* ids, int n, const float* E, int vocab, int hidden, float* out,
                   int* bad) {
    if (n <= 0) return;
    hipLaunchKernelGGL(embedding_fwd_kernel, dim3(grid_for((size_t)n * hidden)), dim3(256), 0, ctx->stream, ids, n,
                       E, vocab, hidden, out, bad);
    check_launch("embedding_fwd_kernel");
}
void embedding_bwd(laya_ctx* ctx, const int* sorted_pos, const int* unique_ids, const int* offsets, int n_unique,
                   const float* d, int hidden, float* grad) {
    if (n_unique <= 0) return;
    ProfileScope scope(ctx, "embedding_bwd", 0.0, 0.0);
    hipLaunchKernelGGL(embedding_bwd_kernel, dim3(n_unique), dim3(256), 0, ctx->stream, sorted_pos, unique_ids,
                       offsets, d, hidden, grad);
    check_launch("embedding_bwd_kernel");
}
void gather_rows(laya_ctx* ctx, const float* src, const int* rows, int n, int width, float* dst) {
    if (n <= 0) return;
    hipLaunchKernelGGL(gather_rows_kernel, dim3(grid_for((size_t)n * width)), dim3(256), 0, ctx->stream, src, rows, n,
                       width, dst);
    check_launch("gather_rows_kernel");
}
void scatter_add_rows(laya_ctx* ctx, const float* src, const int* rows, int n, int width, float* dst) {
    if (n <= 0) return;
    hipLaunchKernelGGL(scatter_add_rows_kernel, dim3((width + 255) / 256), dim3(256), 0, ctx->stream, src, rows, n,
                       width, dst);
    check_launch("scatter_add_rows_kernel");
}
void type_embedding_bwd(laya_ctx* ctx, const float* d, const int* seg_start, const int* seg_len, const int* qtypes,
                        int nseg, int width, float* grad) {
    if (nseg <= 0) return;
    float* part = static_cast<float*>(ctx->workspace(1, sizeof(float) * (size_t)nseg * width));
    hipLaunchKernelGGL(segment_sum_kernel, dim3((width + 255) / 256, nseg), dim3(256), 0, ctx->stream, d, seg_start,
                       seg_len, width, part);
    check_launch("segment_sum_kernel");
    hipLaunchKernelGGL(type_accumulate_kernel, dim3((width + 255) / 256), dim3(256), 0, ctx->stream, part, qtypes,
                       nseg, width, grad);
    check_launch("type_accumulate_kernel");
}
void softmax_ce_bwd(laya_ctx* ctx, const float* logits, const float* targets, const int* offsets, int n_items,
                    float ce_weight, float s, float* grad, float* loss) {
    if (n_items <= 0) return;
    hipLaunchKernelGGL(softmax_ce_kernel, dim3(1), dim3(64), 0, ctx->stream, logits, targets, offsets, n_items,
                       ce_weight, s, grad, loss);
    check_launch("softmax_ce_kernel");
}
void init_param(laya_ctx* ctx, float* dst, size_t n, int kind, float std, uint64_t seed) {
    if (!n) return;
    hipLaunchKernelGGL(init_kernel, dim3(grid_for(n)), dim3(256), 0, ctx->stream, dst, n, kind, std, seed);
    check_launch("init_kernel");
}

}  // namespace laya
