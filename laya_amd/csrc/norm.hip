// LayerNorm forward and backward, one 64-lane wavefront per row.
//
// Forward restates SimdOps.LayerNorm (src/StructuredDecisions.Base/Numerics/SimdOps.cs:234-272):
// biased variance, eps inside the square root, optional bias; it also saves the row mean and
// rstd so the backward reads x once instead of recomputing statistics (the reference recomputes
// them in double, Ops.cs:124-136). Optional fusions: gathering input rows by token id (the
// embedding lookup, TrainableDecisionModel.cs:277-285) and adding a per-row table vector after
// the norm (the type embedding, TrainableDecisionModel.cs:300-304).
//
// Backward restates Ops.LayerNormBackward (Ops.cs:117-186) in one pass: each wave writes dx for
// its rows and keeps dγ/dβ partials in registers for a fixed row stride; a second kernel sums the
// partials in wave order. Bytes per row: x, dy, dx in, dx out = 16·n.
#include "elementwise.hpp"

#include <mutex>

namespace laya {
namespace {

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ f32x4 ld4(const float* p) { return *reinterpret_cast<const f32x4*>(p); }
__device__ __forceinline__ void st4(float* p, f32x4 v) { *reinterpret_cast<f32x4*>(p) = v; }

// One wave's row of the forward; returns max|y| over the lane's elements (amax_bits).
template <int NCH>
__device__ __forceinline__ unsigned ln_fwd_row(const float* __restrict__ x, int row, int lane, int n,
                                               const float* __restrict__ w, const float* __restrict__ b, float eps,
                                               float* __restrict__ y, float* __restrict__ mean_out,
                                               float* __restrict__ rstd_out, const int* __restrict__ gather_ids,
                                               int gather_rows, const float* __restrict__ add_table,
                                               const int* __restrict__ add_index, __bf16* __restrict__ y16) {
    unsigned m = 0;
    const float* src = x + (long)row * n;
    bool zero = false;
    if (gather_ids) {
        const int id = gather_ids[row];
        zero = (unsigned)id >= (unsigned)gather_rows;
        src = x + (long)(zero ? 0 : id) * n;
    }
    // Issue every load of the row (x, γ, β, the added table row) before the reductions.
    const float* add = add_table ? add_table + (long)add_index[row] * n : nullptr;
    f32x4 v[NCH], gw[NCH], bw[NCH], aw[NCH];
#pragma unroll
    for (int c = 0; c < NCH; ++c) {
        const int col = (c * 64 + lane) * 4;
        v[c] = (col < n && !zero) ? ld4(src + col) : f32x4{0, 0, 0, 0};
        gw[c] = col < n ? ld4(w + col) : f32x4{0, 0, 0, 0};
        bw[c] = (col < n && b) ? ld4(b + col) : f32x4{0, 0, 0, 0};
        aw[c] = (col < n && add) ? ld4(add + col) : f32x4{0, 0, 0, 0};
    }
    float s = 0.0f;
#pragma unroll
    for (int c = 0; c < NCH; ++c) s += (v[c][0] + v[c][1]) + (v[c][2] + v[c][3]);
    const float mean = wave_sum(s) / (float)n;
    float q = 0.0f;
#pragma unroll
    for (int c = 0; c < NCH; ++c) {
        const int col = (c * 64 + lane) * 4;
        if (col < n) {
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const float d = v[c][e] - mean;
                q += d * d;
            }
        }
    }
    const float var = wave_sum(q) / (float)n;
    const float rstd = 1.0f / sqrtf(var + eps);
#pragma unroll
    for (int c = 0; c < NCH; ++c) {
        const int col = (c * 64 + lane) * 4;
        if (col < n) {
            f32x4 o = (v[c] - mean) * rstd * gw[c];
            if (b) o += bw[c];
            if (add) o += aw[c];
            st4(y + (long)row * n + col, o);
            if (y16) *reinterpret_cast<bf16x4*>(y16 + (long)row * n + col) = __builtin_convertvector(o, bf16x4);
            m = max(m, amax_bits4(o));
        }
    }
    if (lane == 0) {
        if (mean_out) mean_out[row] = mean;
        if (rstd_out) rstd_out[row] = rstd;
    }
    return m;
}

// Four rows per block, one wave each; amax (optional): max|y| folded in (the output's magnitude word).
template <int NCH>
__global__ __launch_bounds__(256) void ln_fwd_kernel(const float* __restrict__ x, int rows, int n,
                                                     const float* __restrict__ w, const float* __restrict__ b,
                                                     float eps, float* __restrict__ y, float* __restrict__ mean_out,
                                                     float* __restrict__ rstd_out, const int* __restrict__ gather_ids,
                                                     int gather_rows, const float* __restrict__ add_table,
                                                     const int* __restrict__ add_index, __bf16* __restrict__ y16,
                                                     unsigned* amax) {
    const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    const unsigned m = row < rows ? ln_fwd_row<NCH>(x, row, lane, n, w, b, eps, y, mean_out, rstd_out, gather_ids,
                                                    gather_rows, add_table, add_index, y16)
                                  : 0u;
    block_amax_fold(m, amax);
}

// One row's operands for the backward: x (gathered when ids are given), dy, and the dx it adds into.
template <int NCH>
__device__ __forceinline__ void ln_bwd_load(const float* __restrict__ x, const float* __restrict__ dy,
                                            const float* __restrict__ dx, int row, int n, int lane,
                                            const int* __restrict__ gather_ids, int gather_rows, f32x4 (&xv)[NCH],
                                            f32x4 (&gv)[NCH], f32x4 (&dv)[NCH]) {
    const float* src = x + (long)row * n;
    bool zero = false;
    if (gather_ids) {
        const int id = gather_ids[row];
        zero = (unsigned)id >= (unsigned)gather_rows;
        src = x + (long)(zero ? 0 : id) * n;
    }
#pragma unroll
    for (int c = 0; c < NCH; ++c) {
        const int col = (c * 64 + lane) * 4;
        xv[c] = (col < n && !zero) ? ld4(src + col) : f32x4{0, 0, 0, 0};
        gv[c] = col < n ? ld4(dy + (long)row * n + col) : f32x4{0, 0, 0, 0};
        dv[c] = col < n ? ld4(dx + (long)row * n + col) : f32x4{0, 0, 0, 0};
    }
}

// Rows up to 1024 wide (NCH ≤ 4) keep the next row's loads in flight while the current row computes.
template <int NCH>
__global__ __launch_bounds__(256) void ln_bwd_kernel(const float* __restrict__ x, int rows, int n,
                                                     const float* __restrict__ w, float eps,
                                                     const float* __restrict__ dy, float* __restrict__ dx,
                                                     const float* __restrict__ mean_in,
                                                     const float* __restrict__ rstd_in,
                                                     const int* __restrict__ gather_ids, int gather_rows,
                                                     int total_waves, float* __restrict__ part_g,
                                                     float* __restrict__ part_b, unsigned* amax) {
    // total_waves is a multiple of 4 (whole blocks); a wave past the last row only adds zeros.
    constexpr bool PIPE = NCH <= 4;
    const int wave = blockIdx.x * 4 + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    f32x4 gacc[NCH], bacc[NCH], gm[NCH];
#pragma unroll
    for (int c = 0; c < NCH; ++c) {
        gacc[c] = f32x4{0, 0, 0, 0};
        bacc[c] = f32x4{0, 0, 0, 0};
        const int col = (c * 64 + lane) * 4;
        gm[c] = col < n ? ld4(w + col) : f32x4{0, 0, 0, 0};
    }
    const float inv_n = 1.0f / (float)n;
    unsigned am = 0;  // max|dx| (amax_bits) of the lane's elements
    f32x4 xv[NCH], gv[NCH], dv[NCH];
    if (PIPE && wave < rows) ln_bwd_load<NCH>(x, dy, dx, wave, n, lane, gather_ids, gather_rows, xv, gv, dv);
    for (int row = wave; row < rows; row += total_waves) {
        f32x4 xn[NCH], gn[NCH], dn[NCH];
        const int next = row + total_waves;
        if (PIPE) {
            if (next < rows) ln_bwd_load<NCH>(x, dy, dx, next, n, lane, gather_ids, gather_rows, xn, gn, dn);
        } else {
            ln_bwd_load<NCH>(x, dy, dx, row, n, lane, gather_ids, gather_rows, xv, gv, dv);
        }
        float mean, rstd;
        if (mean_in) {
            mean = mean_in[row];
            rstd = rstd_in[row];
        } else {
            float s = 0.0f;
#pragma unroll
            for (int c = 0; c < NCH; ++c) s += (xv[c][0] + xv[c][1]) + (xv[c][2] + xv[c][3]);
            mean = wave_sum(s) * inv_n;
            float q = 0.0f;
#pragma unroll
            for (int c = 0; c < NCH; ++c) {
                const int col = (c * 64 + lane) * 4;
                if (col < n) {
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        const float d = xv[c][e] - mean;
                        q += d * d;
                    }
                }
            }
            rstd = 1.0f / sqrtf(wave_sum(q) * inv_n + eps);
        }
        float sg = 0.0f, sgx = 0.0f;
#pragma unroll
        for (int c = 0; c < NCH; ++c) {
            const int col = (c * 64 + lane) * 4;
            if (col < n) {
                const f32x4 xh = (xv[c] - mean) * rstd;
                const f32x4 g = gv[c] * gm[c];
                sg += (g[0] + g[1]) + (g[2] + g[3]);
                const f32x4 gx = g * xh;
                sgx += (gx[0] + gx[1]) + (gx[2] + gx[3]);
                gacc[c] += gv[c] * xh;
                bacc[c] += gv[c];
            }
        }
        const float mg = wave_sum(sg) * inv_n, mgx = wave_sum(sgx) * inv_n;
#pragma unroll
        for (int c = 0; c < NCH; ++c) {
            const int col = (c * 64 + lane) * 4;
            if (col < n) {
                const f32x4 xh = (xv[c] - mean) * rstd;
                const f32x4 o = dv[c] + rstd * (gv[c] * gm[c] - mg - xh * mgx);
                st4(dx + (long)row * n + col, o);
                am = max(am, amax_bits4(o));
            }
        }
        if (PIPE) {
#pragma unroll
            for (int c = 0; c < NCH; ++c) {
                xv[c] = xn[c];
                gv[c] = gn[c];
                dv[c] = dn[c];
            }
        }
    }
    block_amax_fold(am, amax);
    // The block's 4 waves combine their dγ/dβ partials in LDS (in wave order): one partial per block.
    if (!part_g && !part_b) return;
    extern __shared__ __attribute__((aligned(16))) float red[];  // [2][4][n]
    const int wv = threadIdx.x >> 6;
#pragma unroll
    for (int c = 0; c < NCH; ++c) {
        const int col = (c * 64 + lane) * 4;
        if (col < n) {
            st4(red + (long)wv * n + col, gacc[c]);
            st4(red + (long)(4 + wv) * n + col, bacc[c]);
        }
    }
    __syncthreads();
    for (int col = threadIdx.x; col < n; col += 256) {
        if (part_g) part_g[(long)blockIdx.x * n + col] = ((red[col] + red[n + col]) + red[2 * n + col]) + red[3 * n + col];
        if (part_b)
            part_b[(long)blockIdx.x * n + col] =
                ((red[4 * n + col] + red[5 * n + col]) + red[6 * n + col]) + red[7 * n + col];
    }
}

// out[c] += Σ_k part[k][c]: 16 groups of 64 columns each sum every 16th partial in order, then the
// group sums are added in group order, so the result is independent of timing.
constexpr int RED_COLS = 64, RED_GROUPS = 16;
__global__ __launch_bounds__(RED_COLS* RED_GROUPS) void partial_reduce_kernel(const float* __restrict__ part,
                                                                              int count, int n,
                                                                              float* __restrict__ out) {
    __shared__ float sums[RED_GROUPS][RED_COLS];
    const int lc = threadIdx.x % RED_COLS, g = threadIdx.x / RED_COLS;
    const int c = blockIdx.x * RED_COLS + lc;
    float s = 0.0f;
    if (c < n)
        for (int k = g; k < count; k += RED_GROUPS) s += part[(long)k * n + c];
    sums[g][lc] = s;
    __syncthreads();
    if (g == 0 && c < n) {
        float t = 0.0f;
        for (int k = 0; k < RED_GROUPS; ++k) t += sums[k][lc];
        out[c] += t;
    }
}

bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

// Blocks of four waves for a backward over `rows` rows: at most 2048 waves, rows dealt round-robin.
int ln_bwd_blocks(int rows) { return (std::min(rows, 2048) + 3) / 4; }

int chunks_for(int n) {
    LAYA_REQUIRE(n > 0 && n % 4 == 0, "layernorm: the row width must be a positive multiple of 4");
    const int nch = (n + 255) / 256;
    LAYA_REQUIRE(nch <= 8, "layernorm: rows wider than 2048 are not supported");
    return nch;
}

}  // namespace

void layernorm_fwd(laya_ctx* ctx, const float* x, int rows, int n, const float* w, const float* b, float eps, float* y,
                   float* mean, float* rstd, const int* gather_ids, const float* add_table, const int* add_index,
                   __bf16* y16, unsigned* amax) {
    if (rows <= 0) return;
    const int nch = chunks_for(n);
    // With gather_ids, x is a table of `gather_rows` rows; the caller validates ids on the host.
    const int gather_rows = gather_ids ? INT32_MAX : 0;
    dim3 grid((rows + 3) / 4), block(256);
    ProfileScope scope(ctx, "layernorm_fwd", 0.0, (8.0 * n + (y16 ? 2.0 * n : 0.0) + 8.0) * rows + 4.0 * n * (b ? 2 : 1));
#define LN_FWD(C)                                                                                                 \
    case C:                                                                                                       \
        LAYA_LAUNCH(ln_fwd_kernel<C>, grid, block, 0, ctx->stream, x, rows, n, w, b, eps, y, mean, rstd, \
                           gather_ids, gather_rows, add_table, add_index, y16, amax);                            \
        break;
    switch (nch) { LN_FWD(1) LN_FWD(2) LN_FWD(3) LN_FWD(4) LN_FWD(5) LN_FWD(6) LN_FWD(7) LN_FWD(8) }
#undef LN_FWD
    check_launch("ln_fwd_kernel");
}

// The backward with its dγ/dβ partials in `ws` (2·blocks·n floats, or null for the context's workspace).
// `profile`: bracket the launch for the live profile (events may be created on first use).
static void layernorm_bwd_impl(laya_ctx* ctx, const float* x, int rows, int n, const float* w, float eps,
                               const float* dy, float* dx, float* dgamma, float* dbeta, const float* mean,
                               const float* rstd, const int* gather_ids, float* ws, bool profile,
                               ColumnSumJobs* defer = nullptr, unsigned* amax = nullptr) {
    if (rows <= 0) return;
    const int nch = chunks_for(n);
    const int gather_rows = gather_ids ? INT32_MAX : 0;
    // A fixed row → wave assignment (wave w takes rows w, w + W, …) keeps dγ/dβ independent of timing.
    const int blocks = ln_bwd_blocks(rows);
    const int waves = 4 * blocks;
    float* pg = nullptr;
    float* pb = nullptr;
    if (dgamma || dbeta) {
        if (!ws) ws = static_cast<float*>(ctx->workspace(2, sizeof(float) * 2 * (size_t)blocks * n));
        if (dgamma) pg = ws;
        if (dbeta) pb = ws + (size_t)blocks * n;
    }
    const size_t lds = (pg || pb) ? sizeof(float) * 8 * (size_t)n : 0;
    dim3 grid(blocks), block(256);
    {
        ProfileScope scope(ctx, profile ? "layernorm_bwd" : nullptr, 0.0,
                           (16.0 * n + (mean ? 8.0 : 0.0)) * rows + 4.0 * n);
#define LN_BWD(C)                                                                                                \
    case C:                                                                                                      \
        LAYA_LAUNCH(ln_bwd_kernel<C>, grid, block, lds, ctx->stream, x, rows, n, w, eps, dy, dx, mean,  \
                           rstd, gather_ids, gather_rows, waves, pg, pb, amax);                                  \
        break;
        switch (nch) { LN_BWD(1) LN_BWD(2) LN_BWD(3) LN_BWD(4) LN_BWD(5) LN_BWD(6) LN_BWD(7) LN_BWD(8) }
#undef LN_BWD
        check_launch("ln_bwd_kernel");
    }
    if (n % 4 == 0) {  // the partials are 16-byte aligned (workspace and scratch); the parameter gradients may not be
        auto reduce = [&](float*& part, float* out) {
            if (!part || !aligned16(out)) return;
            if (defer) {
                if (defer->n == MAX_COLUMN_JOBS) {
                    column_reduce_batch(ctx, *defer);
                    defer->n = 0;
                }
                defer->job[defer->n++] = ColumnSumJob{part, out, blocks, n};
            } else {
                ProfileScope scope(ctx, profile ? "layernorm_bwd_reduce" : nullptr, 0.0, 4.0 * n * (blocks + 2.0));
                column_reduce(ctx, part, blocks, n, out);
            }
            part = nullptr;
        };
        reduce(pg, dgamma);
        reduce(pb, dbeta);
    }
    const dim3 rgrid((n + RED_COLS - 1) / RED_COLS), rblock(RED_COLS * RED_GROUPS);
    ProfileScope scope(ctx, (pg || pb) && profile ? "layernorm_bwd_reduce" : nullptr, 0.0,
                       4.0 * n * (blocks + 2.0) * ((pg ? 1 : 0) + (pb ? 1 : 0)));
    if (pg) {
        LAYA_LAUNCH(partial_reduce_kernel, rgrid, rblock, 0, ctx->stream, pg, blocks, n, dgamma);
        check_launch("partial_reduce_kernel");
    }
    if (pb) {
        LAYA_LAUNCH(partial_reduce_kernel, rgrid, rblock, 0, ctx->stream, pb, blocks, n, dbeta);
        check_launch("partial_reduce_kernel");
    }
}

void layernorm_bwd(laya_ctx* ctx, const float* x, int rows, int n, const float* w, float eps, const float* dy,
                   float* dx, float* dgamma, float* dbeta, const float* mean, const float* rstd,
                   const int* gather_ids, unsigned* amax) {
    layernorm_bwd_impl(ctx, x, rows, n, w, eps, dy, dx, dgamma, dbeta, mean, rstd, gather_ids, nullptr, true,
                       nullptr, amax);
}

int ln_bwd_partial_rows(int rows) { return ln_bwd_blocks(std::max(rows, 1)); }

void layernorm_bwd_deferred(laya_ctx* ctx, const float* x, int rows, int n, const float* w, float eps,
                            const float* dy, float* dx, float* dgamma, float* dbeta, const float* mean,
                            const float* rstd, const int* gather_ids, float* ws, ColumnSumJobs& jobs,
                            unsigned* amax) {
    LAYA_REQUIRE(ws != nullptr, "layernorm_bwd_deferred: no partial buffer");
    layernorm_bwd_impl(ctx, x, rows, n, w, eps, dy, dx, dgamma, dbeta, mean, rstd, gather_ids, ws, true, &jobs,
                       amax);
}

// ------------------------------------------------------------------ the allocation-free variant
//
// laya_layernorm_bwd_noalloc keeps its dγ/dβ partials in this file-scope device array instead of the
// context's workspace: at most 512 blocks × 2048 columns × (γ, β) floats, 8 MiB, which every GPU the
// library runs on holds until the process ends. The kernel writes every partial it later reads, so
// nothing in it needs clearing between calls; calls that overlap on one GPU (two streams) race on it.
constexpr size_t NOALLOC_SCRATCH_FLOATS = 2u * 512u * 2048u;
static __device__ __align__(256) float scratch[NOALLOC_SCRATCH_FLOATS];

namespace {
constexpr int NOALLOC_MAX_DEVICES = 64;
std::mutex g_scratch_mutex;
float* g_scratch_ptr[NOALLOC_MAX_DEVICES] = {};
}  // namespace

void noalloc_scratch_init(int device) {
    std::lock_guard<std::mutex> lock(g_scratch_mutex);
    LAYA_REQUIRE(device >= 0 && device < NOALLOC_MAX_DEVICES, "noalloc scratch: device index out of range");
    if (g_scratch_ptr[device]) return;
    void* p = nullptr;
    // The array's name is a host-side stand-in; its device address on the current device comes from here.
    LAYA_HIP(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
    g_scratch_ptr[device] = static_cast<float*>(p);
}

void layernorm_bwd_noalloc(laya_ctx* ctx, const float* x, int rows, int n, const float* w, float eps,
                           const float* dy, float* dx, float* dgamma, float* dbeta, const float* mean,
                           const float* rstd) {
    LAYA_REQUIRE(n > 0 && n <= 2048 && n % 4 == 0,
                 "layernorm_bwd_noalloc: the row width must be a multiple of 4 of at most 2048 (the partials of "
                 "its static scratch are sized for 512 blocks of 2048 columns)");
    float* ws = nullptr;
    {
        std::lock_guard<std::mutex> lock(g_scratch_mutex);
        ws = ctx->device >= 0 && ctx->device < NOALLOC_MAX_DEVICES ? g_scratch_ptr[ctx->device] : nullptr;
    }
    if (!ws) throw Error(LAYA_ERR_STATE, "layernorm_bwd_noalloc: the scratch address of this device is not set up");
    LAYA_REQUIRE(2 * (size_t)ln_bwd_blocks(rows) * n <= NOALLOC_SCRATCH_FLOATS,
                 "layernorm_bwd_noalloc: partials exceed the static scratch");
    layernorm_bwd_impl(ctx, x, rows, n, w, eps, dy, dx, dgamma, dbeta, mean, rstd, nullptr, ws, false);
}

}  // namespace laya
