// Launchers of the memory-bound kernels (elementwise.hip) and the optimizer kernels (optim.hip).
#pragma once
#include "common.hpp"

namespace laya {

void fill(laya_ctx* ctx, float* dst, float v, size_t n);
void add(laya_ctx* ctx, float* dst, const float* src, size_t n);
void scale(laya_ctx* ctx, float* dst, float s, size_t n);
void gelu_fwd(laya_ctx* ctx, const float* x, size_t n, float* y);
void gelu_bwd(laya_ctx* ctx, const float* u, float* g, size_t n);
// The optional __bf16* outputs are copies rounded to nearest even, for the bf16 products that read them;
// the optional unsigned* amax outputs fold max|output| into a magnitude word (absmax_into).
void geglu_fwd(laya_ctx* ctx, const float* wide, int rows, int inter, float* act, __bf16* act16 = nullptr,
               unsigned* amax = nullptr);
void to_bf16(laya_ctx* ctx, const float* src, size_t n, __bf16* dst);
// dst = float(bf16(src)) (round to nearest even; the widening back to fp32 is exact). dst may alias src.
void round_bf16(laya_ctx* ctx, const float* src, size_t n, float* dst);
void geglu_bwd(laya_ctx* ctx, const float* wide, const float* dact, int rows, int inter, float* dwide,
               unsigned* amax = nullptr);
void dropout(laya_ctx* ctx, float* v, size_t n, float p, uint64_t seed);
// v = Dropout(v) + r (one pass where the arrays allow float4 access).
void dropout_add(laya_ctx* ctx, float* v, const float* r, size_t n, float p, uint64_t seed);
// dst = Dropout(src) out of place (one pass).
void dropout_copy(laya_ctx* ctx, const float* src, float* dst, size_t n, float p, uint64_t seed);
void relu_dropout_fwd(laya_ctx* ctx, const float* wide, size_t n, float p, uint64_t seed, float* dropped,
                      __bf16* dropped16 = nullptr, unsigned* amax = nullptr);
void relu_dropout_bwd(laya_ctx* ctx, const float* wide, float* g, size_t n, float p, uint64_t seed);
void rotary_apply(laya_ctx* ctx, const float* cos_t, const float* sin_t, int head_dim, float* vec, int rows,
                  const int* pos, int inverse);
void embedding_fwd(laya_ctx* ctx, const int* ids, int n, const float* E, int vocab, int hidden, float* out, int* bad);
void embedding_bwd(laya_ctx* ctx, const int* sorted_pos, const int* unique_ids, const int* offsets, int n_unique,
                   const float* d, int hidden, float* grad);
void gather_rows(laya_ctx* ctx, const float* src, const int* rows, int n, int width, float* dst);
void scatter_add_rows(laya_ctx* ctx, const float* src, const int* rows, int n, int width, float* dst);
// grad[type] += Σ over rows r with row_type[r] == type of d[r] (TrainableDecisionModel.cs:512-521).
void type_embedding_bwd(laya_ctx* ctx, const float* d, const int* row_type, int rows, int width, float* grad);
// dst[r] += table[idx[r]] for rows r of width floats (the type embedding's add).
void add_indexed_rows(laya_ctx* ctx, float* dst, const int* idx, int rows, int width, const float* table);
// ReLU + dropout backward from the forward's output (positive exactly where the gradient passes).
void relu_dropout_bwd_from_output(laya_ctx* ctx, const float* dropped, float* g, size_t n, float p,
                                  unsigned* amax = nullptr);
// out[type·n + c] += Σ rows of x[r][c] (per row type when row_type is given; types 1 or 3), in a fixed
// order, through workspace `slot`; n % 4 == 0, 16-byte aligned.
void column_sums(laya_ctx* ctx, const float* x, int rows, int n, const int* row_type, int types, float* out, int slot,
                 unsigned* amax = nullptr);
// out[c] += Σ_k part[k][c] for count partial rows of width n, in a fixed order.
void column_reduce(laya_ctx* ctx, const float* part, int count, int n, float* out);
// Several column reductions out[c] += Σ_k part[k][c] in one launch (each in column_reduce's order).
void column_reduce_batch(laya_ctx* ctx, const ColumnSumJobs& jobs);
void softmax_ce_bwd(laya_ctx* ctx, const float* logits, const float* targets, const int* offsets, int n_items,
                    float ce_weight, float scale, float* grad, float* loss);
void init_param(laya_ctx* ctx, float* dst, size_t n, int kind, float std, uint64_t seed);

// Σ g² over the arena in double, in a fixed order; writes norm, the clip coefficient
// min(1, max/(norm + 1e-6)) as the reference computes it, and a non-finite flag.
void grad_norm(laya_ctx* ctx, const float* g, size_t n, double max_norm, double* norm, float* coef, int* nonfinite);

struct AdamGroups {
    int n;
    size_t begin[4], end[4];
    float decay[4], step_size[4];
};
// Elements outside every group are left alone (frozen parameters); zero_grads clears all n gradients;
// mirror (optional, n bf16) receives bf16(p) of every updated element.
// The weights whose magnitude words the AdamW kernel folds the updated values into, so the next forward need
// not measure them: tensor t spans float4s [begin[t], end[t]) of the arena (sorted, disjoint) and folds into
// the word group at words + word[t]·AMAX_GROUP (cleared beforehand). block[b] says which tensor covers
// workgroup b's 256 float4s whole (-1: none, -2: several or part of one: each lane looks its tensor up).
struct AdamFold {
    const int* block = nullptr;
    const long* begin = nullptr;
    const long* end = nullptr;
    const int* word = nullptr;
    int n = 0;
    unsigned* words = nullptr;
};
void adamw_arena(laya_ctx* ctx, float* p, float* g, float* m, float* v, size_t n, const AdamGroups& groups,
                 float beta1, float beta2, float eps, float sqrt_c2, const float* coef, int zero_grads,
                 __bf16* mirror = nullptr, const AdamFold* fold = nullptr);

}  // namespace laya
