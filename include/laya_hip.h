/* laya_hip.h — C-ABI of liblaya_hip.so, the MI355X (gfx950) fine-tuning library for the Laya
 * ModernBERT decision model.
 *
 * The reference has no FFI: its swap point is the C# op surface `internal static class Ops`
 * (src/StructuredDecisions.Laya.Training/Ops.cs:17), plus `AdamW.Step` (AdamW.cs:29) and
 * `Gradients.ClipByGlobalNorm` (AdamW.cs:103). Each entry point below replaces one of those
 * methods (cited beside it) and keeps its argument meaning and its accumulate/overwrite
 * convention (Ops.cs:12-15): a forward writes its output; laya_linear_bwd OVERWRITES dx; every
 * other backward ADDS into its input gradient; parameter gradients always ACCUMULATE.
 *
 * Conventions of this ABI:
 *  - Every function returns an int status (LAYA_OK = 0); laya_last_error() gives a thread-local
 *    message for the last failure on the calling thread.
 *  - Tensor arguments are DEVICE pointers (from laya_alloc) to row-major fp32 data unless noted;
 *    sizes are element counts. Index tables (ids, rows, positions) are device int32 arrays; a segment
 *    list is a laya_segments handle made from host arrays.
 *  - Calls are ordered on the context's single HIP stream and asynchronous until laya_sync().
 *    A context is not re-entrant; separate contexts are independent.
 *  - Results do not depend on launch configuration: no floating-point atomics; every reduction
 *    over rows runs in a fixed order.
 */
#ifndef LAYA_HIP_H
#define LAYA_HIP_H
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Status codes. The C# binding rethrows them as the reference's exception types. */
#define LAYA_OK 0
#define LAYA_ERR_ARGUMENT 1     /* ArgumentException (size mismatch, PackedMatrix.cs:124-126) */
#define LAYA_ERR_OUT_OF_RANGE 2 /* ArgumentOutOfRangeException (token id, TrainableDecisionModel.cs:281) */
#define LAYA_ERR_MEMORY 3       /* out of device memory, or over the context's allocation cap */
#define LAYA_ERR_HIP 4          /* a HIP runtime error */
#define LAYA_ERR_NOT_FINITE 5   /* a non-finite gradient norm */
#define LAYA_ERR_STATE 6        /* call order (backward with no tape) */
#define LAYA_ERR_MISSING 7      /* InvalidDataException: missing tensor (TrainableDecisionModel.cs:184-186) */

typedef struct laya_ctx laya_ctx;
typedef struct laya_rotary laya_rotary;
typedef struct laya_segments laya_segments;
typedef struct laya_model laya_model;

const char* laya_last_error(void);
const char* laya_version(void);

/* ---------------------------------------------------------------- context, memory, stream */
int laya_ctx_create(int device, laya_ctx** out);
int laya_ctx_destroy(laya_ctx* ctx);
/* Caps the bytes laya_alloc may hold (0 = no cap); an allocation over it fails with LAYA_ERR_MEMORY. */
int laya_ctx_set_memory_cap(laya_ctx* ctx, size_t bytes);
/* Precision of the matrix products launched on the context afterwards (linear layers and the model's
 * projections; the elementwise kernels stay fp32), per product class. An fp32 class (the
 * default) is computed on the 16-bit matrix cores with fp32 accumulation and fp32 results as accurate as
 * the fp32 matrix-core path (within 1e-6 relative L2 of the fp64 product on every tested shape): the
 * 256-wide kernels (the large products) split each operand, scaled by a power of two taken from its
 * largest finite magnitude, into two fp16 pieces and add three piece products per fp32 product; the
 * other kernels split each operand exactly into three bf16 pieces and add six piece products. The
 * operand-wide scale bounds the two-piece products' accuracy row by row: an output row whose operand row
 * lies 2^-k below the operand's largest keeps ≈ 2^(k-39) relative error (fp32 itself: 2^-24), so rows
 * within 2^15 of the largest are fp32-accurate, rows 2^20 below it carry ≈ 2e-6, and rows below 2^-39 of it
 * lose their precision. A caller whose rows span more selects LAYA_MATMUL_SPLIT3_* for that class; the
 * model's backward does so by itself when the items' logit gradients span more than 2^14
 * (laya_model_backward_fallback).
 * LAYA_MATMUL_SPLIT3_* keeps a class on the three-piece splits everywhere; LAYA_MATMUL_FP32_MFMA selects
 * the fp32 matrix cores instead. A bf16 class rounds both operands
 * to bf16 (nearest even) as they are staged and multiplies on the bf16 matrix cores with fp32
 * accumulation and fp32 outputs: the mixed-precision mode (bf16 weights and activations in the
 * products, fp32 master weights, gradients and statistics). Attention's products (head_dim 64) use the
 * same fp32-accurate split products under every policy except LAYA_MATMUL_FP32_MFMA, which keeps them on
 * the fp32 matrix cores; attention never drops to bf16. No counterpart in the reference, whose products are
 * all fp32 (PackedMatrixBf16, PackedMatrixBf16.cs:7-21, only stores weights in bf16 and widens them to fp32
 * before multiplying). */
enum {
    LAYA_MATMUL_FP32 = 0,             /* fp32-accurate products (the default), from bf16 pieces (below) */
    LAYA_MATMUL_BF16_FORWARD = 1,     /* y = x·Wᵀ (and the fused RoPE projection) */
    LAYA_MATMUL_BF16_INPUT_GRAD = 2,  /* dx = dy·W */
    LAYA_MATMUL_BF16_WEIGHT_GRAD = 4, /* dW += dyᵀ·x */
    LAYA_MATMUL_BF16 = 7,             /* every product */
    LAYA_MATMUL_FP32_MFMA = 8,        /* the fp32 classes on v_mfma_f32_32x32x2_f32 instead */
    LAYA_MATMUL_SPLIT3_FORWARD = 16,  /* per class: an fp32 class on three-piece bf16 splits in every */
    LAYA_MATMUL_SPLIT3_INPUT_GRAD = 32,  /*   kernel (no two-piece fp16 products); the backward pair */
    LAYA_MATMUL_SPLIT3_WEIGHT_GRAD = 64, /*   takes them unless both of its classes allow them */
    LAYA_MATMUL_SPLIT3_ATTENTION = 128, /* attention's products on three-piece bf16 splits */
    LAYA_MATMUL_FP32_SPLIT3 = 240,    /* every fp32 product (attention's too) on three-piece bf16 splits */
    LAYA_MATMUL_SPLIT_ALL = 7
};
int laya_ctx_set_matmul_precision(laya_ctx* ctx, int precision);
int laya_ctx_memory_in_use(laya_ctx* ctx, size_t* bytes);
int laya_alloc(laya_ctx* ctx, size_t bytes, void** out);
int laya_free(laya_ctx* ctx, void* ptr);
int laya_upload(laya_ctx* ctx, void* dst, const void* src_host, size_t bytes);
int laya_download(laya_ctx* ctx, void* dst_host, const void* src, size_t bytes);
int laya_fill(laya_ctx* ctx, float* dst, float value, size_t count);
int laya_sync(laya_ctx* ctx);
/* Stage timers: laya_timer_begin/end bracket stream work with HIP events; elapsed in ms. */
int laya_timer_begin(laya_ctx* ctx, int slot);
int laya_timer_end(laya_ctx* ctx, int slot);
int laya_timer_elapsed(laya_ctx* ctx, int slot, float* ms);

/* Live kernel profile: while enabled, every launch is bracketed by HIP events on the context's
 * stream and tagged with its algorithmic work (flops for matrix-core kernels, compulsory HBM bytes
 * for memory-bound ones). laya_profile_summary aggregates per kernel name, after a sync. */
int laya_profile_begin(laya_ctx* ctx);
int laya_profile_end(laya_ctx* ctx);
int laya_profile_count(laya_ctx* ctx, int* kernels);
int laya_profile_get(laya_ctx* ctx, int i, const char** name, int* launches, double* total_ms, double* flops,
                     double* bytes);

/* ---------------------------------------------------------------------------- ops (Ops.cs) */

/* Ops.Linear (Ops.cs:22-27): y[rows,out] = x[rows,in] · W[out,in]ᵀ (+ b[out]) (+ residual[rows,out]).
 * b and residual may be NULL; residual may alias y (the skip add of TrainableDecisionModel.cs:384, 401). */
int laya_linear_fwd(laya_ctx* ctx, const float* x, int rows, int in, const float* W, int out, const float* b,
                    const float* residual, float* y);

/* Ops.LinearBackward (Ops.cs:33-69): dx = dy·W (OVERWRITE; skipped when dx is NULL),
 * dW += dyᵀ·x and db += Σ_rows dy (each skipped when NULL). */
int laya_linear_bwd(laya_ctx* ctx, const float* x, const float* dy, int rows, int in, int out, const float* W,
                    float* dx, float* dW, float* db);

/* Ops.LayerNorm (Ops.cs:103-110; SimdOps.cs:234-272): torch LayerNorm, biased variance, eps inside
 * the square root, b may be NULL. mean/rstd (may be NULL) receive the row statistics. */
int laya_layernorm_fwd(laya_ctx* ctx, const float* x, int rows, int n, const float* w, const float* b, float eps,
                       float* y, float* mean, float* rstd);

/* Ops.LayerNormBackward (Ops.cs:117-186): dx += rstd·(g − mean(g) − x̂·mean(g·x̂)), g = dy·γ;
 * dgamma += Σ dy·x̂; dbeta += Σ dy (each may be NULL). mean/rstd from laya_layernorm_fwd, or NULL to
 * recompute them from x. */
int laya_layernorm_bwd(laya_ctx* ctx, const float* x, int rows, int n, const float* w, float eps, const float* dy,
                       float* dx, float* dgamma, float* dbeta, const float* mean, const float* rstd);

/* laya_layernorm_bwd with no allocation. No counterpart in the reference: for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc). Same arguments, results bit-identical to laya_layernorm_bwd; its dγ/dβ partials live in a
 * static device array of 8 MiB (512 blocks × 2048 columns × 2 floats) that each GPU holds until the
 * process ends, so n is limited to a multiple of 4 of at most 2048 (rows unlimited). Calls that overlap
 * on one GPU (two contexts or streams at once) race on that array. */
int laya_layernorm_bwd_noalloc(laya_ctx* ctx, const float* x, int rows, int n, const float* w, float eps,
                               const float* dy, float* dx, float* dgamma, float* dbeta, const float* mean,
                               const float* rstd);

/* SimdOps.Gelu (SimdOps.cs:305-323), exact erf GELU: y = gelu(x). y may alias x. */
int laya_gelu_fwd(laya_ctx* ctx, const float* x, size_t n, float* y);
/* Ops.GeluBackward (Ops.cs:194-218): grad *= Φ(u) + u·φ(u) (in place). */
int laya_gelu_bwd(laya_ctx* ctx, const float* u, float* grad, size_t n);

/* GeGLU (TrainableDecisionModel.cs:390-398): act[t,i] = gelu(wide[t,i]) · wide[t,I+i], halves [input | gate]. */
int laya_geglu_fwd(laya_ctx* ctx, const float* wide, int rows, int inter, float* act);
/* GeGLU backward (TrainableDecisionModel.cs:564-579): dwide = [dact·gate·gelu'(input) | dact·gelu(input)] (overwrite). */
int laya_geglu_bwd(laya_ctx* ctx, const float* wide, const float* dact, int rows, int inter, float* dwide);

/* Ops.Uniform / Ops.Mix (Ops.cs:227-241): host-side counter RNG, bit-identical to the device kernels. */
float laya_uniform(uint64_t seed, uint64_t index);
uint64_t laya_mix(uint64_t seed, uint64_t salt);
/* Ops.Dropout (Ops.cs:244-258): in place, x·keep/(1−p) with keep = Uniform(seed, i) ≥ p; its own backward. */
int laya_dropout(laya_ctx* ctx, float* values, size_t n, float p, uint64_t seed);
/* Head FFN activation (TrainableDecisionModel.cs:449-451): dropped = Dropout(ReLU(wide)). */
int laya_relu_dropout_fwd(laya_ctx* ctx, const float* wide, size_t n, float p, uint64_t seed, float* dropped);
/* Its backward (TrainableDecisionModel.cs:620-624): grad = Dropout(grad), then 0 where wide ≤ 0 (in place). */
int laya_relu_dropout_bwd(laya_ctx* ctx, const float* wide, float* grad, size_t n, float p, uint64_t seed);
/* SimdOps.Add (SimdOps.cs:84-93): dst += src. */
int laya_add(laya_ctx* ctx, float* dst, const float* src, size_t n);

/* Rotary (Ops.cs:446-504): cos/sin tables built in double and rounded to float, θ_i = θ^(−2i/d). */
int laya_rotary_create(laya_ctx* ctx, int head_dim, double theta, int positions, laya_rotary** out);
int laya_rotary_destroy(laya_ctx* ctx, laya_rotary* rot);
/* Rotary.Apply (Ops.cs:489-503) on rows of [rows, head_dim] at positions pos[rows] (device int32). */
int laya_rotary_apply(laya_ctx* ctx, const laya_rotary* rot, float* vec, int rows, const int* pos, int inverse);

/* The segment list a batch's attention calls share (ModernBertEncoder.cs:30-33: Segment(Start, Length);
 * TrainableDecisionModel.cs:254-264 builds it once per batch and passes it to every AttentionForward and
 * AttentionBackward). start/length are HOST arrays [nseg]: they are validated, copied to the device once,
 * and kept on the host so attention calls size their launches without reading the device back. */
int laya_segments_create(laya_ctx* ctx, const int* start, const int* length, int nseg, laya_segments** out);
int laya_segments_destroy(laya_ctx* ctx, laya_segments* segs);

/* Ops.AttentionForward (Ops.cs:275-277, 329-366): multi-head attention per segment over qkv rows
 * [q | k | v] (head slice at head·d_h), RoPE with segment-local positions (rot NULL: none), window
 * [t − w, t + w] clipped to the segment (half_window < 0: none), softmax(scale·qkᵀ), prob-dropout p
 * with the counter RNG at index head<<42 | row<<21 | key (Ops.cs:318). lse [rows·heads] receives the
 * row log-sum-exp (base 2, of the scaled scores) the backward can reuse. Asynchronous. */
int laya_attention_fwd(laya_ctx* ctx, const float* qkv, const laya_segments* segs, int hidden, int heads, float scale,
                       int half_window, const laya_rotary* rot, float p_drop, uint64_t seed, float* context,
                       float* lse);
/* Ops.AttentionBackward (Ops.cs:280-282, 368-438): dq, dk, dv WRITTEN (not added) into dqkv, with
 * inverse RoPE on dq and dk. context and lse from laya_attention_fwd, or both NULL (the reference's
 * signature carries neither): the row statistics are then recomputed, as Ops.AttentionBackward
 * recomputes each row's softmax (Ops.cs:390-394). Asynchronous. */
int laya_attention_bwd(laya_ctx* ctx, const float* qkv, const laya_segments* segs, int hidden, int heads, float scale,
                       int half_window, const laya_rotary* rot, float p_drop, uint64_t seed, const float* context,
                       const float* lse, const float* dcontext, float* dqkv);

/* Embedding gather (TrainableDecisionModel.cs:277-283): out[t] = E[ids[t]]; ids are checked on the
 * device: an id outside [0, vocab) writes zeros and sets *bad_count (device int32, may be NULL). */
int laya_embedding_fwd(laya_ctx* ctx, const int* ids, int n, const float* E, int vocab, int hidden, float* out,
                       int* bad_count);
/* Deterministic scatter plan on the host: token positions stably sorted by id, the unique ids and
 * their run offsets (offsets has n_unique + 1 entries). */
int laya_embedding_plan(const int* ids, int n, int vocab, int* sorted_pos, int* unique_ids, int* offsets,
                        int* n_unique);
/* Embedding-gradient scatter (TrainableDecisionModel.cs:543-547): grad[id] += Σ d[t] over that id's
 * tokens, in token order. Plan arrays are device copies of laya_embedding_plan's output. */
int laya_embedding_bwd(laya_ctx* ctx, const int* sorted_pos, const int* unique_ids, const int* offsets, int n_unique,
                       const float* d, int hidden, float* grad);

/* Marker gather (TrainableDecisionModel.cs:315) and scatter-add (500-504), in marker order. */
int laya_gather_rows(laya_ctx* ctx, const float* src, const int* rows_idx, int n, int width, float* dst);
int laya_scatter_add_rows(laya_ctx* ctx, const float* src, const int* rows_idx, int n, int width, float* dst);

/* Type embedding (TrainableDecisionModel.cs:300-304): states[r] += table[qtype_of_row[r]] for every row (the
 * item's question type repeated over its rows, device int32 in [0, 3)); width a multiple of 4. */
int laya_type_embedding_fwd(laya_ctx* ctx, float* states, const int* qtype_of_row, int rows, int width,
                            const float* table);
/* Its gradient (TrainableDecisionModel.cs:512-521): grad[q] += Σ dstates[r] over the rows of type q, each
 * type's rows summed in a fixed order (deterministic); grad is [3, width], width a multiple of 4. */
int laya_type_embedding_bwd(laya_ctx* ctx, const float* dstates, const int* qtype_of_row, int rows, int width,
                            float* grad);

/* Soft cross-entropy gradient of RlcdObjective (RlcdObjective.cs:139-148, 150), policy term off:
 * g_o = ce_weight·(p_o·Σt − t_o)/n_items·scale with p = softmax(logits). Device arrays; options
 * concatenated, option_offsets[n_items + 1]. loss (device, may be NULL) receives the cross-entropy. */
int laya_softmax_ce_bwd(laya_ctx* ctx, const float* logits, const float* targets, const int* option_offsets,
                        int n_items, float ce_weight, float scale, float* grad, float* loss);

/* RlcdObjective.Compute (RlcdObjective.cs:57-155) with supplied draws, all operands on the device:
 * option_offsets [n_items + 1] and qtypes [n_items] (int), logits / targets [total_options], draws
 * [groups][total_options] (double); grad [total_options] = ∂loss/∂logit · scale; losses [4] (double):
 * total, policy, cross-entropy, mean reward. max_options (≤ 64) bounds any item's option count.
 * groups = 0 is the cross-entropy-only objective (no draws read; mean reward NaN, as 0/0 in the reference). */
int laya_rlcd_objective(laya_ctx* ctx, const float* logits, const float* targets, const int* option_offsets,
                        const int* qtypes, int n_items, int total_options, int max_options, int groups,
                        const double* draws, double sigma, double spherical_weight, double rps_weight,
                        double ce_weight, double scale, float* grad, double* losses);

/* Gradients.ClipByGlobalNorm (AdamW.cs:103-130) over a flat arena: Σg² in double, in a fixed order.
 * Writes the norm (double) and the clip coefficient (float, 1 when not clipping) to device memory.
 * A NaN or infinite norm leaves the coefficient at 1, as the reference does (its `coefficient < 1`
 * test is false for NaN), and raises the context's non-finite flag, which laya_grad_norm_status reads. */
int laya_grad_norm(laya_ctx* ctx, const float* grads, size_t n, double max_norm, double* norm_out, float* coef_out);
/* Synchronises and returns LAYA_ERR_NOT_FINITE when the last laya_grad_norm on the context met a NaN or
 * infinite gradient, LAYA_OK otherwise (LAYA_ERR_STATE before any laya_grad_norm). The reference has no such
 * check (AdamW.cs:122-128 lets a NaN norm through); this is the detection its callers lack. */
int laya_grad_norm_status(laya_ctx* ctx);
/* Multi-tensor AdamW (AdamW.cs:29-73) over a flat arena split into parameter groups:
 * element i of group g (ranges [begin[g], end[g])) uses lr[g]; g_i is scaled by *coef (device, may be
 * NULL = 1) as the clip does; zero_grads clears the gradient after it is read. */
int laya_adamw(laya_ctx* ctx, float* params, float* grads, float* m, float* v, int n_groups, const size_t* begin,
               const size_t* end, const double* lr, double beta1, double beta2, double eps, double weight_decay,
               int step, const float* coef, int zero_grads);

/* ---------------------------------------------- operand magnitude words (per-op binding state)
 *
 * No counterpart in the reference: state a binding may keep beside its device buffers, as it keeps
 * attention's context and LSE (the `Ops` signatures stay as they are). The fp32-accurate products split
 * each operand into two fp16 pieces scaled by a power of two from the operand's largest finite magnitude;
 * an entry point above measures each operand with a pass over it. A magnitude word group is
 * LAYA_AMAX_WORDS uint32 words of device memory (laya_alloc). The _w variants below, each the entry point of
 * the same name with the same meaning otherwise, fill an output's group (cleared first) with the largest
 * finite magnitude of what they write, and take an input's group in place of measuring that input. A group
 * describes its buffer as the call that filled it left it: a binding passes it while nothing else has
 * written the buffer since, and NULL (measure) otherwise. A NULL output group is not written. */
#define LAYA_AMAX_WORDS 1024
/* Fills `words` (cleared first) with max|x| over the finite elements of x[n]. */
int laya_amax(laya_ctx* ctx, const float* x, size_t n, unsigned* words);
int laya_linear_fwd_w(laya_ctx* ctx, const float* x, int rows, int in, const float* W, int out, const float* b,
                      const float* residual, float* y, const unsigned* x_words, const unsigned* W_words,
                      unsigned* y_words);
int laya_linear_bwd_w(laya_ctx* ctx, const float* x, const float* dy, int rows, int in, int out, const float* W,
                      float* dx, float* dW, float* db, const unsigned* x_words, const unsigned* dy_words,
                      const unsigned* W_words, unsigned* dx_words);
int laya_layernorm_fwd_w(laya_ctx* ctx, const float* x, int rows, int n, const float* w, const float* b, float eps,
                         float* y, float* mean, float* rstd, unsigned* y_words);
/* dx_words: of dx as written (laya_layernorm_bwd adds into dx). */
int laya_layernorm_bwd_w(laya_ctx* ctx, const float* x, int rows, int n, const float* w, float eps, const float* dy,
                         float* dx, float* dgamma, float* dbeta, const float* mean, const float* rstd,
                         unsigned* dx_words);
int laya_geglu_fwd_w(laya_ctx* ctx, const float* wide, int rows, int inter, float* act, unsigned* act_words);
int laya_geglu_bwd_w(laya_ctx* ctx, const float* wide, const float* dact, int rows, int inter, float* dwide,
                     unsigned* dwide_words);
/* qkv_words: of qkv as stored (unused when a rotary table makes the kernels read a rotated copy, which
 * measures itself as it is written). */
int laya_attention_fwd_w(laya_ctx* ctx, const float* qkv, const laya_segments* segs, int hidden, int heads,
                         float scale, int half_window, const laya_rotary* rot, float p_drop, uint64_t seed,
                         float* context, float* lse, const unsigned* qkv_words, unsigned* context_words);
int laya_attention_bwd_w(laya_ctx* ctx, const float* qkv, const laya_segments* segs, int hidden, int heads,
                         float scale, int half_window, const laya_rotary* rot, float p_drop, uint64_t seed,
                         const float* context, const float* lse, const float* dcontext, float* dqkv,
                         const unsigned* qkv_words, const unsigned* dcontext_words, unsigned* dqkv_words);

/* ---------------------------------------------- model (TrainableDecisionModel.cs, Trainer.cs) */

typedef struct {
    int vocab, hidden, intermediate, layers, heads;
    int local_attention;    /* full sliding window (ModernBertConfig.cs:51: a token sees ±local_attention/2) */
    int global_every;       /* when layer_kinds is NULL: layer l is global iff l % global_every == 0 */
    const int* layer_kinds; /* host [layers]: 0 global, 1 sliding; may be NULL */
    double theta_global, theta_local;
    float norm_eps;
    int norm_bias, attention_bias, mlp_bias;
    int head_layers, head_ff, n_act;
} laya_model_config;

typedef struct {
    int n_items;
    const int* lengths;   /* host [n_items] */
    const int* tokens;    /* host [Σ lengths], concatenated with no padding */
    const int* n_options; /* host [n_items] */
    const int* markers;   /* host [Σ n_options], positions inside each item */
    const int* qtypes;    /* host [n_items]: 0 choice, 1 score, 2 noul */
} laya_batch;

/* TrainableDecisionModel constructor (TrainableDecisionModel.cs:105-182). Parameters live in one
 * device arena in module order; names follow the checkpoint's state-dict names. */
int laya_model_create(laya_ctx* ctx, const laya_model_config* cfg, laya_model** out);
int laya_model_destroy(laya_model* model);
int laya_model_num_params(laya_model* model, int* count);
int laya_model_param_info(laya_model* model, int i, const char** name, int* ndim, int* dims /* [4] */,
                          size_t* offset, size_t* numel, int* trainable);
int laya_model_find_param(laya_model* model, const char* name, int* index);
int laya_model_set_param(laya_model* model, int i, const float* host);
int laya_model_get_param(laya_model* model, int i, float* host);
int laya_model_get_grad(laya_model* model, int i, float* host);
int laya_model_has_grad(laya_model* model, int i, int* has);
/* Inspection of the last forward's saved head feed-forward activations (no counterpart in the reference, whose
 * HeadLayerBackward recomputes them, TrainableDecisionModel.cs:605-624): the device address and float count
 * ([tokens × head_ff]) of head layer `layer`'s linear1 output (which = 0, the ReLU's input) or of its
 * ReLU-dropout output (which = 1, whose sign is the mask the backward applies). Valid until the next forward;
 * LAYA_ERR_STATE before any forward. Tests use it to compare ReLU decisions with the oracle's. */
int laya_model_head_activation(laya_model* model, int layer, int which, float** device, size_t* count);
/* Synthetic init: matrices and embeddings N(0, std) from the counter RNG, norm weights 1, biases 0. */
int laya_model_init_random(laya_model* model, uint64_t seed, float std);
/* SetTrainableEncoderLayers (TrainableDecisionModel.cs:206-231); n < 0 trains everything. */
int laya_model_set_trainable_encoder_layers(laya_model* model, int n);
int laya_model_set_head_dropout(laya_model* model, float p);
/* Layer checkpointing (TrainableDecisionModel.cs:61-64: the reference checkpoints every layer, always):
 * mode 0 keeps every encoder layer's activations resident from forward to backward; 1 keeps only each
 * layer's input and recomputes the layer's internals just before its backward, as the reference does
 * (the two head layers stay resident); 2 (the default) keeps everything when the activation arena fits
 * under the context's memory cap and the device's free memory, and recomputes otherwise. Gradients are
 * bitwise the same in every mode. A change takes effect at the next forward. */
int laya_model_set_layer_checkpointing(laya_model* model, int mode);
/* The mode, and whether the current arena recomputes (0 before the first forward). Either may be NULL. */
int laya_model_layer_checkpointing(laya_model* model, int* mode, int* recomputing);
/* bf16 copies for the bf16 products (PackedMatrixBf16, src/StructuredDecisions.Base/Numerics/
 * PackedMatrixBf16.cs:7-21, keeps weights as bf16 for its products; here the fp32 arenas stay the masters).
 * While the context's precision policy has bf16 products (laya_ctx_set_matmul_precision), the model keeps
 * bf16(weights), updated by the AdamW step with each update, and bf16 copies of the saved activations the
 * products read (written by the kernels that produce them); the products read those copies instead of
 * rounding fp32 operands on their way into LDS — the same values, half the bytes. on = 1 (default) keeps
 * them, 0 drops them (less memory). Results are the same either way. Takes effect at the next forward. */
int laya_model_set_bf16_copies(laya_model* model, int on);
/* bf16 weights, as PackedMatrixBf16 holds a projection weight (src/StructuredDecisions.Base/Numerics/
 * PackedMatrixBf16.cs:7-21: a bf16 weight widened exactly to fp32 inside an fp32 product): with on = 1 every
 * matrix product (the encoder's, head's and scorer's linears, forward and input gradient) reads each weight
 * rounded to bf16 (nearest even) and widened back to fp32, under whatever precision policy the context sets
 * for the product itself; activations, embeddings, norms and biases stay fp32, and the fp32 arena stays the
 * master that AdamW updates (the rounded copy follows each update and each host write). Weight gradients are
 * those of the rounded weights. Off (0) by default. Takes effect at the next forward. */
int laya_model_set_bf16_weights(laya_model* model, int on);
/* Parameter i's bf16 copy (numel uint16, the bf16 bit patterns); LAYA_ERR_STATE when no current copy exists. */
int laya_model_get_param_bf16(laya_model* model, int i, uint16_t* host);
/* Forward (TrainableDecisionModel.cs:248-353). Keeps what the backward needs resident in HBM (all of it,
 * or the encoder layers' inputs under layer checkpointing). logits_host (may be NULL) receives
 * Σ n_options floats and synchronises. */
int laya_model_forward(laya_model* model, const laya_batch* batch, int training, uint64_t seed, float* logits_host);
/* DecisionModel.ReadOut (src/StructuredDecisions.Laya/Models/DecisionModel.cs:170-226) for every item of
 * the last forward, on the device: the option logits (logits_host, Σ n_options floats, may be NULL), the
 * action probabilities act_probs_host [n_items][n_act] from the act head on [h[start], top1, top1 − top2,
 * normalised entropy, K/255], and those four calibration features (features_host [n_items][4], may be
 * NULL). DecisionModel.Forward's outputs for a batch = laya_model_forward (training 0) + this. Synchronises. */
int laya_model_readout(laya_model* model, float* logits_host, float* act_probs_host, float* features_host);
/* Backward (TrainableDecisionModel.cs:479-549): dlogits_host has Σ n_options floats. */
int laya_model_backward(laya_model* model, const float* dlogits_host);
/* Whether the last backward ran its products (linears and attention) on three-piece bf16 splits instead of the
 * two-piece fp16 products the precision policy selects: it does when the items' largest |dL/dlogit| span more
 * than 2^14. Every activation-gradient row of an item scales with that item's logit gradients, and a two-piece
 * product scales its operand from the operand's largest magnitude, so rows far below it would keep less than
 * fp32's relative precision; the three-piece pieces carry fp32's exponent range. (No counterpart in the
 * reference, whose fp32 products have no operand scale.) */
int laya_model_backward_fallback(laya_model* model, int* split3);
/* Gradients.ClipByGlobalNorm (AdamW.cs:103-130); norm_out (may be NULL) synchronises, and then a NaN or
 * infinite norm returns LAYA_ERR_NOT_FINITE (norm_out still written, gradients left unscaled as the
 * reference leaves them). */
int laya_model_clip_grad_norm(laya_model* model, double max_norm, double* norm_out);
/* Synchronises and returns LAYA_ERR_NOT_FINITE when the model's last gradient norm (its clip, or the clip
 * inside laya_model_train_step[_staged]) was not finite; LAYA_ERR_STATE before any. No counterpart in the
 * reference, which does not detect non-finite gradients (AdamW.cs:122-128). */
int laya_model_grad_norm_status(laya_model* model);
/* AdamW.Step (AdamW.cs:29-73) with the trainer's groups (Trainer.cs:96-100): "encoder." parameters at
 * lr_encoder, the rest at lr_head. Applies the clip coefficient of the last clip, if any. */
int laya_model_adamw_step(laya_model* model, double lr_encoder, double lr_head, double beta1, double beta2,
                          double eps, double weight_decay);
int laya_model_zero_grad(laya_model* model);
/* One full optimizer step (Trainer.cs:131-144 with GradAccum = 1): forward, soft cross-entropy
 * gradient on the device (targets_host: Σ n_options floats), backward, clip, AdamW, zero grads.
 * Synchronises only when loss_out is non-NULL. */
int laya_model_train_step(laya_model* model, const laya_batch* batch, const float* targets_host, float ce_weight,
                          float loss_scale, uint64_t seed, double max_norm, double lr_encoder, double lr_head,
                          double beta1, double beta2, double eps, double weight_decay, float* loss_out);
int laya_model_steps(laya_model* model, int* steps);
/* Adam moments of parameter i (numel floats each; zeros before the first step) and the step count
 * that drives bias correction. No counterpart in the reference, whose trainer cannot resume (TODO.md:74):
 * the moments are what a checkpoint needs beyond the weights (AdamW.cs:24 keeps them per parameter). */
int laya_model_get_moments(laya_model* model, int i, float* m1_host, float* m2_host);
int laya_model_set_moments(laya_model* model, int i, const float* m1_host, const float* m2_host);
int laya_model_set_steps(laya_model* model, int steps);

/* RlcdObjective.Compute on the last forward's logits (RlcdObjective.cs:57-155, as Trainer.cs:134-136 calls it),
 * with the standard-normal draws supplied as in its second overload: targets_host [Σ n_options], draws_host
 * [groups][Σ n_options] (double). The scaled logit gradient stays on the device for
 * laya_model_backward_from_objective; losses_host [4] = total, policy, cross-entropy, mean reward (may be
 * NULL; non-NULL synchronises). At most 64 options per item; groups = 0 drops the policy term. */
int laya_model_objective_rlcd(laya_model* model, const float* targets_host, const double* draws_host, int groups,
                              double sigma, double spherical_weight, double rps_weight, double ce_weight,
                              double scale, double* losses_host);
/* TrainableDecisionModel.Backward (TrainableDecisionModel.cs:479-549) from the logit gradient the last
 * objective left on the device (no host round trip). */
int laya_model_backward_from_objective(laya_model* model);

/* Device-resident batches. No counterpart in the reference, whose batches are host arrays: these split
 * laya_model_train_step's host work (validation, layout, embedding-gradient plan, uploads) from the
 * step, so a caller that prepares batches ahead (a data loader, a benchmark) runs steps on inputs
 * already in HBM. stage_batch validates exactly as train_step does, uploads the batch and its targets
 * once and returns a slot; train_step_staged is train_step on that slot; release_batch frees it. */
int laya_model_stage_batch(laya_model* model, const laya_batch* batch, const float* targets_host, int* slot);
int laya_model_train_step_staged(laya_model* model, int slot, float ce_weight, float loss_scale, uint64_t seed,
                                 double max_norm, double lr_encoder, double lr_head, double beta1, double beta2,
                                 double eps, double weight_decay, float* loss_out);
int laya_model_release_batch(laya_model* model, int slot);

#ifdef __cplusplus
}
#endif
#endif
