/* Oracle C-ABI (test infrastructure only).
 *
 * A CPU restatement of the reference's C# fine-tuning path
 * (src/StructuredDecisions.Laya.Training/{Ops,TrainableDecisionModel,AdamW,RlcdObjective}.cs and
 * src/StructuredDecisions.Base/Numerics/SimdOps.cs), compiled twice over the same templates:
 * fp32 (what the reference computes) and fp64 (the mathematical pin). Only the tests, the smoke
 * check and the CPU-baseline leg of the benchmark load it; the product library never does.
 */
#ifndef LAYA_ORACLE_H
#define LAYA_ORACLE_H
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct {
    int vocab, hidden, intermediate, layers, heads;
    int local_attention;        /* full sliding window; a token sees [t - w/2, t + w/2] */
    int global_every;           /* layer kind when layer_kinds is NULL: l % n == 0 is global */
    const int* layer_kinds;     /* per layer: 0 global, 1 sliding; may be NULL */
    double theta_global, theta_local;
    float norm_eps;
    int norm_bias, attention_bias, mlp_bias;
    int head_layers, head_ff, n_act;
} orc_config;

const char* orc_last_error(void);

/* ---- model (TrainableDecisionModel.cs) */
void* orc_model_create(const orc_config* cfg, int use_double);
void orc_model_destroy(void* model);
int orc_model_num_params(void* model);
const char* orc_model_param_name(void* model, int i);
int orc_model_param_ndim(void* model, int i);
int orc_model_param_dim(void* model, int i, int d);
long orc_model_param_numel(void* model, int i);
int orc_model_param_trainable(void* model, int i);
int orc_model_has_grad(void* model, int i);
int orc_model_set_param(void* model, int i, const float* data);
int orc_model_get_param(void* model, int i, double* out);
int orc_model_get_grad(void* model, int i, double* out);
void orc_model_set_trainable_encoder_layers(void* model, int n); /* n < 0: everything trains */
void orc_model_set_head_dropout(void* model, float p);
int orc_model_forward(void* model, int n_items, const int* lengths, const int* tokens, const int* n_options,
                      const int* markers, const int* qtypes, int training, int keep_tape, uint64_t seed,
                      double* logits_out);
int orc_model_backward(void* model, const float* dlogits);
/* DecisionModel.ReadOut on the last forward: act_probs [n_items][n_act], features [n_items][4]
 * (top1, top1 − top2, normalised entropy, K/255), pooled [n_items][d] (may be NULL). */
int orc_model_readout(void* model, float* act_probs, float* features, double* pooled);
/* OpenMP threads for the calls that follow (n > 0); returns the previous maximum. */
int orc_set_threads(int n);
void orc_model_zero_grad(void* model);
double orc_model_clip(void* model, double max_norm);
void orc_model_adamw(void* model, double lr_encoder, double lr_head, double beta1, double beta2, double eps,
                     double weight_decay);
int orc_model_steps(void* model);
/* Diagnostics: keep each head layer's linear1 output (the ReLU's input) of every later forward, in double;
 * orc_model_head_preactivation copies layer `layer`'s [tokens × head_ff] values (out may be NULL) and
 * returns their count, or -1 when none was kept. */
void orc_model_set_capture_head(void* model, int on);
long orc_model_head_preactivation(void* model, int layer, double* out);

/* ---- ops (Ops.cs, SimdOps.cs), fp32 (_f32) and fp64 (_f64) */
float orc_uniform(uint64_t seed, uint64_t index);
uint64_t orc_mix(uint64_t seed, uint64_t salt);
float orc_exp_f32(float x);
float orc_erf_f32(float x);

#define ORC_DECLARE_OPS(R, S)                                                                                   \
    void orc_gemm_##S(int M, int N, int K, const R* A, long sam, long sak, const R* B, long sbk, long sbn, R* C, \
                      long ldc, int accumulate);                                                                \
    void orc_linear_##S(const R* x, int rows, int in, const R* W, int out, const R* b, R* y);                   \
    void orc_linear_backward_##S(const R* x, const R* dy, int rows, int in, int out, const R* W, R* dx, R* dW,  \
                                 R* db);                                                                        \
    void orc_layernorm_##S(const R* x, int rows, int n, const R* w, const R* b, float eps, R* y);               \
    void orc_layernorm_backward_##S(const R* x, int rows, int n, const R* w, float eps, const R* dy, R* dx,     \
                                    R* dgamma, R* dbeta);                                                       \
    void orc_gelu_##S(R* x, long n);                                                                            \
    void orc_gelu_backward_##S(const R* u, R* grad, long n);                                                    \
    void orc_geglu_##S(const R* wide, int rows, int inter, R* act);                                             \
    void orc_geglu_backward_##S(const R* wide, const R* dact, int rows, int inter, R* dwide);                   \
    void orc_dropout_##S(R* values, long n, float p, uint64_t seed);                                            \
    void orc_rotary_apply_##S(double theta, int head_dim, R* vec, int position, int inverse);                   \
    void orc_attention_forward_##S(const R* qkv, int nseg, const int* seg_start, const int* seg_len, int hidden, \
                                   int heads, float scale, int half_window, double theta, float dropout,        \
                                   uint64_t seed, R* context);                                                  \
    void orc_attention_backward_##S(const R* qkv, int nseg, const int* seg_start, const int* seg_len,           \
                                    int hidden, int heads, float scale, int half_window, double theta,          \
                                    float dropout, uint64_t seed, const R* dcontext, R* dqkv);                  \
    void orc_adamw_tensor_##S(R* p, const R* g, R* m, R* v, long n, double lr, double beta1, double beta2,      \
                              double eps, double weight_decay, int step);

ORC_DECLARE_OPS(float, f32)
ORC_DECLARE_OPS(double, f64)

double orc_clip_f32(int n, float** grads, const long* lens, double max_norm);

/* ---- objective (RlcdObjective.cs) */
/* Soft cross-entropy term only (groups = 0). Returns the cross-entropy; grads per option concatenated. */
double orc_cross_entropy(int n_items, const int* n_options, const float* logits, const float* targets,
                         double ce_weight, double scale, float* grad_out);
/* The full objective with supplied standard-normal draws [group][item][option] (concatenated). */
int orc_rlcd(int n_items, const int* n_options, const int* qtypes, const float* logits, const float* targets,
             int groups, const double* draws, double sigma, double spherical_weight, double rps_weight,
             double ce_weight, double scale, float* grad_out, double* loss_out /* [loss, policy, ce, reward] */);
double orc_proper_reward(int n, const float* reported, const float* target, int qtype, double spherical_weight,
                         double rps_weight);

#ifdef __cplusplus
}
#endif
#endif
