// The model driver: TrainableDecisionModel (src/StructuredDecisions.Laya.Training/TrainableDecisionModel.cs),
// AdamW / Gradients (AdamW.cs) and the trainer's micro-step (Trainer.cs:125-154), restated as host C++ over
// the library's kernels.
//
// What changes from the reference, MI355X-first:
//  - parameters, gradients and both Adam moments live in four flat fp32 arenas in HBM, in module
//    order, so the optimizer and the norm are single launches over contiguous memory;
//  - the forward keeps every activation the backward needs resident in HBM (about 0.85 MB per token
//    for 22 layers at d = 768) instead of checkpointing each layer's input and recomputing it, which
//    removes the reference's extra forward pass (TrainableDecisionModel.cs:551-557, 605-612);
//  - LayerNorm statistics are saved by the forward, attention saves its row log-sum-exp;
//  - the skip adds are fused into the epilogue of the GEMM that produces the branch.
// The order of operations, the accumulate/overwrite conventions and every parity trap of the
// reference are kept: layer 0 has no attn_norm, the head uses ReLU and biased norms with eps 1e-5,
// the act head gets no gradient but is weight-decayed, the temperature buffer is frozen.
#include <algorithm>
#include <cmath>
#include <cstring>
#include <map>
#include <memory>
#include <vector>

#include "elementwise.hpp"

namespace laya {
void build_rotary(laya_ctx* ctx, laya_rotary* r, int head_dim, double theta, int positions);
void free_rotary(laya_ctx* ctx, laya_rotary* r);
}  // namespace laya

using namespace laya;

namespace {

enum InitKind { INIT_NORMAL = 0, INIT_ONES = 1, INIT_ZEROS = 2 };

struct Param {
    std::string name;
    std::vector<int> shape;
    size_t offset = 0, numel = 0;
    bool trainable = true, touched = false;
    int init = INIT_NORMAL;
};

// Carves one device allocation into 256-byte aligned tensors.
struct Carver {
    size_t bytes = 0;
    std::vector<std::pair<void**, size_t>> slots;
    void add(float*& p, size_t floats) { add_bytes(reinterpret_cast<void**>(&p), floats * sizeof(float)); }
    void add(__bf16*& p, size_t n) { add_bytes(reinterpret_cast<void**>(&p), n * sizeof(__bf16)); }
    void add_bytes(void** p, size_t b) {
        slots.push_back({p, bytes});
        bytes += (b + 255) / 256 * 256;
    }
    void bind(char* base) {
        for (auto& s : slots) *s.first = base + s.second;
    }
};

}  // namespace

// The device int32 tables of one batch (TrainableDecisionModel.cs:254-274 layout).
struct BatchTables {
    int *tokens, *seg_start, *seg_len, *row_type, *marker_rows, *qtypes, *opt_off, *sorted, *unique, *uoff, *pos,
        *blocks;
};

// A batch planned on the host and uploaded once, ahead of the steps that use it.
struct StagedBatch {
    int T = 0, nseg = 0, nmark = 0, max_len = 0, n_unique = 0, max_opts = 0, n_blocks = 0;
    double keys_full = 0, keys_local = 0;
    std::vector<int> opt_off;  // host copy: item i's options are logits [opt_off[i], opt_off[i + 1])
    void* block = nullptr;  // the tables, then the soft-CE targets
    BatchTables tables{};
    float* targets = nullptr;
};

// Host-side layout of one batch: every table the kernels read, before upload.
struct BatchPlan {
    int T = 0, nseg = 0, nmark = 0, max_len = 0, n_unique = 0, max_opts = 0, n_blocks = 0;
    double keys_full = 0, keys_local = 0;
    std::vector<int> tokens, start, len, marker_rows, qtypes, opt_off, row_type, sorted, unique, uoff, pos, blocks;
};

// The int tables of one batch inside a Carver, sized for Tz tokens, Mc markers and Sc items.
struct TableCarve {
    float *tok, *ps, *st, *ln, *rt, *mr, *qt, *oo, *so, *un, *uo, *bl;
    void add(Carver& cv, size_t Tz, size_t Mc, size_t Sc) {
        cv.add(tok, Tz);
        cv.add(ps, Tz);
        cv.add(st, Sc);
        cv.add(ln, Sc);
        cv.add(rt, Tz);
        cv.add(mr, Mc);
        cv.add(qt, Sc);
        cv.add(oo, Sc + 1);
        cv.add(so, Tz);
        cv.add(un, Tz + 1);
        cv.add(uo, Tz + 2);
        cv.add(bl, Tz / laya::ATTENTION_BLOCK_ROWS + Sc + 1);  // Σ ⌈len / rows⌉ ≤ tokens / rows + segments
    }
    BatchTables bind() const {
        auto i = [](float* p) { return reinterpret_cast<int*>(p); };
        return {i(tok), i(st), i(ln), i(rt), i(mr), i(qt), i(oo), i(so), i(un), i(uo), i(ps), i(bl)};
    }
};

struct laya_model {
    laya_ctx* ctx = nullptr;
    laya_model_config cfg{};
    std::vector<int> kinds;
    std::vector<Param> params;
    std::map<std::string, int> by_name;
    size_t total = 0;
    float* P = nullptr;
    float* G = nullptr;
    float* M1 = nullptr;
    float* M2 = nullptr;
    laya_rotary rot_global, rot_local;
    int head_heads = 1, head_dim = 0;
    float head_dropout = 0.1f;
    int first_trainable = 0;
    bool embeddings_trainable = true;
    int steps = 0;

    struct Enc {
        int attn_norm = -1, attn_norm_b = -1, wqkv, wqkv_b = -1, wo, wo_b = -1, mlp_norm, mlp_norm_b = -1, wi,
            wi_b = -1, mlp_wo, mlp_wo_b = -1, kind;
    };
    struct Head {
        int norm1, norm1_b, in_proj, in_proj_b, out_proj, out_proj_b, norm2, norm2_b, linear1, linear1_b, linear2,
            linear2_b;
    };
    std::vector<Enc> enc;
    std::vector<Head> head;
    int tok_emb, emb_norm, emb_norm_b = -1, final_norm, final_norm_b = -1, type_emb, sc_norm, sc_norm_b, sc1, sc1_b,
        sc2, sc2_b;

    // ----- activations (capacity-sized, reused across steps)
    int cap_tokens = 0, cap_markers = 0, cap_segs = 0;
    // Layer checkpointing (TrainableDecisionModel.cs:61-64): 0 keeps every encoder layer's activations,
    // 1 keeps only each layer's input and recomputes the layer before its backward, 2 (the default) does
    // that only when keeping everything would not fit (the context's cap, or the device's memory).
    int checkpoint_mode = 2;
    bool recompute = false;  // the arena's current layout
    // bf16 copies for the bf16 products (a bf16 precision policy): the fp32 arenas stay the masters; WB is
    // bf16(P), refreshed from P when stale and written by AdamW with each update; the activation arena then
    // also holds bf16 copies of the saved activations the products read (written by their producers). A
    // product reads a copy instead of rounding its fp32 operand on the way into LDS: the same values.
    bool bf16_copies = true;   // the option (laya_model_set_bf16_copies)
    bool copies = false;       // the activation arena's current layout has the copies
    __bf16* WB = nullptr;
    bool wb_fresh = false;
    // bf16 weights (laya_model_set_bf16_weights): the products read PW, each weight rounded to bf16 and widened
    // back to fp32 (exact), refreshed from the fp32 masters P when a host write or an update left it stale.
    bool bf16_weights = false;
    float* PW = nullptr;
    bool pw_fresh = false;
    void* act_block = nullptr;
    struct EncAct {
        float *x, *normed, *mean1, *rstd1, *qkv, *ctx, *lse, *res, *mlpn, *mean2, *rstd2, *wide, *act;
        __bf16 *normed16, *ctx16, *mlpn16, *act16;  // layer 0: normed16 = bf16(x), its QKV input
    };
    struct HeadAct {
        float *x, *n1, *mean1, *rstd1, *qkv, *ctx, *lse, *res, *n2, *mean2, *rstd2, *wide, *drop;
        __bf16 *n1_16, *ctx16, *n2_16, *drop16;
    };
    std::vector<EncAct> ea;
    std::vector<HeadAct> ha;
    float *x_final = nullptr, *emb_mean = nullptr, *emb_rstd = nullptr, *fin_mean = nullptr, *fin_rstd = nullptr;
    float *head_out = nullptr;
    float *s_in = nullptr, *s_mean = nullptr, *s_rstd = nullptr, *s_norm = nullptr, *s_pre = nullptr, *s_act = nullptr,
          *scores = nullptr;
    // backward scratch
    float *dS = nullptr, *dE = nullptr, *dqkv = nullptr, *dctx = nullptr, *dwide = nullptr, *dact = nullptr,
          *dn = nullptr, *dy = nullptr;
    float *ds_scores = nullptr, *ds_act = nullptr, *ds_norm = nullptr, *ds_mark = nullptr, *targets = nullptr;
    // batch tables (device int32): `own` lives in the activation block and takes uploads of batches
    // passed by value; `cur` is what the kernels read (own, or a staged batch's tables)
    BatchTables own{}, cur{};
    std::vector<StagedBatch> staged;  // laya_model_stage_batch slots; a null block marks a free slot
    // The current batch's option offsets on the host, and the logit gradients of the last backward read back
    // for the range check below.
    std::vector<int> opt_off_host;
    std::vector<float> dl_host;
    // The last backward ran its products on three-piece splits because the items' logit gradients spanned more
    // than BACKWARD_RANGE (laya_model_backward_fallback).
    bool backward_split3 = false;
    // LayerNorm dγ/dβ partials of one backward (a slice per LayerNorm) and their deferred reductions, run
    // as one launch at the end of the backward
    float* ln_part = nullptr;
    size_t ln_part_cap = 0, ln_part_used = 0;
    ColumnSumJobs ln_jobs;
    // optimizer scalars
    double* d_norm = nullptr;
    float* d_coef = nullptr;
    float* d_loss = nullptr;
    int* d_nonfinite = nullptr;
    bool coef_valid = false;
    bool norm_done = false;  // a gradient norm has been computed (d_nonfinite holds its flag)

    // max|operand| words of the two-piece fp16 products: one per parameter, one per product site for its
    // input (four per encoder layer: the QKV, Wo, Wi and MLP-output inputs; four per head layer; two for
    // the scorer; plus each attention's qkv), and one per site for its output gradient (plus each
    // attention's context gradient); the host flags say which hold the current values. The weight and input words are cleared at each forward (a weight is measured once per step,
    // an input once per forward and reused by its backward product), the gradient words at each backward.
    unsigned* amax_words = nullptr;
    std::vector<unsigned char> amax_known;
    // The products' weights, measured together once per forward (absmax_multi): per block the arena
    // offset, length and parameter index (device), and the parameter indices.
    long* wm_off = nullptr;
    int* wm_len = nullptr;
    int* wm_word = nullptr;
    int wm_blocks = 0;
    double wm_bytes = 0;
    std::vector<int> wm_params;
    // AdamW's fold of the updated weights' magnitudes (laya::AdamFold): the device tables, and the trainable
    // flags they were made for (empty: not made).
    int* fold_block = nullptr;
    long* fold_begin = nullptr;
    long* fold_end = nullptr;
    int* fold_word = nullptr;
    int fold_n = 0;
    std::vector<int> fold_params;  // the parameter index of each folded tensor
    std::vector<unsigned char> fold_for;
    size_t amax_sites() const { return (size_t)scorer_site(2); }
    laya::AmaxRef word(size_t k) {
        return amax_words ? laya::AmaxRef{amax_words + k * laya::AMAX_GROUP, &amax_known[k]} : laya::AmaxRef{};
    }
    // A weight's word; with bf16 weights the products read PW, whose values are bf16 values.
    laya::AmaxRef wref(int i) {
        if (i < 0) return laya::AmaxRef{};
        laya::AmaxRef r = word(i);
        r.bf16 = bf16_weights && PW && r.word;
        return r;
    }
    laya::AmaxRef aref(int site) { return word(params.size() + site); }
    laya::AmaxRef dref(int site) { return word(params.size() + amax_sites() + site); }
    // The word a producing kernel folds its output into, when a product of the classes `bits` will read it
    // as two-piece products (else null: no fold); the word counts as measured from then on.
    unsigned* produce(laya::AmaxRef r, int bits) {
        if (!r.word || !(ctx->matmul_pair & bits)) return nullptr;
        *r.known = 1;
        return r.word;
    }
    // The same for attention's operands (qkv, the context gradient), read as two-piece products.
    unsigned* produce_attention(laya::AmaxRef r) {
        if (!r.word || !ctx->attention_pair) return nullptr;
        *r.known = 1;
        return r.word;
    }
    // Five sites per layer: k = 0 … 3 the four products (their inputs' words, and in the backward their
    // output gradients'), k = 4 attention (qkv's word, and in the backward the context gradient's).
    int enc_site(int l, int k) const { return 5 * l + k; }
    int head_site(int j, int k) const { return 5 * cfg.layers + 5 * j + k; }
    int scorer_site(int k) const { return 5 * cfg.layers + 5 * cfg.head_layers + k; }

    // ----- the batch of the last forward
    bool has_tape = false, training = false;
    uint64_t seed = 0;
    int T = 0, nseg = 0, nmark = 0, max_len = 0, n_unique = 0, max_opts = 0;
    int n_blocks = 0;  // entries of the current batch's attention block list
    double keys_full = 0, keys_local = 0;  // Σ_q attended keys of the batch, full and sliding window
    // RLCD objective: the draws of the last call (device, grown on demand) and its losses
    double* d_draws = nullptr;
    size_t draws_cap = 0;
    double* d_rlcd_losses = nullptr;

    int d() const { return cfg.hidden; }
    int I() const { return cfg.intermediate; }

    int add_param(const std::string& name, std::vector<int> shape, int init) {
        Param p;
        p.name = name;
        p.shape = std::move(shape);
        p.numel = 1;
        for (int s : p.shape) p.numel *= (size_t)s;
        p.offset = total;
        p.init = init;
        total += (p.numel + 63) / 64 * 64;  // 256-byte aligned tensors for vector loads
        by_name[name] = (int)params.size();
        params.push_back(p);
        return (int)params.size() - 1;
    }

    float* W(int i) const { return i >= 0 ? P + params[i].offset : nullptr; }
    // The weight matrix a product reads: the master, or its bf16 rounding under bf16 weights.
    const float* PWt(int i) const { return i >= 0 ? (bf16_weights && PW ? PW : P) + params[i].offset : nullptr; }
    // The bf16 copy of parameter i when the products read copies (else null: they round W themselves).
    const __bf16* W16(int i) const { return i >= 0 && copies && WB && wb_fresh ? WB + params[i].offset : nullptr; }
    int find(const std::string& name) const {
        auto it = by_name.find(name);
        if (it == by_name.end()) throw laya::Error(LAYA_ERR_MISSING, "the model has no '" + name + "' tensor");
        return it->second;
    }
    // Parameter.GradientBuffer (Parameter.cs:177): the gradient of a trainable parameter, else null.
    float* Gt(int i) {
        if (i < 0 || !params[i].trainable) return nullptr;
        params[i].touched = true;
        return G + params[i].offset;
    }
};

namespace {

void build_layout(laya_model* m) {
    const auto& c = m->cfg;
    const int d = c.hidden, I = c.intermediate;
    const std::string e = "encoder.";
    m->tok_emb = m->add_param(e + "embeddings.tok_embeddings.weight", {c.vocab, d}, INIT_NORMAL);
    m->emb_norm = m->add_param(e + "embeddings.norm.weight", {d}, INIT_ONES);
    if (c.norm_bias) m->emb_norm_b = m->add_param(e + "embeddings.norm.bias", {d}, INIT_ZEROS);
    for (int l = 0; l < c.layers; ++l) {
        const std::string p = e + "layers." + std::to_string(l) + ".";
        laya_model::Enc L;
        if (l > 0) {
            L.attn_norm = m->add_param(p + "attn_norm.weight", {d}, INIT_ONES);
            if (c.norm_bias) L.attn_norm_b = m->add_param(p + "attn_norm.bias", {d}, INIT_ZEROS);
        }
        L.wqkv = m->add_param(p + "attn.Wqkv.weight", {3 * d, d}, INIT_NORMAL);
        if (c.attention_bias) L.wqkv_b = m->add_param(p + "attn.Wqkv.bias", {3 * d}, INIT_ZEROS);
        L.wo = m->add_param(p + "attn.Wo.weight", {d, d}, INIT_NORMAL);
        if (c.attention_bias) L.wo_b = m->add_param(p + "attn.Wo.bias", {d}, INIT_ZEROS);
        L.mlp_norm = m->add_param(p + "mlp_norm.weight", {d}, INIT_ONES);
        if (c.norm_bias) L.mlp_norm_b = m->add_param(p + "mlp_norm.bias", {d}, INIT_ZEROS);
        L.wi = m->add_param(p + "mlp.Wi.weight", {2 * I, d}, INIT_NORMAL);
        if (c.mlp_bias) L.wi_b = m->add_param(p + "mlp.Wi.bias", {2 * I}, INIT_ZEROS);
        L.mlp_wo = m->add_param(p + "mlp.Wo.weight", {d, I}, INIT_NORMAL);
        if (c.mlp_bias) L.mlp_wo_b = m->add_param(p + "mlp.Wo.bias", {d}, INIT_ZEROS);
        L.kind = m->kinds[l];
        m->enc.push_back(L);
    }
    m->final_norm = m->add_param(e + "final_norm.weight", {d}, INIT_ONES);
    if (c.norm_bias) m->final_norm_b = m->add_param(e + "final_norm.bias", {d}, INIT_ZEROS);
    for (int l = 0; l < c.head_layers; ++l) {
        const std::string p = "head.layers." + std::to_string(l) + ".";
        laya_model::Head H;
        H.in_proj = m->add_param(p + "self_attn.in_proj_weight", {3 * d, d}, INIT_NORMAL);
        H.in_proj_b = m->add_param(p + "self_attn.in_proj_bias", {3 * d}, INIT_ZEROS);
        H.out_proj = m->add_param(p + "self_attn.out_proj.weight", {d, d}, INIT_NORMAL);
        H.out_proj_b = m->add_param(p + "self_attn.out_proj.bias", {d}, INIT_ZEROS);
        H.linear1 = m->add_param(p + "linear1.weight", {c.head_ff, d}, INIT_NORMAL);
        H.linear1_b = m->add_param(p + "linear1.bias", {c.head_ff}, INIT_ZEROS);
        H.linear2 = m->add_param(p + "linear2.weight", {d, c.head_ff}, INIT_NORMAL);
        H.linear2_b = m->add_param(p + "linear2.bias", {d}, INIT_ZEROS);
        H.norm1 = m->add_param(p + "norm1.weight", {d}, INIT_ONES);
        H.norm1_b = m->add_param(p + "norm1.bias", {d}, INIT_ZEROS);
        H.norm2 = m->add_param(p + "norm2.weight", {d}, INIT_ONES);
        H.norm2_b = m->add_param(p + "norm2.bias", {d}, INIT_ZEROS);
        m->head.push_back(H);
    }
    m->type_emb = m->add_param("type_emb.weight", {3, d}, INIT_NORMAL);
    m->sc_norm = m->add_param("scorer.0.weight", {d}, INIT_ONES);
    m->sc_norm_b = m->add_param("scorer.0.bias", {d}, INIT_ZEROS);
    m->sc1 = m->add_param("scorer.1.weight", {d, d}, INIT_NORMAL);
    m->sc1_b = m->add_param("scorer.1.bias", {d}, INIT_ZEROS);
    m->sc2 = m->add_param("scorer.3.weight", {1, d}, INIT_NORMAL);
    m->sc2_b = m->add_param("scorer.3.bias", {1}, INIT_ZEROS);
    m->add_param("act_head.0.weight", {256, d + 4}, INIT_NORMAL);
    m->add_param("act_head.0.bias", {256}, INIT_ZEROS);
    m->add_param("act_head.2.weight", {c.n_act, 256}, INIT_NORMAL);
    m->add_param("act_head.2.bias", {c.n_act}, INIT_ZEROS);
    const int temp = m->add_param("temperature", {3}, INIT_ONES);
    m->params[temp].trainable = false;  // a buffer, not a parameter (TrainableDecisionModel.cs:117-118)
}

void ensure_rotary(laya_model* m, int positions) {
    if (m->rot_global.positions >= positions && m->rot_global.cos_t) return;
    const int p = std::max(positions, std::max(1024, m->rot_global.positions * 2));
    const int hd = m->cfg.hidden / m->cfg.heads;
    build_rotary(m->ctx, &m->rot_global, hd, m->cfg.theta_global, p);
    build_rotary(m->ctx, &m->rot_local, hd, m->cfg.theta_local, p);
}

// The activation arena's layout for Tc tokens; with `recompute`, the encoder layers share one set of
// internal buffers and keep only their inputs.
Carver carve_activations(laya_model* m, size_t Tz, size_t Mc, bool recompute, bool copies) {
    const size_t d = m->d(), I = m->I(), ff = m->cfg.head_ff;
    const size_t H = m->cfg.heads, HH = m->head_heads;
    Carver cv;
    m->ea.assign(m->cfg.layers, {});
    for (size_t l = 0; l < m->ea.size(); ++l) {
        auto& a = m->ea[l];
        cv.add(a.x, Tz * d);
        if (recompute && l > 0) continue;  // internals shared with layer 0's (assigned after binding)
        cv.add(a.normed, Tz * d);
        cv.add(a.mean1, Tz);
        cv.add(a.rstd1, Tz);
        cv.add(a.qkv, Tz * 3 * d);
        cv.add(a.ctx, Tz * d);
        cv.add(a.lse, Tz * H);
        cv.add(a.res, Tz * d);
        cv.add(a.mlpn, Tz * d);
        cv.add(a.mean2, Tz);
        cv.add(a.rstd2, Tz);
        cv.add(a.wide, Tz * 2 * I);
        cv.add(a.act, Tz * I);
        if (copies) {
            cv.add(a.normed16, Tz * d);
            cv.add(a.ctx16, Tz * d);
            cv.add(a.mlpn16, Tz * d);
            cv.add(a.act16, Tz * I);
        }
    }
    m->ha.assign(m->cfg.head_layers, {});
    for (auto& a : m->ha) {
        cv.add(a.x, Tz * d);
        cv.add(a.n1, Tz * d);
        cv.add(a.mean1, Tz);
        cv.add(a.rstd1, Tz);
        cv.add(a.qkv, Tz * 3 * d);
        cv.add(a.ctx, Tz * d);
        cv.add(a.lse, Tz * HH);
        cv.add(a.res, Tz * d);
        cv.add(a.n2, Tz * d);
        cv.add(a.mean2, Tz);
        cv.add(a.rstd2, Tz);
        cv.add(a.wide, Tz * ff);
        cv.add(a.drop, Tz * ff);
        if (copies) {
            cv.add(a.n1_16, Tz * d);
            cv.add(a.ctx16, Tz * d);
            cv.add(a.n2_16, Tz * d);
            cv.add(a.drop16, Tz * ff);
        }
    }
    cv.add(m->x_final, Tz * d);
    cv.add(m->emb_mean, Tz);
    cv.add(m->emb_rstd, Tz);
    cv.add(m->fin_mean, Tz);
    cv.add(m->fin_rstd, Tz);
    cv.add(m->head_out, Tz * d);
    cv.add(m->s_in, (size_t)Mc * d);
    cv.add(m->s_mean, Mc);
    cv.add(m->s_rstd, Mc);
    cv.add(m->s_norm, (size_t)Mc * d);
    cv.add(m->s_pre, (size_t)Mc * d);
    cv.add(m->s_act, (size_t)Mc * d);
    cv.add(m->scores, Mc);
    cv.add(m->dS, Tz * d);
    cv.add(m->dE, Tz * d);
    cv.add(m->dqkv, Tz * 3 * d);
    cv.add(m->dctx, Tz * d);
    cv.add(m->dwide, Tz * std::max(2 * I, ff));
    cv.add(m->dact, Tz * std::max(I, ff));
    cv.add(m->dn, Tz * d);
    cv.add(m->dy, Tz * d);
    cv.add(m->ds_scores, Mc);
    cv.add(m->ds_act, (size_t)Mc * d);
    cv.add(m->ds_norm, (size_t)Mc * d);
    cv.add(m->ds_mark, (size_t)Mc * d);
    cv.add(m->targets, Mc);
    return cv;
}

void share_layer_internals(laya_model* m) {
    for (size_t l = 1; l < m->ea.size(); ++l) {
        float* x = m->ea[l].x;
        m->ea[l] = m->ea[0];
        m->ea[l].x = x;
    }
}

void ensure_activations(laya_model* m, int T, int nmark, int nseg) {
    const bool want_full = m->checkpoint_mode != 1;
    const bool copies = m->bf16_copies && m->ctx->matmul_bf16 != 0;
    const bool layout_ok = (m->checkpoint_mode == 2 || m->recompute == (m->checkpoint_mode == 1)) && m->copies == copies;
    if (T <= m->cap_tokens && nmark <= m->cap_markers && nseg <= m->cap_segs && m->act_block && layout_ok) return;
    m->has_tape = false;  // the activations of the last forward go with the old block
    if (m->act_block) {
        m->ctx->release(m->act_block);
        m->act_block = nullptr;
    }
    const int Tc = std::max(T, m->cap_tokens), Mc = std::max(std::max(nmark, m->cap_markers), 1),
              Sc = std::max(std::max(nseg, m->cap_segs), 1);
    bool recompute = !want_full;
    Carver cv = carve_activations(m, Tc, Mc, recompute, copies);
    TableCarve tc;
    tc.add(cv, Tc, Mc, Sc);
    if (m->checkpoint_mode == 2) {
        // Keep everything when it fits under the context's cap and the device's free memory, else recompute.
        size_t free_b = 0, total_b = 0;
        if (hipMemGetInfo(&free_b, &total_b) != hipSuccess) free_b = SIZE_MAX;
        const bool over_cap = m->ctx->cap && m->ctx->in_use + cv.bytes > m->ctx->cap;
        if (over_cap || cv.bytes + (64u << 20) > free_b) {
            recompute = true;
            cv = carve_activations(m, Tc, Mc, true, copies);
            tc = TableCarve{};
            tc.add(cv, Tc, Mc, Sc);
        }
    }
    m->act_block = m->ctx->alloc(cv.bytes);
    cv.bind(static_cast<char*>(m->act_block));
    if (recompute) share_layer_internals(m);
    m->recompute = recompute;
    m->copies = copies;
    m->own = tc.bind();
    m->cur = m->own;
    m->cap_tokens = Tc;
    m->cap_markers = Mc;
    m->cap_segs = Sc;
}

// The products' weights measured in one launch (their words cleared beforehand): the block tables are
// made on first use (the weights' layout never changes), 16,384 values per block.
void measure_weights(laya_model* m) {
    if (m->wm_params.empty()) {
        for (const auto& L : m->enc)
            for (int i : {L.wqkv, L.wo, L.wi, L.mlp_wo}) m->wm_params.push_back(i);
        for (const auto& H : m->head)
            for (int i : {H.in_proj, H.out_proj, H.linear1, H.linear2}) m->wm_params.push_back(i);
        for (int i : {m->sc1, m->sc2}) m->wm_params.push_back(i);
        std::vector<long> off;
        std::vector<int> len, word;
        constexpr long CHUNK = 16384;
        for (int i : m->wm_params) {
            const Param& p = m->params[i];
            for (long c = 0; c < (long)p.numel; c += CHUNK) {
                off.push_back((long)p.offset + c);
                len.push_back((int)std::min<long>(CHUNK, (long)p.numel - c));
                word.push_back(i);
            }
            m->wm_bytes += 4.0 * p.numel;
        }
        m->wm_blocks = (int)off.size();
        m->wm_off = static_cast<long*>(m->ctx->alloc(sizeof(long) * off.size()));
        m->wm_len = static_cast<int*>(m->ctx->alloc(sizeof(int) * len.size()));
        m->wm_word = static_cast<int*>(m->ctx->alloc(sizeof(int) * word.size()));
        LAYA_HIP(hipMemcpyAsync(m->wm_off, off.data(), sizeof(long) * off.size(), hipMemcpyHostToDevice, m->ctx->stream));
        LAYA_HIP(hipMemcpyAsync(m->wm_len, len.data(), sizeof(int) * len.size(), hipMemcpyHostToDevice, m->ctx->stream));
        LAYA_HIP(hipMemcpyAsync(m->wm_word, word.data(), sizeof(int) * word.size(), hipMemcpyHostToDevice,
                                m->ctx->stream));
        LAYA_HIP(hipStreamSynchronize(m->ctx->stream));  // the host vectors go out of scope
    }
    absmax_multi(m->ctx, m->bf16_weights && m->PW ? m->PW : m->P, m->wm_off, m->wm_len, m->wm_word, m->wm_blocks,
                 m->amax_words, m->wm_bytes);
    for (int i : m->wm_params) m->amax_known[i] = 1;
}

// After a host write of the weights: the bf16 copy is stale, and so are the weights' magnitude words
// (cleared, to be measured again by the next product that reads them).
void weights_changed(laya_model* m) {
    m->wb_fresh = false;
    m->pw_fresh = false;
    if (m->amax_words) {
        fill(m->ctx, reinterpret_cast<float*>(m->amax_words), 0.0f, AMAX_GROUP * m->params.size());
        std::fill(m->amax_known.begin(), m->amax_known.begin() + m->params.size(), 0);
    }
}

// The weights' bf16 copy, when the products read copies: allocated on first use, refreshed from the fp32
// masters when a host write or an update without it left it stale.
void ensure_mirror(laya_model* m) {
    if (m->bf16_weights) {
        if (!m->PW) {
            m->PW = static_cast<float*>(m->ctx->alloc(m->total * sizeof(float)));
            m->pw_fresh = false;
        }
        if (!m->pw_fresh) {
            round_bf16(m->ctx, m->P, m->total, m->PW);
            m->pw_fresh = true;
        }
    }
    if (!m->copies) return;
    if (!m->WB) {
        m->WB = static_cast<__bf16*>(m->ctx->alloc(m->total * sizeof(__bf16)));
        m->wb_fresh = false;
    }
    if (!m->wb_fresh) {
        to_bf16(m->ctx, m->P, m->total, m->WB);
        m->wb_fresh = true;
    }
}

void upload_ints(laya_model* m, int* dst, const std::vector<int>& src) {
    if (src.empty()) return;
    LAYA_HIP(hipMemcpyAsync(dst, src.data(), src.size() * sizeof(int), hipMemcpyHostToDevice, m->ctx->stream));
}

// The batch layout of Forward (TrainableDecisionModel.cs:254-274), with the checks that run before any math.
BatchPlan plan_batch(const laya_model* m, const laya_batch* b) {
    LAYA_REQUIRE(b && b->n_items > 0, "forward: empty batch");
    LAYA_REQUIRE(b->lengths && b->tokens && b->n_options && b->markers && b->qtypes, "forward: null batch array");
    BatchPlan bp;
    const int n = b->n_items;
    bp.start.assign(n, 0);
    bp.len.assign(b->lengths, b->lengths + n);
    bp.qtypes.assign(b->qtypes, b->qtypes + n);
    long total = 0, marks = 0;
    int longest = 0;
    for (int i = 0; i < n; ++i) {
        LAYA_REQUIRE(b->lengths[i] > 0, "forward: an item has no tokens");
        LAYA_REQUIRE(b->n_options[i] >= 0, "forward: negative option count");
        LAYA_REQUIRE(b->qtypes[i] >= 0 && b->qtypes[i] < 3, "forward: question type outside [0, 3)");
        bp.start[i] = (int)total;
        total += b->lengths[i];
        marks += b->n_options[i];
        longest = std::max(longest, b->lengths[i]);
        bp.max_opts = std::max(bp.max_opts, b->n_options[i]);
    }
    bp.T = (int)total;
    bp.nseg = n;
    bp.nmark = (int)marks;
    bp.max_len = longest;
    bp.tokens.assign(b->tokens, b->tokens + total);
    for (int t = 0; t < bp.T; ++t)
        if ((unsigned)bp.tokens[t] >= (unsigned)m->cfg.vocab)
            throw Error(LAYA_ERR_OUT_OF_RANGE, "token id " + std::to_string(bp.tokens[t]) + " is outside the vocabulary.");
    bp.marker_rows.assign(bp.nmark, 0);
    bp.opt_off.assign(n + 1, 0);
    for (int i = 0, k = 0; i < n; ++i) {
        bp.opt_off[i + 1] = bp.opt_off[i] + b->n_options[i];
        for (int o = 0; o < b->n_options[i]; ++o, ++k) {
            const int pos = std::max(0, b->markers[k]);
            LAYA_REQUIRE(pos < b->lengths[i], "forward: a marker lies beyond its item");
            bp.marker_rows[k] = bp.start[i] + pos;
        }
    }
    bp.blocks = attention_block_list(bp.len);
    bp.n_blocks = (int)bp.blocks.size();
    bp.row_type.assign(bp.T, 0);
    bp.pos.assign(bp.T, 0);
    for (int i = 0; i < n; ++i) {
        bp.keys_full += window_keys(bp.len[i], -1);
        bp.keys_local += window_keys(bp.len[i], m->cfg.local_attention / 2);
        for (int t = 0; t < b->lengths[i]; ++t) {
            bp.row_type[bp.start[i] + t] = b->qtypes[i];
            bp.pos[bp.start[i] + t] = t;  // segment-local RoPE position
        }
    }
    // Embedding-gradient plan: positions stably sorted by id (counting sort), one run per unique id.
    bp.sorted.assign(bp.T, 0);
    bp.unique.assign(bp.T + 1, 0);
    bp.uoff.assign(bp.T + 2, 0);
    int nu = 0;
    if (laya_embedding_plan(bp.tokens.data(), bp.T, m->cfg.vocab, bp.sorted.data(), bp.unique.data(), bp.uoff.data(),
                            &nu) != LAYA_OK)
        throw Error(LAYA_ERR_OUT_OF_RANGE, laya_last_error());
    bp.n_unique = nu;
    return bp;
}

void upload_tables(laya_model* m, const BatchTables& t, const BatchPlan& bp) {
    upload_ints(m, t.tokens, bp.tokens);
    upload_ints(m, t.seg_start, bp.start);
    upload_ints(m, t.seg_len, bp.len);
    upload_ints(m, t.row_type, bp.row_type);
    upload_ints(m, t.marker_rows, bp.marker_rows);
    upload_ints(m, t.qtypes, bp.qtypes);
    upload_ints(m, t.opt_off, bp.opt_off);
    upload_ints(m, t.sorted, bp.sorted);
    upload_ints(m, t.unique, bp.unique);
    upload_ints(m, t.uoff, bp.uoff);
    upload_ints(m, t.pos, bp.pos);
    upload_ints(m, t.blocks, bp.blocks);
}

// Makes a batch's sizes the model's current ones and sizes the activations and rotary tables for it.
template <typename B> void set_batch_sizes(laya_model* m, const B& b) {
    m->T = b.T;
    m->nseg = b.nseg;
    m->nmark = b.nmark;
    m->max_len = b.max_len;
    m->n_unique = b.n_unique;
    m->max_opts = b.max_opts;
    m->keys_full = b.keys_full;
    m->keys_local = b.keys_local;
    m->n_blocks = b.n_blocks;
    m->opt_off_host = b.opt_off;
    ensure_activations(m, b.T, b.nmark, b.nseg);
    ensure_rotary(m, b.max_len);
}

void prepare_batch(laya_model* m, const laya_batch* b) {
    const BatchPlan bp = plan_batch(m, b);
    set_batch_sizes(m, bp);
    m->cur = m->own;
    upload_tables(m, m->cur, bp);
}

// The encoder's QKV projection applies RoPE in its epilogue when a head is 64 wide (the epilogue's
// layout); other widths rotate a copy inside the attention entry points.
bool fused_rope(const laya_model* m) { return m->d() / m->cfg.heads == 64; }

AttentionArgs enc_attention(laya_model* m, const float* qkv, int kind) {
    AttentionArgs a{};
    a.qkv = qkv;
    a.seg_start = m->cur.seg_start;
    a.seg_len = m->cur.seg_len;
    a.nseg = m->nseg;
    a.max_len = m->max_len;
    a.hidden = m->d();
    a.heads = m->cfg.heads;
    a.head_dim = m->d() / m->cfg.heads;
    a.half_window = kind == 1 ? m->cfg.local_attention / 2 : -1;
    a.keys = kind == 1 ? m->keys_local : m->keys_full;
    a.scale = 1.0f / std::sqrt((float)a.head_dim);
    a.p_drop = 0.0f;
    a.seed = 0;
    const laya_rotary& r = kind == 0 ? m->rot_global : m->rot_local;
    a.cos_table = r.cos_t;
    a.sin_table = r.sin_t;
    a.positions = r.positions;
    a.rotated = fused_rope(m);  // q and k left the QKV projection rotated
    a.rows = m->T;
    a.blocks = m->n_blocks > 0 ? m->cur.blocks : nullptr;
    a.n_blocks = m->n_blocks;
    return a;
}

uint64_t salt(uint64_t seed, int layer, int site) { return mix64(seed, (uint64_t)(layer * 16 + site + 1)); }

AttentionArgs head_attention(laya_model* m, const float* qkv, int index, float p, uint64_t seed) {
    AttentionArgs a{};
    a.qkv = qkv;
    a.seg_start = m->cur.seg_start;
    a.seg_len = m->cur.seg_len;
    a.nseg = m->nseg;
    a.max_len = m->max_len;
    a.hidden = m->d();
    a.heads = m->head_heads;
    a.head_dim = m->d() / m->head_heads;
    a.half_window = -1;
    a.keys = m->keys_full;
    a.scale = 1.0f / std::sqrt((float)(m->d() / m->head_heads));
    a.p_drop = p;
    a.seed = salt(seed, index, 0);
    a.rows = m->T;
    a.blocks = m->n_blocks > 0 ? m->cur.blocks : nullptr;
    a.n_blocks = m->n_blocks;
    return a;
}

// x16: x's bf16 copy, or null; ax: x's magnitude word; ay (optional): y's, to fold y into.
void linear(laya_model* m, const float* x, int rows, int in, int wi, int bi, int out, const float* residual, float* y,
            const __bf16* x16 = nullptr, AmaxRef ax = {}, unsigned* ay = nullptr) {
    gemm(m->ctx, GemmLayout::NT, GemmEpilogue::Store, rows, out, in, x, in, m->PWt(wi), in, y, out, m->W(bi), residual,
         out, x16, m->W16(wi), ax, m->wref(wi), ay);
}

// Ops.LinearBackward (Ops.cs:33-69): dx = dy·W (overwrite; + residual when given), dW += dyᵀ·x, db += Σ dy.
// site: the product's magnitude-word site (its input's word and its output gradient's), or -1; adx
// (optional): dx's magnitude word, to fold dx into.
void linear_backward(laya_model* m, const float* x, const float* dy, int rows, int in, int out, int wi, int bi,
                     float* dx, const float* dx_residual = nullptr, const __bf16* x16 = nullptr, int site = -1,
                     unsigned* adx = nullptr) {
    float* dW = m->Gt(wi);
    if (dx && dW) {
        gemm_backward_pair(m->ctx, rows, in, out, dy, m->PWt(wi), x, dx, dx_residual, dW, m->W16(wi), x16,
                           site >= 0 ? m->dref(site) : AmaxRef{}, m->wref(wi),
                           site >= 0 ? m->aref(site) : AmaxRef{}, adx);
    } else if (dx) {
        gemm(m->ctx, GemmLayout::NN, GemmEpilogue::Store, rows, in, out, dy, out, m->PWt(wi), in, dx, in, nullptr,
             dx_residual, in, nullptr, m->W16(wi), {}, {}, adx);
    } else if (dW) {
        gemm(m->ctx, GemmLayout::TN, GemmEpilogue::Accumulate, out, in, rows, dy, out, x, in, dW, in, nullptr, nullptr,
             0, nullptr, x16);
    }
    if (float* db = m->Gt(bi)) column_sum_add(m->ctx, dy, rows, out, db);
}

void dropout_copy(laya_model* m, const float* src, float* dst, size_t n, float p, uint64_t seed) {
    laya::dropout_copy(m->ctx, src, dst, n, p, seed);
}

// Forward (TrainableDecisionModel.cs:248-353) with EncoderLayerForward (361-414) and HeadLayerForward (428-468).
// Forward over the current batch (prepare_batch or a staged batch made it current).
// EncoderLayerForward (TrainableDecisionModel.cs:361-414) of layer l from its input ea[l].x: its internals
// into ea[l] and, with `output`, its output into the next layer's input (or x_final). A recompute before the
// layer's backward needs only the internals: the output is still held as the next layer's input.
void encoder_forward(laya_model* m, int l, bool output = true) {
    laya_ctx* ctx = m->ctx;
    const int T = m->T, d = m->d(), I = m->I();
    const float eps = m->cfg.norm_eps;
    auto& L = m->enc[l];
    auto& a = m->ea[l];
    float* out = l + 1 < m->cfg.layers ? m->ea[l + 1].x : m->x_final;
    const float* normed = a.x;
    // The products' inputs fold their magnitudes in as they are written (forward NT and backward pair).
    if (L.attn_norm >= 0) {
        layernorm_fwd(ctx, a.x, T, d, m->W(L.attn_norm), m->W(L.attn_norm_b), eps, a.normed, a.mean1, a.rstd1,
                      nullptr, nullptr, nullptr, a.normed16, m->produce(m->aref(m->enc_site(l, 0)), 7));
        normed = a.normed;
    } else if (a.normed16) {
        to_bf16(ctx, a.x, (size_t)T * d, a.normed16);  // nn.Identity: the QKV input is x itself
    }
    if (fused_rope(m)) {
        const laya_rotary& r = L.kind == 0 ? m->rot_global : m->rot_local;
        gemm_rope(ctx, T, 3 * d, d, normed, m->PWt(L.wqkv), a.qkv, m->W(L.wqkv_b), m->cur.pos, r.cos_t, r.sin_t,
                  2 * d, a.normed16, m->W16(L.wqkv), m->aref(m->enc_site(l, 0)), m->wref(L.wqkv),
                  m->produce_attention(m->aref(m->enc_site(l, 4))));
    } else {
        linear(m, normed, T, d, L.wqkv, L.wqkv_b, 3 * d, nullptr, a.qkv, a.normed16, m->aref(m->enc_site(l, 0)),
               m->produce_attention(m->aref(m->enc_site(l, 4))));
    }
    attention_fwd(ctx, enc_attention(m, a.qkv, L.kind), a.ctx, a.lse, a.ctx16,
                  m->produce(m->aref(m->enc_site(l, 1)), 7), m->aref(m->enc_site(l, 4)));
    linear(m, a.ctx, T, d, L.wo, L.wo_b, d, a.x, a.res, a.ctx16, m->aref(m->enc_site(l, 1)));  // x1 = x + attn
    layernorm_fwd(ctx, a.res, T, d, m->W(L.mlp_norm), m->W(L.mlp_norm_b), eps, a.mlpn, a.mean2, a.rstd2, nullptr,
                  nullptr, nullptr, a.mlpn16, m->produce(m->aref(m->enc_site(l, 2)), 7));
    gemm_geglu(ctx, T, I, d, a.mlpn, m->PWt(L.wi), m->W(L.wi_b), a.wide, a.act, a.act16, a.mlpn16, m->W16(L.wi),
               m->aref(m->enc_site(l, 2)), m->wref(L.wi), m->produce(m->aref(m->enc_site(l, 3)), 7));
    if (output)  // x2 = x1 + mlp
        linear(m, a.act, T, I, L.mlp_wo, L.mlp_wo_b, d, a.res, out, a.act16, m->aref(m->enc_site(l, 3)));
}

void forward(laya_model* m, bool train, uint64_t seed) {
    laya_ctx* ctx = m->ctx;
    const int T = m->T, d = m->d(), I = m->I(), ff = m->cfg.head_ff;
    const float eps = m->cfg.norm_eps;
    m->training = train;
    m->seed = seed;
    ensure_mirror(m);
    if (!m->amax_words) {
        const size_t n = m->params.size() + 2 * m->amax_sites();
        m->amax_words = static_cast<unsigned*>(ctx->alloc(sizeof(unsigned) * AMAX_GROUP * n));
        m->amax_known.assign(n, 0);
    }
    // The input words are cleared at every forward (+0.0f: all-zero bits); the weights' only when one of the
    // product weights is not known (the AdamW step folds the trainable ones back in as it updates them).
    const size_t np = m->params.size(), ns = m->amax_sites();
    fill(ctx, reinterpret_cast<float*>(m->amax_words + AMAX_GROUP * np), 0.0f, AMAX_GROUP * ns);
    std::fill(m->amax_known.begin() + np, m->amax_known.begin() + np + ns, 0);
    if (ctx->matmul_pair & 3) {
        bool known = !m->wm_params.empty();
        for (int i : m->wm_params) known = known && m->amax_known[i];
        if (!known) {
            fill(ctx, reinterpret_cast<float*>(m->amax_words), 0.0f, AMAX_GROUP * np);
            std::fill(m->amax_known.begin(), m->amax_known.begin() + np, 0);
            measure_weights(m);
        }
    }

    // Embedding gather fused into the embedding LayerNorm.
    float* x0 = m->cfg.layers > 0 ? m->ea[0].x : m->x_final;
    // Layer 0's QKV input is x itself when it has no attention norm.
    unsigned* x0_amax =
        m->cfg.layers > 0 && m->enc[0].attn_norm < 0 ? m->produce(m->aref(m->enc_site(0, 0)), 7) : nullptr;
    layernorm_fwd(ctx, m->W(m->tok_emb), T, d, m->W(m->emb_norm), m->W(m->emb_norm_b), eps, x0, m->emb_mean,
                  m->emb_rstd, m->cur.tokens, nullptr, nullptr, nullptr, x0_amax);
    for (int l = 0; l < m->cfg.layers; ++l) encoder_forward(m, l);
    // Final norm, then each question's type vector on its rows (TrainableDecisionModel.cs:294-304).
    float* h0 = m->cfg.head_layers > 0 ? m->ha[0].x : m->head_out;
    layernorm_fwd(ctx, m->x_final, T, d, m->W(m->final_norm), m->W(m->final_norm_b), eps, h0, m->fin_mean, m->fin_rstd,
                  nullptr, m->W(m->type_emb), m->cur.row_type);
    const float p = train ? m->head_dropout : 0.0f;
    for (int j = 0; j < m->cfg.head_layers; ++j) {
        auto& H = m->head[j];
        auto& a = m->ha[j];
        float* out = j + 1 < m->cfg.head_layers ? m->ha[j + 1].x : m->head_out;
        layernorm_fwd(ctx, a.x, T, d, m->W(H.norm1), m->W(H.norm1_b), 1e-5f, a.n1, a.mean1, a.rstd1, nullptr,
                      nullptr, nullptr, a.n1_16, m->produce(m->aref(m->head_site(j, 0)), 7));
        linear(m, a.n1, T, d, H.in_proj, H.in_proj_b, 3 * d, nullptr, a.qkv, a.n1_16, m->aref(m->head_site(j, 0)),
               m->produce_attention(m->aref(m->head_site(j, 4))));
        attention_fwd(ctx, head_attention(m, a.qkv, j, p, seed), a.ctx, a.lse, a.ctx16,
                      m->produce(m->aref(m->head_site(j, 1)), 7), m->aref(m->head_site(j, 4)));
        if (p > 0.0f) {
            linear(m, a.ctx, T, d, H.out_proj, H.out_proj_b, d, nullptr, a.res, a.ctx16, m->aref(m->head_site(j, 1)));
            dropout_add(ctx, a.res, a.x, (size_t)T * d, p, salt(seed, j, 1));
        } else {
            linear(m, a.ctx, T, d, H.out_proj, H.out_proj_b, d, a.x, a.res, a.ctx16, m->aref(m->head_site(j, 1)));
        }
        layernorm_fwd(ctx, a.res, T, d, m->W(H.norm2), m->W(H.norm2_b), 1e-5f, a.n2, a.mean2, a.rstd2, nullptr,
                      nullptr, nullptr, a.n2_16, m->produce(m->aref(m->head_site(j, 2)), 7));
        linear(m, a.n2, T, d, H.linear1, H.linear1_b, ff, nullptr, a.wide, a.n2_16, m->aref(m->head_site(j, 2)));
        relu_dropout_fwd(ctx, a.wide, (size_t)T * ff, p, salt(seed, j, 2), a.drop, a.drop16,
                         m->produce(m->aref(m->head_site(j, 3)), 7));
        if (p > 0.0f) {
            linear(m, a.drop, T, ff, H.linear2, H.linear2_b, d, nullptr, out, a.drop16, m->aref(m->head_site(j, 3)));
            dropout_add(ctx, out, a.res, (size_t)T * d, p, salt(seed, j, 3));
        } else {
            linear(m, a.drop, T, ff, H.linear2, H.linear2_b, d, a.res, out, a.drop16, m->aref(m->head_site(j, 3)));
        }
    }
    // Scorer at the option markers (TrainableDecisionModel.cs:313-323).
    const int M = m->nmark;
    gather_rows(ctx, m->head_out, m->cur.marker_rows, M, d, m->s_in);
    layernorm_fwd(ctx, m->s_in, M, d, m->W(m->sc_norm), m->W(m->sc_norm_b), 1e-5f, m->s_norm, m->s_mean, m->s_rstd);
    linear(m, m->s_norm, M, d, m->sc1, m->sc1_b, d, nullptr, m->s_pre, nullptr, m->aref(m->scorer_site(0)));
    gelu_fwd(ctx, m->s_pre, (size_t)M * d, m->s_act);
    linear(m, m->s_act, M, d, m->sc2, m->sc2_b, 1, nullptr, m->scores, nullptr, m->aref(m->scorer_site(1)));
    m->has_tape = true;
}

// Ops.LayerNormBackward with its dγ/dβ reduction deferred to the end of the backward.
void ln_backward(laya_model* m, const float* x, int rows, int n, int w, int b, float eps, const float* dy, float* dx,
                 const float* mean, const float* rstd, const int* gather_ids = nullptr, unsigned* amax = nullptr) {
    float* dg = m->Gt(w);
    float* db = m->Gt(b);
    float* ws = nullptr;
    if (dg || db) {
        const size_t need = 2 * (size_t)ln_bwd_partial_rows(rows) * n;
        LAYA_REQUIRE(m->ln_part_used + need <= m->ln_part_cap, "layernorm partials: buffer too small");
        ws = m->ln_part + m->ln_part_used;
        m->ln_part_used += (need + 63) / 64 * 64;
    }
    layernorm_bwd_deferred(m->ctx, x, rows, n, m->W(w), eps, dy, dx, dg, db, mean, rstd, gather_ids,
                           ws ? ws : m->ln_part, m->ln_jobs, amax);
}

// EncoderLayerBackward (TrainableDecisionModel.cs:551-603); dS holds dOutput and becomes dx.
void encoder_backward(laya_model* m, int l, bool need_input) {
    laya_ctx* ctx = m->ctx;
    auto& L = m->enc[l];
    auto& a = m->ea[l];
    const int T = m->T, d = m->d(), I = m->I();
    const float eps = m->cfg.norm_eps;
    linear_backward(m, a.act, m->dS, T, I, d, L.mlp_wo, L.mlp_wo_b, m->dact, nullptr, a.act16, m->enc_site(l, 3));
    // The products' output gradients fold their magnitudes in as they are written (backward pairs).
    geglu_bwd(ctx, a.wide, m->dact, T, I, m->dwide, m->produce(m->dref(m->enc_site(l, 2)), 6));
    linear_backward(m, a.mlpn, m->dwide, T, d, 2 * I, L.wi, L.wi_b, m->dn, nullptr, a.mlpn16, m->enc_site(l, 2));
    ln_backward(m, a.res, T, d, L.mlp_norm, L.mlp_norm_b, eps, m->dn, m->dS, a.mean2, a.rstd2, nullptr,
                m->produce(m->dref(m->enc_site(l, 1)), 6));
    linear_backward(m, a.ctx, m->dS, T, d, d, L.wo, L.wo_b, m->dctx, nullptr, a.ctx16, m->enc_site(l, 1),
                    m->produce_attention(m->dref(m->enc_site(l, 4))));
    attention_bwd(ctx, enc_attention(m, a.qkv, L.kind), T, a.ctx, a.lse, m->dctx, m->dqkv,
                  m->produce(m->dref(m->enc_site(l, 0)), 6), m->aref(m->enc_site(l, 4)), m->dref(m->enc_site(l, 4)));
    const float* normed = L.attn_norm >= 0 ? a.normed : a.x;
    const int an = m->enc_site(l, 0);
    if (!need_input) {
        linear_backward(m, normed, m->dqkv, T, d, 3 * d, L.wqkv, L.wqkv_b, nullptr, nullptr, a.normed16, an);
        return;
    }
    if (L.attn_norm < 0) {
        // Layer 0: nn.Identity, so dx = dResidual + dNormed, fused as the GEMM's residual.
        linear_backward(m, normed, m->dqkv, T, d, 3 * d, L.wqkv, L.wqkv_b, m->dS, m->dS, a.normed16, an);
    } else {
        linear_backward(m, normed, m->dqkv, T, d, 3 * d, L.wqkv, L.wqkv_b, m->dn, nullptr, a.normed16, an);
        // dS is now the output gradient of layer l − 1, the input of its MLP output product's backward.
        ln_backward(m, a.x, T, d, L.attn_norm, L.attn_norm_b, eps, m->dn, m->dS, a.mean1, a.rstd1, nullptr,
                    l > 0 ? m->produce(m->dref(m->enc_site(l - 1, 3)), 6) : nullptr);
    }
}

// HeadLayerBackward (TrainableDecisionModel.cs:605-640); dS holds dOutput and becomes dx.
void head_backward(laya_model* m, int j) {
    laya_ctx* ctx = m->ctx;
    auto& H = m->head[j];
    auto& a = m->ha[j];
    const int T = m->T, d = m->d(), ff = m->cfg.head_ff;
    const float p = m->training ? m->head_dropout : 0.0f;
    const size_t nd = (size_t)T * d;
    const float* dy = m->dS;
    if (p > 0.0f) {
        dropout_copy(m, m->dS, m->dy, nd, p, salt(m->seed, j, 3));
        dy = m->dy;
    }
    linear_backward(m, a.drop, dy, T, ff, d, H.linear2, H.linear2_b, m->dact, nullptr, a.drop16,
                    m->head_site(j, 3));
    if (ff % 4 == 0)
        relu_dropout_bwd_from_output(ctx, a.drop, m->dact, (size_t)T * ff, p,
                                     m->produce(m->dref(m->head_site(j, 2)), 6));
    else
        relu_dropout_bwd(ctx, a.wide, m->dact, (size_t)T * ff, p, salt(m->seed, j, 2));
    linear_backward(m, a.n2, m->dact, T, d, ff, H.linear1, H.linear1_b, m->dn, nullptr, a.n2_16,
                    m->head_site(j, 2));
    ln_backward(m, a.res, T, d, H.norm2, H.norm2_b, 1e-5f, m->dn, m->dS, a.mean2, a.rstd2);
    const float* datt = m->dS;
    if (p > 0.0f) {
        dropout_copy(m, m->dS, m->dy, nd, p, salt(m->seed, j, 1));
        datt = m->dy;
    }
    linear_backward(m, a.ctx, datt, T, d, d, H.out_proj, H.out_proj_b, m->dctx, nullptr, a.ctx16,
                    m->head_site(j, 1), m->produce_attention(m->dref(m->head_site(j, 4))));
    attention_bwd(ctx, head_attention(m, a.qkv, j, p, m->seed), T, a.ctx, a.lse, m->dctx, m->dqkv, nullptr,
                  m->aref(m->head_site(j, 4)), m->dref(m->head_site(j, 4)));
    linear_backward(m, a.n1, m->dqkv, T, d, 3 * d, H.in_proj, H.in_proj_b, m->dn, nullptr, a.n1_16,
                    m->head_site(j, 0));
    ln_backward(m, a.x, T, d, H.norm1, H.norm1_b, 1e-5f, m->dn, m->dS, a.mean1, a.rstd1);
}

void backward_body(laya_model* m);

// Backward (TrainableDecisionModel.cs:479-549), from dscores already on the device. The LayerNorm dγ/dβ
// partials of every site are reduced in one launch at the end (each in its fixed order).
// The backward is linear in the logit gradients and, apart from the parameter gradients' sums, separate per
// item: every activation-gradient row of item i scales with item i's logit gradients. A two-piece product scales
// its operand by one power of two from the operand's largest magnitude, so a row far below that largest loses
// relative precision (a row 2^-k of it keeps ≈ 2^(k-39) relative error, from subnormal fp16 pieces). When the
// items' largest |dL/dlogit| span more than this factor, the backward runs its products (linears and
// attention) on exact three-piece bf16 splits, whose pieces carry fp32's exponent range.
constexpr float BACKWARD_RANGE = 16384.0f;  // 2^14

bool logit_range_too_wide(const laya_model* m, const float* dl) {
    float hi = 0.0f, lo = INFINITY;
    for (size_t i = 0; i + 1 < m->opt_off_host.size(); ++i) {
        float a = 0.0f;
        for (int o = m->opt_off_host[i]; o < m->opt_off_host[i + 1]; ++o) a = std::max(a, std::fabs(dl[o]));
        if (!(a > 0.0f) || !std::isfinite(a)) continue;  // zero (or non-finite) items: no range to keep
        hi = std::max(hi, a);
        lo = std::min(lo, a);
    }
    return hi > 0.0f && hi > BACKWARD_RANGE * lo;
}

// Restores the context's two-piece choices when a backward that set them aside ends (or throws).
struct PairPolicyScope {
    laya_ctx* ctx;
    int pair;
    bool attention;
    explicit PairPolicyScope(laya_ctx* c) : ctx(c), pair(c->matmul_pair), attention(c->attention_pair) {
        ctx->matmul_pair &= ~(LAYA_MATMUL_BF16_INPUT_GRAD | LAYA_MATMUL_BF16_WEIGHT_GRAD);
        ctx->attention_pair = false;
    }
    ~PairPolicyScope() {
        ctx->matmul_pair = pair;
        ctx->attention_pair = attention;
    }
};

// dl_host: the logit gradients already on the host (else read back from ds_scores when the range check needs
// them, which only the two-piece products do).
void backward(laya_model* m, const float* dl_host = nullptr) {
    LAYA_REQUIRE(m->has_tape, "backward: run forward first");
    laya_ctx* ctx = m->ctx;
    bool wide = false;
    if (m->nmark > 0 && ((ctx->matmul_pair & (LAYA_MATMUL_BF16_INPUT_GRAD | LAYA_MATMUL_BF16_WEIGHT_GRAD)) ||
                         ctx->attention_pair)) {
        if (!dl_host) {
            m->dl_host.resize(m->nmark);
            LAYA_HIP(hipMemcpyAsync(m->dl_host.data(), m->ds_scores, sizeof(float) * m->nmark,
                                    hipMemcpyDeviceToHost, ctx->stream));
            LAYA_HIP(hipStreamSynchronize(ctx->stream));
            dl_host = m->dl_host.data();
        }
        wide = logit_range_too_wide(m, dl_host);
    }
    m->backward_split3 = wide;
    std::unique_ptr<PairPolicyScope> scope;
    if (wide) scope.reset(new PairPolicyScope(ctx));
    ensure_mirror(m);
    const int d = m->d();
    const size_t sites = 2 * (size_t)m->cfg.layers + 2 * (size_t)m->cfg.head_layers + 3;
    const size_t need = sites * ((2 * (size_t)ln_bwd_partial_rows(std::max(m->T, m->nmark)) * d + 63) / 64 * 64);
    if (need > m->ln_part_cap) {
        if (m->ln_part) m->ctx->release(m->ln_part);
        m->ln_part = nullptr;
        m->ln_part_cap = 0;
        const size_t cap = sites * ((2 * (size_t)ln_bwd_partial_rows(1 << 30) * d + 63) / 64 * 64);
        m->ln_part = static_cast<float*>(m->ctx->alloc(sizeof(float) * cap));
        m->ln_part_cap = cap;
    }
    m->ln_part_used = 0;
    m->ln_jobs.n = 0;
    if (m->amax_words) {
        const size_t k = m->params.size() + m->amax_sites();
        fill(m->ctx, reinterpret_cast<float*>(m->amax_words + AMAX_GROUP * k), 0.0f, AMAX_GROUP * m->amax_sites());
        std::fill(m->amax_known.begin() + k, m->amax_known.end(), 0);
    }
    backward_body(m);
    column_reduce_batch(m->ctx, m->ln_jobs);
    m->ln_jobs.n = 0;
}

void backward_body(laya_model* m) {
    laya_ctx* ctx = m->ctx;
    const int T = m->T, d = m->d(), M = m->nmark;
    const float eps = m->cfg.norm_eps;
    linear_backward(m, m->s_act, m->ds_scores, M, d, 1, m->sc2, m->sc2_b, m->ds_act, nullptr, nullptr,
                    m->scorer_site(1));
    gelu_bwd(ctx, m->s_pre, m->ds_act, (size_t)M * d);
    linear_backward(m, m->s_norm, m->ds_act, M, d, d, m->sc1, m->sc1_b, m->ds_norm, nullptr, nullptr,
                    m->scorer_site(0));
    fill(ctx, m->ds_mark, 0.0f, (size_t)M * d);
    ln_backward(m, m->s_in, M, d, m->sc_norm, m->sc_norm_b, 1e-5f, m->ds_norm, m->ds_mark, m->s_mean, m->s_rstd);
    fill(ctx, m->dS, 0.0f, (size_t)T * d);
    scatter_add_rows(ctx, m->ds_mark, m->cur.marker_rows, M, d, m->dS);
    for (int j = m->cfg.head_layers - 1; j >= 0; --j) head_backward(m, j);
    if (float* g = m->Gt(m->type_emb))
        type_embedding_bwd(ctx, m->dS, m->cur.row_type, T, d, g);
    if (m->first_trainable >= m->cfg.layers) return;  // the encoder is frozen
    fill(ctx, m->dE, 0.0f, (size_t)T * d);
    ln_backward(m, m->x_final, T, d, m->final_norm, m->final_norm_b, eps, m->dS, m->dE, m->fin_mean, m->fin_rstd,
                nullptr, m->cfg.layers > 0 ? m->produce(m->dref(m->enc_site(m->cfg.layers - 1, 3)), 6) : nullptr);
    std::swap(m->dS, m->dE);
    for (int l = m->cfg.layers - 1; l >= m->first_trainable; --l) {
        // Layer checkpointing: the layer's internals are recomputed from its kept input (the same kernels on
        // the same inputs give the same values) just before its backward, as the reference always does.
        if (m->recompute) encoder_forward(m, l, false);
        encoder_backward(m, l, l > m->first_trainable || m->embeddings_trainable);
    }
    if (m->embeddings_trainable && m->first_trainable == 0) {
        fill(ctx, m->dE, 0.0f, (size_t)T * d);
        ln_backward(m, m->W(m->tok_emb), T, d, m->emb_norm, m->emb_norm_b, eps, m->dS, m->dE, m->emb_mean, m->emb_rstd,
                    m->cur.tokens);
        if (float* g = m->Gt(m->tok_emb))
            embedding_bwd(ctx, m->cur.sorted, m->cur.unique, m->cur.uoff, m->n_unique, m->dE, d, g);
    }
}

// The trainer's groups (Trainer.cs:96-100) as contiguous trainable ranges of the arena.
AdamGroups adam_groups(laya_model* m, double lr_enc, double lr_head, double wd, double c1, size_t* n_out) {
    AdamGroups g{};
    std::vector<std::pair<size_t, size_t>> ranges[2];
    for (const auto& p : m->params) {
        if (!p.trainable) continue;
        const int grp = p.name.find("encoder.") != std::string::npos ? 0 : 1;
        auto& r = ranges[grp];
        const size_t b = p.offset, e = p.offset + (p.numel + 63) / 64 * 64;
        if (!r.empty() && r.back().second == b)
            r.back().second = e;
        else
            r.push_back({b, e});
    }
    for (int grp = 0; grp < 2; ++grp) {
        const double lr = grp == 0 ? lr_enc : lr_head;
        for (auto& r : ranges[grp]) {
            LAYA_REQUIRE(g.n < 4, "adamw: trainable parameters form more than 4 ranges");
            g.begin[g.n] = r.first;
            g.end[g.n] = r.second;
            g.decay[g.n] = (float)(1.0 - lr * wd);
            g.step_size[g.n] = (float)(lr / c1);
            g.n++;
        }
    }
    *n_out = m->total;
    return g;
}

void ensure_moments(laya_model* m) {
    if (m->M1) return;
    m->M1 = static_cast<float*>(m->ctx->alloc(m->total * sizeof(float)));
    m->M2 = static_cast<float*>(m->ctx->alloc(m->total * sizeof(float)));
    fill(m->ctx, m->M1, 0.0f, m->total);
    fill(m->ctx, m->M2, 0.0f, m->total);
}

// The AdamW fold's tables for the current trainable flags: the product weights that lie inside the update's
// groups, and per workgroup of 256 float4s the tensor that covers it whole (-1 none, -2 several or in part).
void ensure_fold(laya_model* m, const AdamGroups& g) {
    std::vector<unsigned char> now(m->params.size());
    for (size_t i = 0; i < m->params.size(); ++i) now[i] = m->params[i].trainable;
    if (m->fold_block && now == m->fold_for) return;
    auto inside = [&](size_t b, size_t e) {
        for (int k = 0; k < g.n; ++k)
            if (b >= g.begin[k] && e <= g.end[k]) return true;
        return false;
    };
    std::vector<std::pair<long, int>> ts;  // (first float4, parameter)
    for (int i : m->wm_params) {
        const Param& p = m->params[i];
        LAYA_REQUIRE(p.offset % 4 == 0, "adamw fold: tensors must start on a float4");
        if (p.trainable && inside(p.offset, p.offset + p.numel)) ts.push_back({(long)(p.offset / 4), i});
    }
    std::sort(ts.begin(), ts.end());
    std::vector<long> begin, end;
    std::vector<int> word;
    m->fold_params.clear();
    for (auto& t : ts) {
        const Param& p = m->params[t.second];
        begin.push_back(t.first);
        end.push_back(t.first + (long)(p.numel / 4));  // numel is a multiple of 4 for every product weight
        word.push_back(t.second);
        m->fold_params.push_back(t.second);
        LAYA_REQUIRE(p.numel % 4 == 0, "adamw fold: product weights hold a multiple of 4 values");
    }
    const long n4 = (long)(m->total / 4);
    const long blocks = (n4 + 255) / 256;
    std::vector<int> blk(blocks, -1);
    size_t t = 0;
    for (long b = 0; b < blocks; ++b) {
        const long lo = b * 256, hi = std::min(n4, lo + 256);
        while (t < begin.size() && end[t] <= lo) ++t;
        if (t >= begin.size() || begin[t] >= hi) continue;      // no tensor meets the block
        blk[b] = begin[t] <= lo && end[t] >= hi ? (int)t : -2;  // whole, or a boundary inside
    }
    for (void* p : {(void*)m->fold_block, (void*)m->fold_begin, (void*)m->fold_end, (void*)m->fold_word})
        if (p) m->ctx->release(p);
    const size_t nt = std::max<size_t>(begin.size(), 1);
    m->fold_block = static_cast<int*>(m->ctx->alloc(sizeof(int) * blocks));
    m->fold_begin = static_cast<long*>(m->ctx->alloc(sizeof(long) * nt));
    m->fold_end = static_cast<long*>(m->ctx->alloc(sizeof(long) * nt));
    m->fold_word = static_cast<int*>(m->ctx->alloc(sizeof(int) * nt));
    m->fold_n = (int)begin.size();
    LAYA_HIP(hipMemcpyAsync(m->fold_block, blk.data(), sizeof(int) * blocks, hipMemcpyHostToDevice, m->ctx->stream));
    if (m->fold_n) {
        LAYA_HIP(hipMemcpyAsync(m->fold_begin, begin.data(), sizeof(long) * begin.size(), hipMemcpyHostToDevice,
                                m->ctx->stream));
        LAYA_HIP(hipMemcpyAsync(m->fold_end, end.data(), sizeof(long) * end.size(), hipMemcpyHostToDevice,
                                m->ctx->stream));
        LAYA_HIP(hipMemcpyAsync(m->fold_word, word.data(), sizeof(int) * word.size(), hipMemcpyHostToDevice,
                                m->ctx->stream));
    }
    LAYA_HIP(hipStreamSynchronize(m->ctx->stream));  // the host vectors go out of scope
    m->fold_for = now;
}

void adamw_step(laya_model* m, double lr_enc, double lr_head, double b1, double b2, double eps, double wd,
                bool zero_grads) {
    ensure_moments(m);
    m->steps++;
    const double c1 = 1.0 - std::pow(b1, m->steps), c2 = 1.0 - std::pow(b2, m->steps);
    size_t n = 0;
    AdamGroups g = adam_groups(m, lr_enc, lr_head, wd, c1, &n);
    // The weights' bf16 copy is updated with them when the products read it; otherwise it goes stale.
    __bf16* mirror = m->copies && m->WB && m->wb_fresh ? m->WB : nullptr;
    // The update moves the weights, so their magnitude words no longer bound them: cleared (an unknown word
    // holds zero). When the products read the fp32 weights themselves, the update folds the new magnitudes of
    // the trainable product weights back in (the rest are measured again by the next forward, or by a backward
    // product that runs before one).
    const AdamFold* fold = nullptr;
    AdamFold f{};
    if (m->amax_words) {
        fill(m->ctx, reinterpret_cast<float*>(m->amax_words), 0.0f, AMAX_GROUP * m->params.size());
        std::fill(m->amax_known.begin(), m->amax_known.begin() + m->params.size(), 0);
        if (!m->bf16_weights && !m->wm_params.empty()) {
            ensure_fold(m, g);
            f = AdamFold{m->fold_block, m->fold_begin, m->fold_end, m->fold_word, m->fold_n, m->amax_words};
            fold = &f;
        }
    }
    adamw_arena(m->ctx, m->P, m->G, m->M1, m->M2, n, g, (float)b1, (float)b2, (float)eps, (float)std::sqrt(c2),
                m->coef_valid ? m->d_coef : nullptr, zero_grads ? 1 : 0, mirror, fold);
    if (fold)
        for (int k = 0; k < m->fold_n; ++k) m->amax_known[m->fold_params[k]] = 1;
    if (!mirror) m->wb_fresh = false;
    m->pw_fresh = false;  // the bf16 weights are rounded again before the next product reads them
    m->coef_valid = false;
}

laya_model* checked(laya_model* m) {
    LAYA_REQUIRE(m != nullptr, "null model");
    LAYA_HIP(hipSetDevice(m->ctx->device));
    return m;
}

}  // namespace

extern "C" {

int laya_model_create(laya_ctx* ctx, const laya_model_config* cfg, laya_model** out) {
    return guarded([&] {
        LAYA_REQUIRE(ctx && cfg && out, "null argument");
        LAYA_REQUIRE(cfg->vocab > 0 && cfg->hidden > 0 && cfg->intermediate > 0 && cfg->layers >= 0 && cfg->heads > 0,
                     "model: bad configuration");
        LAYA_REQUIRE(cfg->hidden % cfg->heads == 0, "model: hidden must be a multiple of heads");
        auto* m = new laya_model();
        m->ctx = ctx;
        m->cfg = *cfg;
        m->cfg.layer_kinds = nullptr;
        m->kinds.resize(cfg->layers);
        for (int l = 0; l < cfg->layers; ++l)
            m->kinds[l] = cfg->layer_kinds ? cfg->layer_kinds[l] : (l % std::max(1, cfg->global_every) == 0 ? 0 : 1);
        m->head_heads = std::max(1, cfg->hidden / 64);  // TrainableDecisionModel.cs:109
        build_layout(m);
        try {
            m->P = static_cast<float*>(ctx->alloc(m->total * sizeof(float)));
            m->G = static_cast<float*>(ctx->alloc(m->total * sizeof(float)));
            fill(ctx, m->P, 0.0f, m->total);
            fill(ctx, m->G, 0.0f, m->total);
            m->d_norm = static_cast<double*>(ctx->alloc(64));
            m->d_coef = static_cast<float*>(ctx->alloc(64));
            m->d_loss = static_cast<float*>(ctx->alloc(64));
            m->d_nonfinite = static_cast<int*>(ctx->alloc(64));
            ensure_rotary(m, 1024);
        } catch (...) {
            for (void* p : {(void*)m->P, (void*)m->G, (void*)m->d_norm, (void*)m->d_coef, (void*)m->d_loss,
                            (void*)m->d_nonfinite})
                if (p) ctx->release(p);
            delete m;
            throw;
        }
        *out = m;
    });
}

int laya_model_destroy(laya_model* m) {
    return guarded([&] {
        if (!m) return;
        laya_ctx* ctx = m->ctx;
        for (void* p : {(void*)m->P, (void*)m->G, (void*)m->M1, (void*)m->M2, m->act_block, (void*)m->d_norm,
                        (void*)m->d_coef, (void*)m->d_loss, (void*)m->d_nonfinite})
            if (p) ctx->release(p);
        for (auto& s : m->staged)
            if (s.block) ctx->release(s.block);
        for (void* p : {(void*)m->d_draws, (void*)m->d_rlcd_losses, (void*)m->ln_part, (void*)m->WB, (void*)m->PW,
                        (void*)m->amax_words, (void*)m->wm_off, (void*)m->wm_len, (void*)m->wm_word,
                        (void*)m->fold_block, (void*)m->fold_begin, (void*)m->fold_end, (void*)m->fold_word})
            if (p) ctx->release(p);
        free_rotary(ctx, &m->rot_global);
        free_rotary(ctx, &m->rot_local);
        delete m;
    });
}

int laya_model_num_params(laya_model* m, int* count) {
    return guarded([&] { *count = (int)checked(m)->params.size(); });
}

int laya_model_param_info(laya_model* m, int i, const char** name, int* ndim, int* dims, size_t* offset, size_t* numel,
                          int* trainable) {
    return guarded([&] {
        LAYA_REQUIRE(m && i >= 0 && i < (int)m->params.size(), "param index out of range");
        const Param& p = m->params[i];
        if (name) *name = p.name.c_str();
        if (ndim) *ndim = (int)p.shape.size();
        if (dims)
            for (size_t k = 0; k < p.shape.size() && k < 4; ++k) dims[k] = p.shape[k];
        if (offset) *offset = p.offset;
        if (numel) *numel = p.numel;
        if (trainable) *trainable = p.trainable ? 1 : 0;
    });
}

int laya_model_find_param(laya_model* m, const char* name, int* index) {
    return guarded([&] {
        LAYA_REQUIRE(m && name && index, "null argument");
        auto it = m->by_name.find(name);
        if (it == m->by_name.end())
            throw Error(LAYA_ERR_MISSING, std::string("the checkpoint has no '") + name + "' tensor");
        *index = it->second;
    });
}

int laya_model_set_param(laya_model* m, int i, const float* host) {
    return guarded([&] {
        checked(m);
        LAYA_REQUIRE(i >= 0 && i < (int)m->params.size() && host, "set_param: bad argument");
        const Param& p = m->params[i];
        LAYA_HIP(hipMemcpyAsync(m->P + p.offset, host, p.numel * sizeof(float), hipMemcpyHostToDevice, m->ctx->stream));
        weights_changed(m);
        LAYA_HIP(hipStreamSynchronize(m->ctx->stream));
    });
}

int laya_model_get_param(laya_model* m, int i, float* host) {
    return guarded([&] {
        checked(m);
        LAYA_REQUIRE(i >= 0 && i < (int)m->params.size() && host, "get_param: bad argument");
        const Param& p = m->params[i];
        LAYA_HIP(hipMemcpyAsync(host, m->P + p.offset, p.numel * sizeof(float), hipMemcpyDeviceToHost, m->ctx->stream));
        LAYA_HIP(hipStreamSynchronize(m->ctx->stream));
    });
}

int laya_model_get_grad(laya_model* m, int i, float* host) {
    return guarded([&] {
        checked(m);
        LAYA_REQUIRE(i >= 0 && i < (int)m->params.size() && host, "get_grad: bad argument");
        const Param& p = m->params[i];
        LAYA_HIP(hipMemcpyAsync(host, m->G + p.offset, p.numel * sizeof(float), hipMemcpyDeviceToHost, m->ctx->stream));
        LAYA_HIP(hipStreamSynchronize(m->ctx->stream));
    });
}

int laya_model_has_grad(laya_model* m, int i, int* has) {
    return guarded([&] {
        LAYA_REQUIRE(m && i >= 0 && i < (int)m->params.size() && has, "has_grad: bad argument");
        *has = m->params[i].touched ? 1 : 0;
    });
}

// The head layers' saved feed-forward activations of the last forward, by device address: which = 0 is
// linear1's output (the ReLU's input), 1 the ReLU-dropout output the backward takes its mask from.
int laya_model_head_activation(laya_model* m, int layer, int which, float** device, size_t* count) {
    return guarded([&] {
        checked(m);
        LAYA_REQUIRE(device && count && (which == 0 || which == 1), "head_activation: bad argument");
        LAYA_REQUIRE(layer >= 0 && layer < m->cfg.head_layers, "head_activation: no such head layer");
        if (!m->has_tape) throw Error(LAYA_ERR_STATE, "head_activation: no forward with saved activations");
        const auto& a = m->ha[layer];
        *device = which == 0 ? a.wide : a.drop;
        *count = (size_t)m->T * m->cfg.head_ff;
    });
}

int laya_model_init_random(laya_model* m, uint64_t seed, float std) {
    return guarded([&] {
        checked(m);
        for (size_t i = 0; i < m->params.size(); ++i) {
            const Param& p = m->params[i];
            init_param(m->ctx, m->P + p.offset, p.numel, p.init, std, mix64(seed, (uint64_t)i + 1));
        }
        weights_changed(m);
        LAYA_HIP(hipStreamSynchronize(m->ctx->stream));
    });
}

// SetTrainableEncoderLayers (TrainableDecisionModel.cs:206-231).
int laya_model_set_trainable_encoder_layers(laya_model* m, int n) {
    return guarded([&] {
        checked(m);
        const int count = m->cfg.layers;
        const int trainable = n < 0 ? count : std::clamp(n, 0, count);
        m->first_trainable = count - trainable;
        const bool all = n < 0 || (trainable == count && n >= count);
        for (auto& p : m->params) {
            if (p.name == "temperature") continue;
            if (p.name.rfind("encoder.", 0) != 0) {
                p.trainable = true;
                continue;
            }
            bool train;
            if (p.name.rfind("encoder.embeddings.", 0) == 0)
                train = all;
            else if (p.name.rfind("encoder.final_norm.", 0) == 0)
                train = trainable > 0;
            else
                train = std::stoi(p.name.substr(15, p.name.find('.', 15) - 15)) >= m->first_trainable;
            if (!train && p.trainable) fill(m->ctx, m->G + p.offset, 0.0f, p.numel);
            p.trainable = train;
            if (!train) p.touched = false;
        }
        m->embeddings_trainable = m->params[m->tok_emb].trainable;
    });
}

int laya_model_set_layer_checkpointing(laya_model* m, int mode) {
    return guarded([&] {
        checked(m);
        LAYA_REQUIRE(mode >= 0 && mode <= 2, "layer checkpointing: 0 (keep), 1 (recompute) or 2 (when needed)");
        if (mode == m->checkpoint_mode) return;
        m->checkpoint_mode = mode;
        // The next forward lays the activation arena out for the new mode.
        m->has_tape = false;
        if (m->act_block) m->ctx->release(m->act_block);
        m->act_block = nullptr;
        m->cap_tokens = m->cap_markers = m->cap_segs = 0;
    });
}

int laya_model_set_bf16_weights(laya_model* m, int on) {
    return guarded([&] {
        checked(m);
        if ((on != 0) == m->bf16_weights) return;
        m->bf16_weights = on != 0;
        m->pw_fresh = false;
        // The weights the products read change: their magnitude words are measured again.
        weights_changed(m);
        if (!m->bf16_weights && m->PW) {
            m->ctx->release(m->PW);
            m->PW = nullptr;
        }
    });
}

int laya_model_set_bf16_copies(laya_model* m, int on) {
    return guarded([&] {
        checked(m);
        if ((on != 0) == m->bf16_copies) return;
        m->bf16_copies = on != 0;
        // The next forward lays the activation arena out with or without the copies.
        m->has_tape = false;
        if (m->act_block) m->ctx->release(m->act_block);
        m->act_block = nullptr;
        m->cap_tokens = m->cap_markers = m->cap_segs = 0;
        m->copies = false;
    });
}

int laya_model_get_param_bf16(laya_model* m, int i, uint16_t* host) {
    return guarded([&] {
        checked(m);
        LAYA_REQUIRE(i >= 0 && i < (int)m->params.size() && host, "get_param_bf16: bad argument");
        if (!m->WB || !m->wb_fresh)
            throw Error(LAYA_ERR_STATE, "get_param_bf16: no current bf16 copy (it is kept while a bf16 precision "
                                        "policy's products read it, from the first forward on)");
        const Param& p = m->params[i];
        LAYA_HIP(hipMemcpyAsync(host, m->WB + p.offset, p.numel * sizeof(uint16_t), hipMemcpyDeviceToHost,
                                m->ctx->stream));
        LAYA_HIP(hipStreamSynchronize(m->ctx->stream));
    });
}

int laya_model_layer_checkpointing(laya_model* m, int* mode, int* recomputing) {
    return guarded([&] {
        checked(m);
        if (mode) *mode = m->checkpoint_mode;
        if (recomputing) *recomputing = m->act_block && m->recompute ? 1 : 0;
    });
}

int laya_model_set_head_dropout(laya_model* m, float p) {
    return guarded([&] {
        LAYA_REQUIRE(m && p >= 0.0f && p < 1.0f, "head dropout must be in [0, 1)");
        m->head_dropout = p;
    });
}

int laya_model_forward(laya_model* m, const laya_batch* batch, int training, uint64_t seed, float* logits_host) {
    return guarded([&] {
        checked(m);
        prepare_batch(m, batch);
        forward(m, training != 0, seed);
        if (logits_host) {
            LAYA_HIP(hipMemcpyAsync(logits_host, m->scores, sizeof(float) * m->nmark, hipMemcpyDeviceToHost,
                                    m->ctx->stream));
            LAYA_HIP(hipStreamSynchronize(m->ctx->stream));
        }
    });
}

int laya_model_readout(laya_model* m, float* logits_host, float* act_probs_host, float* features_host) {
    return guarded([&] {
        checked(m);
        LAYA_REQUIRE(m->has_tape, "readout: run forward first");
        LAYA_REQUIRE(act_probs_host, "readout: null output");
        const int a1 = m->find("act_head.0.bias"), na_i = m->find("act_head.2.bias");
        const int w1 = m->find("act_head.0.weight"), w2 = m->find("act_head.2.weight");
        const int A1 = (int)m->params[a1].numel, NA = (int)m->params[na_i].numel, n = m->nseg;
        float* out = static_cast<float*>(m->ctx->workspace(8, sizeof(float) * (size_t)std::max(1, n) * (NA + 4)));
        decision_readout(m->ctx, m->scores, m->cur.opt_off, m->cur.seg_start, n, m->head_out, m->d(), m->W(w1),
                         m->W(a1), A1, m->W(w2), m->W(na_i), NA, out, out + (size_t)n * NA);
        LAYA_HIP(hipMemcpyAsync(act_probs_host, out, sizeof(float) * (size_t)n * NA, hipMemcpyDeviceToHost,
                                m->ctx->stream));
        if (features_host)
            LAYA_HIP(hipMemcpyAsync(features_host, out + (size_t)n * NA, sizeof(float) * (size_t)n * 4,
                                    hipMemcpyDeviceToHost, m->ctx->stream));
        if (logits_host)
            LAYA_HIP(hipMemcpyAsync(logits_host, m->scores, sizeof(float) * m->nmark, hipMemcpyDeviceToHost,
                                    m->ctx->stream));
        LAYA_HIP(hipStreamSynchronize(m->ctx->stream));
    });
}

int laya_model_backward(laya_model* m, const float* dlogits_host) {
    return guarded([&] {
        checked(m);
        LAYA_REQUIRE(m->has_tape, "backward: run forward first");
        LAYA_REQUIRE(dlogits_host || m->nmark == 0, "backward: null logit gradients");
        if (m->nmark)
            LAYA_HIP(hipMemcpyAsync(m->ds_scores, dlogits_host, sizeof(float) * m->nmark, hipMemcpyHostToDevice,
                                    m->ctx->stream));
        backward(m, dlogits_host);
        LAYA_HIP(hipStreamSynchronize(m->ctx->stream));
    });
}

int laya_model_clip_grad_norm(laya_model* m, double max_norm, double* norm_out) {
    return guarded([&] {
        checked(m);
        grad_norm(m->ctx, m->G, m->total, max_norm, m->d_norm, m->d_coef, m->d_nonfinite);
        m->coef_valid = m->norm_done = true;
        if (norm_out) {
            LAYA_HIP(hipMemcpyAsync(norm_out, m->d_norm, sizeof(double), hipMemcpyDeviceToHost, m->ctx->stream));
            LAYA_HIP(hipStreamSynchronize(m->ctx->stream));
            if (!std::isfinite(*norm_out))
                throw Error(LAYA_ERR_NOT_FINITE, "clip: the gradient norm is not finite; the gradients stay "
                                                 "unscaled (Gradients.ClipByGlobalNorm)");
        }
    });
}

int laya_model_grad_norm_status(laya_model* m) {
    return guarded([&] {
        checked(m);
        if (!m->norm_done) throw Error(LAYA_ERR_STATE, "grad_norm_status: no gradient norm since the model was built");
        int flag = 0;
        LAYA_HIP(hipMemcpyAsync(&flag, m->d_nonfinite, sizeof(int), hipMemcpyDeviceToHost, m->ctx->stream));
        LAYA_HIP(hipStreamSynchronize(m->ctx->stream));
        if (flag)
            throw Error(LAYA_ERR_NOT_FINITE, "the last step's gradient norm is not finite (a NaN or infinite "
                                             "gradient): its clip left the gradients unscaled and AdamW applied them, "
                                             "as the reference does");
    });
}

int laya_model_adamw_step(laya_model* m, double lr_encoder, double lr_head, double beta1, double beta2, double eps,
                          double weight_decay) {
    return guarded([&] {
        checked(m);
        adamw_step(m, lr_encoder, lr_head, beta1, beta2, eps, weight_decay, false);
    });
}

int laya_model_zero_grad(laya_model* m) {
    return guarded([&] {
        checked(m);
        fill(m->ctx, m->G, 0.0f, m->total);
    });
}

}  // extern "C"

namespace {

// The optimizer step of Trainer.cs:131-144 on the current batch: forward, soft-CE gradient against
// `targets` (device), backward, global-norm clip and AdamW.
void train_step_current(laya_model* m, const float* targets, float ce_weight, float loss_scale, uint64_t seed,
                        double max_norm, double lr_encoder, double lr_head, double beta1, double beta2, double eps,
                        double weight_decay, float* loss_out) {
    forward(m, true, seed);
    softmax_ce_bwd(m->ctx, m->scores, targets, m->cur.opt_off, m->nseg, ce_weight, loss_scale, m->ds_scores,
                   m->d_loss);
    backward(m);
    grad_norm(m->ctx, m->G, m->total, max_norm, m->d_norm, m->d_coef, m->d_nonfinite);
    m->coef_valid = m->norm_done = true;
    adamw_step(m, lr_encoder, lr_head, beta1, beta2, eps, weight_decay, true);
    if (loss_out) {
        LAYA_HIP(hipMemcpyAsync(loss_out, m->d_loss, sizeof(float), hipMemcpyDeviceToHost, m->ctx->stream));
        LAYA_HIP(hipStreamSynchronize(m->ctx->stream));
    }
}

StagedBatch& staged_slot(laya_model* m, int slot) {
    LAYA_REQUIRE(slot >= 0 && slot < (int)m->staged.size() && m->staged[slot].block,
                 "staged batch: no such slot (never staged or already released)");
    return m->staged[slot];
}

}  // namespace

extern "C" {

int laya_model_train_step(laya_model* m, const laya_batch* batch, const float* targets_host, float ce_weight,
                          float loss_scale, uint64_t seed, double max_norm, double lr_encoder, double lr_head,
                          double beta1, double beta2, double eps, double weight_decay, float* loss_out) {
    return guarded([&] {
        checked(m);
        prepare_batch(m, batch);
        LAYA_REQUIRE(targets_host || m->nmark == 0, "train_step: null targets");
        if (m->nmark)
            LAYA_HIP(hipMemcpyAsync(m->targets, targets_host, sizeof(float) * m->nmark, hipMemcpyHostToDevice,
                                    m->ctx->stream));
        train_step_current(m, m->targets, ce_weight, loss_scale, seed, max_norm, lr_encoder, lr_head, beta1, beta2,
                           eps, weight_decay, loss_out);
    });
}

int laya_model_stage_batch(laya_model* m, const laya_batch* batch, const float* targets_host, int* slot) {
    return guarded([&] {
        checked(m);
        LAYA_REQUIRE(slot, "stage_batch: null slot");
        const BatchPlan bp = plan_batch(m, batch);
        LAYA_REQUIRE(targets_host || bp.nmark == 0, "stage_batch: null targets");
        // Size the shared activations now, so a step on this batch never allocates.
        ensure_activations(m, bp.T, bp.nmark, bp.nseg);
        ensure_rotary(m, bp.max_len);
        StagedBatch s;
        s.T = bp.T;
        s.nseg = bp.nseg;
        s.nmark = bp.nmark;
        s.max_len = bp.max_len;
        s.n_unique = bp.n_unique;
        s.max_opts = bp.max_opts;
        s.keys_full = bp.keys_full;
        s.keys_local = bp.keys_local;
        s.n_blocks = bp.n_blocks;
        s.opt_off = bp.opt_off;
        Carver cv;
        TableCarve tc;
        tc.add(cv, (size_t)bp.T, (size_t)std::max(bp.nmark, 1), (size_t)bp.nseg);
        cv.add(s.targets, (size_t)std::max(bp.nmark, 1));
        s.block = m->ctx->alloc(cv.bytes);
        cv.bind(static_cast<char*>(s.block));
        s.tables = tc.bind();
        upload_tables(m, s.tables, bp);
        if (bp.nmark)
            LAYA_HIP(hipMemcpyAsync(s.targets, targets_host, sizeof(float) * bp.nmark, hipMemcpyHostToDevice,
                                    m->ctx->stream));
        LAYA_HIP(hipStreamSynchronize(m->ctx->stream));  // the host vectors go out of scope
        int k = 0;
        while (k < (int)m->staged.size() && m->staged[k].block) ++k;
        if (k == (int)m->staged.size()) m->staged.emplace_back();
        m->staged[k] = s;
        *slot = k;
    });
}

int laya_model_objective_rlcd(laya_model* m, const float* targets_host, const double* draws_host, int groups,
                              double sigma, double spherical_weight, double rps_weight, double ce_weight,
                              double scale, double* losses_host) {
    return guarded([&] {
        checked(m);
        LAYA_REQUIRE(m->has_tape, "objective: run forward first");
        LAYA_REQUIRE(groups >= 0, "objective: negative group count");
        LAYA_REQUIRE(m->nmark == 0 || (targets_host && (groups == 0 || draws_host)), "objective: null targets or draws");
        const size_t draws = (size_t)groups * m->nmark;
        if (m->draws_cap < draws) {
            if (m->d_draws) m->ctx->release(m->d_draws);
            m->d_draws = static_cast<double*>(m->ctx->alloc(sizeof(double) * draws));
            m->draws_cap = draws;
        }
        if (!m->d_rlcd_losses) m->d_rlcd_losses = static_cast<double*>(m->ctx->alloc(sizeof(double) * 4));
        if (m->nmark) {
            LAYA_HIP(hipMemcpyAsync(m->targets, targets_host, sizeof(float) * m->nmark, hipMemcpyHostToDevice,
                                    m->ctx->stream));
            if (draws)
                LAYA_HIP(hipMemcpyAsync(m->d_draws, draws_host, sizeof(double) * draws, hipMemcpyHostToDevice,
                                        m->ctx->stream));
        }
        rlcd_objective(m->ctx, m->scores, m->targets, m->cur.opt_off, m->cur.qtypes, m->nseg, m->nmark, m->max_opts,
                       groups, m->d_draws, sigma, spherical_weight, rps_weight, ce_weight, scale, m->ds_scores,
                       m->d_rlcd_losses);
        if (losses_host) {
            LAYA_HIP(hipMemcpyAsync(losses_host, m->d_rlcd_losses, sizeof(double) * 4, hipMemcpyDeviceToHost,
                                    m->ctx->stream));
            LAYA_HIP(hipStreamSynchronize(m->ctx->stream));
        }
    });
}

int laya_model_backward_fallback(laya_model* m, int* split3) {
    return guarded([&] {
        checked(m);
        LAYA_REQUIRE(split3, "backward_fallback: null argument");
        *split3 = m->backward_split3 ? 1 : 0;
    });
}

int laya_model_backward_from_objective(laya_model* m) {
    return guarded([&] {
        checked(m);
        LAYA_REQUIRE(m->has_tape, "backward: run forward first");
        backward(m);
    });
}

int laya_model_release_batch(laya_model* m, int slot) {
    return guarded([&] {
        checked(m);
        StagedBatch& s = staged_slot(m, slot);
        if (m->cur.tokens == s.tables.tokens) {  // it was the current batch: its tape goes with it
            m->cur = m->own;
            m->has_tape = false;
        }
        m->ctx->release(s.block);
        s = StagedBatch{};
    });
}

int laya_model_train_step_staged(laya_model* m, int slot, float ce_weight, float loss_scale, uint64_t seed,
                                 double max_norm, double lr_encoder, double lr_head, double beta1, double beta2,
                                 double eps, double weight_decay, float* loss_out) {
    return guarded([&] {
        checked(m);
        const StagedBatch& s = staged_slot(m, slot);
        set_batch_sizes(m, s);
        m->cur = s.tables;
        train_step_current(m, s.targets, ce_weight, loss_scale, seed, max_norm, lr_encoder, lr_head, beta1, beta2,
                           eps, weight_decay, loss_out);
    });
}

int laya_model_steps(laya_model* m, int* steps) {
    return guarded([&] { *steps = checked(m)->steps; });
}

// Optimizer state in and out, one parameter at a time, for checkpoints that resume training.
int laya_model_get_moments(laya_model* m, int i, float* m1_host, float* m2_host) {
    return guarded([&] {
        checked(m);
        LAYA_REQUIRE(i >= 0 && i < (int)m->params.size() && m1_host && m2_host, "get_moments: bad argument");
        const Param& p = m->params[i];
        if (!m->M1) {  // no step taken yet: both moments are zero
            std::fill(m1_host, m1_host + p.numel, 0.0f);
            std::fill(m2_host, m2_host + p.numel, 0.0f);
            return;
        }
        LAYA_HIP(hipMemcpyAsync(m1_host, m->M1 + p.offset, p.numel * sizeof(float), hipMemcpyDeviceToHost,
                                m->ctx->stream));
        LAYA_HIP(hipMemcpyAsync(m2_host, m->M2 + p.offset, p.numel * sizeof(float), hipMemcpyDeviceToHost,
                                m->ctx->stream));
        LAYA_HIP(hipStreamSynchronize(m->ctx->stream));
    });
}

int laya_model_set_moments(laya_model* m, int i, const float* m1_host, const float* m2_host) {
    return guarded([&] {
        checked(m);
        LAYA_REQUIRE(i >= 0 && i < (int)m->params.size() && m1_host && m2_host, "set_moments: bad argument");
        const Param& p = m->params[i];
        ensure_moments(m);
        LAYA_HIP(hipMemcpyAsync(m->M1 + p.offset, m1_host, p.numel * sizeof(float), hipMemcpyHostToDevice,
                                m->ctx->stream));
        LAYA_HIP(hipMemcpyAsync(m->M2 + p.offset, m2_host, p.numel * sizeof(float), hipMemcpyHostToDevice,
                                m->ctx->stream));
        LAYA_HIP(hipStreamSynchronize(m->ctx->stream));
    });
}

int laya_model_set_steps(laya_model* m, int steps) {
    return guarded([&] {
        checked(m);
        LAYA_REQUIRE(steps >= 0, "set_steps: negative step count");
        m->steps = steps;
    });
}

}  // extern "C"
