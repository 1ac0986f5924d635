// The RLCD training objective on the device (src/StructuredDecisions.Laya.Training/RlcdObjective.cs:57-155),
// with the standard-normal draws supplied by the caller, as in the second RlcdObjective.Compute overload.
//
// Per item i with K options and group g: ε = σ·z projected to zero mean; q = softmax(l + ε) (float, as
// SimdOps.Softmax); reward = Calibration.ProperReward(q, t) (log score floored at −9.21, + spherical
// score, − RPS for score questions; Calibration.cs:76-119). Advantages are rewards minus the item's
// group mean, divided by the unbiased standard deviation over all samples (+1e-6). Gradient per option:
// −Σ_g adv·ε/σ²/(G·n) + w_CE·(p·Σt − t)/n with p = softmax(l), all times `scale`.
//
// The work is items × options × groups (thousands of values), so it runs in one workgroup: threads
// take (group, item) samples and then items, and every sum the result depends on (advantage mean and
// variance, the losses) is taken by one thread in the reference's loop order, so the result never
// depends on timing.
#include "common.hpp"

namespace laya {
namespace {

constexpr int THREADS = 256;

struct RlcdArgs {
    const float* logits;    // [Σ K]
    const float* targets;   // [Σ K]
    const int* offsets;     // [n + 1] option offsets of the items
    const int* qtypes;      // [n]
    const double* draws;    // [G][Σ K] standard normal
    int n, groups;
    double sigma, spherical, rps, ce_weight, scale;
    double* eps;            // scratch [G][Σ K]
    double* reward;         // scratch [G][n], then the normalised advantages
    double* item_terms;     // scratch [n][3]: policy, ce, reward sums of each item
    float* grad;            // [Σ K]
    double* losses;         // [4]: total, policy, cross-entropy, mean reward
};

// SimdOps.Softmax (SimdOps.cs:274-297) in float: shift by the max, exponentiate, normalise.
__device__ void softmax_inplace(float* v, int k) {
    float mx = -__builtin_huge_valf();
    for (int o = 0; o < k; ++o) mx = fmaxf(mx, v[o]);
    float total = 0.0f;
    for (int o = 0; o < k; ++o) {
        v[o] = expf(v[o] - mx);
        total += v[o];
    }
    const float inv = 1.0f / total;
    for (int o = 0; o < k; ++o) v[o] *= inv;
}

// Calibration.ProperReward with every option unmasked.
__device__ double proper_reward(const float* q, const float* t, int k, int qtype, double spherical, double rps_w) {
    double log_score = 0.0, dot = 0.0, norm2 = 0.0;
    for (int o = 0; o < k; ++o) {
        const double qo = q[o];
        log_score += t[o] * fmax(log(fmax(qo, 1e-12)), -9.21);
        dot += t[o] * qo;
        norm2 += qo * qo;
    }
    const double reward = log_score + spherical * (dot / fmax(sqrt(norm2), 1e-9));
    if (qtype != 1) return reward;  // ordinal "score" questions also pay the ranked probability score
    double cq = 0.0, ct = 0.0, rps = 0.0;
    for (int o = 0; o < k; ++o) {
        cq += q[o];
        ct += t[o];
        rps += (cq - ct) * (cq - ct);
    }
    return reward - rps_w * rps / (max(k, 2) - 1);
}

constexpr int MAX_OPTIONS = 64;

__global__ __launch_bounds__(THREADS) void rlcd_kernel(RlcdArgs a) {
    const int n = a.n, G = a.groups, P = a.offsets[n];
    // 1. Centred noise, perturbed softmax and reward of every (group, item) sample.
    for (int s = threadIdx.x; s < G * n; s += THREADS) {
        const int g = s / n, i = s - g * n;
        const int b = a.offsets[i], k = a.offsets[i + 1] - b;
        const double* z = a.draws + (long)g * P + b;
        double* e = a.eps + (long)g * P + b;
        double mean = 0.0;
        for (int o = 0; o < k; ++o) {
            e[o] = z[o] * a.sigma;
            mean += e[o];
        }
        mean /= k;
        float q[MAX_OPTIONS];
        for (int o = 0; o < k; ++o) {
            e[o] -= mean;
            q[o] = (float)(a.logits[b + o] + e[o]);
        }
        softmax_inplace(q, k);
        a.reward[(long)g * n + i] = proper_reward(q, a.targets + b, k, a.qtypes[i], a.spherical, a.rps);
    }
    __syncthreads();
    // 2. Group-relative advantages and the global standard deviation, in the reference's order.
    __shared__ double sd_s;
    __shared__ double mean_reward_s;
    if (threadIdx.x == 0) {
        double total = 0.0, reward_sum = 0.0;
        for (int i = 0; i < n; ++i) {
            double mean = 0.0;
            for (int g = 0; g < G; ++g) mean += a.reward[(long)g * n + i];
            mean /= G;
            for (int g = 0; g < G; ++g) {
                reward_sum += a.reward[(long)g * n + i];
                a.reward[(long)g * n + i] -= mean;
                total += a.reward[(long)g * n + i];
            }
        }
        const int count = G * n;
        const double gmean = total / count;
        double var = 0.0;
        for (int g = 0; g < G; ++g)
            for (int i = 0; i < n; ++i) {
                const double d = a.reward[(long)g * n + i] - gmean;
                var += d * d;
            }
        sd_s = count > 1 ? sqrt(var / (count - 1)) : 0.0;
        mean_reward_s = reward_sum / count;
    }
    __syncthreads();
    const double denom = sd_s + 1e-6;
    // 3. Per item: policy-gradient and cross-entropy terms of the gradient and of the losses.
    const int count = G * n;
    const double s2 = a.sigma * a.sigma;
    for (int i = threadIdx.x; i < n; i += THREADS) {
        const int b = a.offsets[i], k = a.offsets[i + 1] - b;
        double grad[MAX_OPTIONS];
        for (int o = 0; o < k; ++o) grad[o] = 0.0;
        double policy = 0.0;
        for (int g = 0; g < G; ++g) {
            const double adv = a.reward[(long)g * n + i] / denom;
            const double* e = a.eps + (long)g * P + b;
            double logp = 0.0;
            for (int o = 0; o < k; ++o) {
                logp -= e[o] * e[o] / (2 * s2);
                grad[o] -= adv * e[o] / s2 / count;
            }
            policy -= adv * logp / count;
        }
        float p[MAX_OPTIONS];
        for (int o = 0; o < k; ++o) p[o] = a.logits[b + o];
        softmax_inplace(p, k);
        double mass = 0.0, ce = 0.0;
        for (int o = 0; o < k; ++o) mass += a.targets[b + o];
        for (int o = 0; o < k; ++o) {
            ce -= a.targets[b + o] * log(fmax((double)p[o], 1e-30)) / n;
            grad[o] += a.ce_weight * (p[o] * mass - a.targets[b + o]) / n;
        }
        for (int o = 0; o < k; ++o) a.grad[b + o] = (float)(grad[o] * a.scale);
        a.item_terms[3 * i] = policy;
        a.item_terms[3 * i + 1] = ce;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        double policy = 0.0, ce = 0.0;
        for (int i = 0; i < n; ++i) {
            policy += a.item_terms[3 * i];
            ce += a.item_terms[3 * i + 1];
        }
        a.losses[0] = policy + a.ce_weight * ce;
        a.losses[1] = policy;
        a.losses[2] = ce;
        a.losses[3] = mean_reward_s;
    }
}

}  // namespace

void rlcd_objective(laya_ctx* ctx, const float* logits, const float* targets, const int* offsets, const int* qtypes,
                    int n_items, int total_options, int max_options, int groups, const double* draws, double sigma,
                    double spherical, double rps, double ce_weight, double scale, float* grad, double* losses) {
    // Zero groups is the cross-entropy-only objective: the policy term vanishes and the mean reward is
    // 0/0, NaN, as in the reference. Zero items still writes the losses.
    LAYA_REQUIRE(n_items >= 0 && groups >= 0 && total_options >= 0, "rlcd: bad size");
    LAYA_REQUIRE(max_options <= MAX_OPTIONS, "rlcd: at most 64 options per item");
    LAYA_REQUIRE(groups == 0 || sigma > 0.0, "rlcd: sigma must be positive");
    LAYA_REQUIRE(offsets && losses, "rlcd: null offsets or losses");
    const size_t scratch = sizeof(double) * ((size_t)groups * total_options + (size_t)groups * n_items + 3 * (size_t)n_items);
    double* base = static_cast<double*>(ctx->workspace(5, std::max<size_t>(scratch, 64)));
    RlcdArgs a{};
    a.logits = logits;
    a.targets = targets;
    a.offsets = offsets;
    a.qtypes = qtypes;
    a.draws = draws;
    a.n = n_items;
    a.groups = groups;
    a.sigma = sigma;
    a.spherical = spherical;
    a.rps = rps;
    a.ce_weight = ce_weight;
    a.scale = scale;
    a.eps = base;
    a.reward = base + (size_t)groups * total_options;
    a.item_terms = a.reward + (size_t)groups * n_items;
    a.grad = grad;
    a.losses = losses;
    ProfileScope scope(ctx, "rlcd_objective", 0.0, 0.0);
    LAYA_LAUNCH(rlcd_kernel, dim3(1), dim3(THREADS), 0, ctx->stream, a);
    check_launch("rlcd_kernel");
}

}  // namespace laya
