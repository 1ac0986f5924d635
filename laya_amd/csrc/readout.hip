// The decision read-out on the device: DecisionModel.ReadOut
// (src/StructuredDecisions.Laya/Models/DecisionModel.cs:170-226) for every item of the last forward.
//
// One workgroup per item. From the item's option logits (the scorer's output): the untempered softmax
// as SimdOps.Softmax computes it (max, e = exp(v − max), Σe, then e·(1/Σe)), the entropy −Σ p·log(max(p,
// 1e-9)) over log(max(2, K)), the top probability and its margin over the second (strict comparisons in
// option order). With the item's first head-output row (pooled = h[start]) they form the act head's input
// [h, top1, top1 − top2, entropy, k/255]; its MLP (Linear → exact GELU → Linear) and a softmax give the
// action probabilities. Each output of a Linear is one wave's dot product.
#include "common.hpp"

namespace laya {
namespace {

constexpr int RO_THREADS = 256;

__device__ float wave_dot(const float* __restrict__ x, const float* __restrict__ w, int n, int lane) {
    float s = 0.0f;
    for (int i = lane; i < n; i += 64) s += x[i] * w[i];
    return wave_sum(s);
}

__global__ __launch_bounds__(RO_THREADS) void readout_kernel(const float* __restrict__ scores,
                                                            const int* __restrict__ opt_off,
                                                            const int* __restrict__ seg_start,
                                                            const float* __restrict__ states, int d,
                                                            const float* __restrict__ w1, const float* __restrict__ b1,
                                                            int a1, const float* __restrict__ w2,
                                                            const float* __restrict__ b2, int na,
                                                            float* __restrict__ probs, float* __restrict__ features) {
    extern __shared__ float sh[];  // x [d + 4], hidden [a1], act logits [na]
    float* x = sh;
    float* hid = x + d + 4;
    float* out = hid + a1;
    const int item = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int o0 = opt_off[item], K = opt_off[item + 1] - o0;
    const float* h = states + (long)seg_start[item] * d;
    for (int i = tid; i < d; i += RO_THREADS) x[i] = h[i];
    if (tid == 0) {
        float mx = -__builtin_huge_valf();
        for (int o = 0; o < K; ++o) mx = fmaxf(mx, scores[o0 + o]);
        float top1 = 0.0f, top2 = 0.0f, entropy = 0.0f;
        if (K > 0 && mx != -__builtin_huge_valf()) {
            float total = 0.0f;
            for (int o = 0; o < K; ++o) total += expf(scores[o0 + o] - mx);
            const float scale = total > 0.0f ? 1.0f / total : 0.0f;
            for (int o = 0; o < K; ++o) {
                const float p = expf(scores[o0 + o] - mx) * scale;
                entropy -= p * logf(fmaxf(p, 1e-9f));
                if (p > top1) {
                    top2 = top1;
                    top1 = p;
                } else if (p > top2) {
                    top2 = p;
                }
            }
        }
        const float k = (float)max(2, K);
        entropy /= logf(k);
        x[d] = top1;
        x[d + 1] = top1 - top2;
        x[d + 2] = entropy;
        x[d + 3] = k / 255.0f;
        if (features) {
            features[item * 4 + 0] = top1;
            features[item * 4 + 1] = top1 - top2;
            features[item * 4 + 2] = entropy;
            features[item * 4 + 3] = k / 255.0f;
        }
    }
    __syncthreads();
    for (int o = wave; o < a1; o += RO_THREADS / 64) {
        const float v = wave_dot(x, w1 + (long)o * (d + 4), d + 4, lane) + b1[o];
        if (lane == 0) hid[o] = gelu_f(v);
    }
    __syncthreads();
    for (int o = wave; o < na; o += RO_THREADS / 64) {
        const float v = wave_dot(hid, w2 + (long)o * a1, a1, lane) + b2[o];
        if (lane == 0) out[o] = v;
    }
    __syncthreads();
    if (tid == 0) {
        float mx = -__builtin_huge_valf();
        for (int o = 0; o < na; ++o) mx = fmaxf(mx, out[o]);
        float total = 0.0f;
        for (int o = 0; o < na; ++o) total += expf(out[o] - mx);
        const float scale = total > 0.0f ? 1.0f / total : 0.0f;
        for (int o = 0; o < na; ++o) probs[item * na + o] = expf(out[o] - mx) * scale;
    }
}

}  // namespace

void decision_readout(laya_ctx* ctx, const float* scores, const int* opt_off, const int* seg_start, int n_items,
                      const float* states, int d, const float* w1, const float* b1, int a1, const float* w2,
                      const float* b2, int na, float* probs, float* features) {
    if (n_items <= 0) return;
    LAYA_REQUIRE(d > 0 && a1 > 0 && na > 0, "readout: bad act-head shape");
    const size_t lds = sizeof(float) * (size_t)(d + 4 + a1 + na);
    LAYA_REQUIRE(lds <= 64 * 1024, "readout: act-head input too wide for one workgroup");
    ProfileScope scope(ctx, "decision_readout", 0.0, 4.0 * n_items * ((double)d + (double)a1 * (d + 4)));
    LAYA_LAUNCH(readout_kernel, dim3(n_items), dim3(RO_THREADS), lds, ctx->stream, scores, opt_off, seg_start,
                       states, d, w1, b1, a1, w2, b2, na, probs, features);
    check_launch("readout_kernel");
}

}  // namespace laya
