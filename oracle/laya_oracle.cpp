// Oracle (test infrastructure only; never linked into the product library).
//
// A CPU restatement of the reference's C# fine-tuning path, templated over the arithmetic type:
// fp32 restates what the reference computes, fp64 runs the same algorithm as a mathematical pin.
// Each function cites the reference file:line it follows. The structure is the reference's own
// (per-layer recompute in the backward pass, per-(segment, head) attention units), so the same
// code is also the CPU baseline that is timed beside the GPU.
//
// Compiled with -ffp-contract=off: C# never contracts a*b+c into an FMA unless it says so
// (Vector.FusedMultiplyAdd / FusedAdd), and those places call std::fma explicitly here.
#include "laya_oracle.h"

#include <algorithm>
#include <cmath>
#include <cstdint>
#include <cstring>
#include <map>
#include <memory>
#include <stdexcept>
#include <string>
#include <vector>
#include <omp.h>

namespace oracle {

template <typename R>
void gemm(int M, int N, int K, const R* A, long sam, long sak, const R* B, long sbk, long sbn, R* C, long ldc,
          bool accumulate);

using u64 = uint64_t;
static thread_local std::string g_error;

// ------------------------------------------------------------------ counter RNG (Ops.cs:227-241)

static inline float uniform(u64 seed, u64 index) {
    u64 z = seed + (index + 1) * 0x9E3779B97F4A7C15ULL;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ULL;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBULL;
    z ^= z >> 31;
    return (float)(z >> 40) * (1.0f / (float)(1 << 24));
}

static inline u64 mix(u64 seed, u64 salt) {
    u64 z = seed ^ (salt * 0xD1B54A32D192ED03ULL + 0x8CB92BA72F3D8DD7ULL);
    z = (z ^ (z >> 33)) * 0xFF51AFD7ED558CCDULL;
    return z ^ (z >> 33);
}

// Ops.cs:318: ((ulong)head << 42) | ((ulong)row << 21) | (uint)key
static inline u64 dropout_index(int head, int row, int key) {
    return ((u64)head << 42) | ((u64)(int64_t)row << 21) | (u64)(uint32_t)key;
}

// ------------------------------------------------- float exp / erf (SimdOps.cs:329-390)

static inline float exp_ref(float value) {
    // Cody-Waite range reduction to 2^n e^r, degree-6 Taylor series on r (SimdOps.cs:368-390).
    const float log2e = 1.4426950408889634f, ln2_hi = 0.693359375f, ln2_lo = -2.12194440e-4f;
    float x = std::min(std::max(value, -87.3f), 88.7f);
    float n = std::floor(std::fma(x, log2e, 0.5f));
    float r = std::fma(n, -ln2_hi, x);
    r = std::fma(n, -ln2_lo, r);
    float p = 1.0f / 720.0f;
    p = std::fma(p, r, 1.0f / 120.0f);
    p = std::fma(p, r, 1.0f / 24.0f);
    p = std::fma(p, r, 1.0f / 6.0f);
    p = std::fma(p, r, 0.5f);
    p = std::fma(p, r, 1.0f);
    p = std::fma(p, r, 1.0f);
    int32_t bits = ((int32_t)n + 127) << 23;
    float scale;
    std::memcpy(&scale, &bits, 4);
    return p * scale;
}

static inline float erf_ref(float value) {
    // Numerical Recipes erfc rational form (SimdOps.cs:329-356), float lanes.
    float sign = value < 0.0f ? -1.0f : 1.0f;
    float ax = std::fabs(value);
    float t = 1.0f / (1.0f + 0.5f * ax);
    float poly = 0.17087277f;
    poly = std::fma(poly, t, -0.82215223f);
    poly = std::fma(poly, t, 1.48851587f);
    poly = std::fma(poly, t, -1.13520398f);
    poly = std::fma(poly, t, 0.27886807f);
    poly = std::fma(poly, t, -0.18628806f);
    poly = std::fma(poly, t, 0.09678418f);
    poly = std::fma(poly, t, 0.37409196f);
    poly = std::fma(poly, t, 1.00002368f);
    poly = std::fma(poly, t, -1.26551223f);
    poly -= ax * ax;
    float y = t * exp_ref(poly);
    return sign * (ax > 6.0f ? 1.0f : 1.0f - y);
}

// Exact GELU (SimdOps.cs:305-323); fp64 uses the library erf.
template <typename R> static inline R gelu(R x);
template <> inline float gelu<float>(float x) { return x * 0.5f * (1.0f + erf_ref(x * 0.70710678118654752f)); }
template <> inline double gelu<double>(double x) { return x * 0.5 * (1.0 + std::erf(x * 0.70710678118654752440)); }

// d gelu / dx = Φ(x) + x φ(x) (Ops.cs:194-218).
template <typename R> static inline R gelu_grad(R x);
template <> inline float gelu_grad<float>(float x) {
    float cdf = 0.5f * (1.0f + erf_ref(x * 0.70710678118654752f));
    float pdf = 0.39894228040143268f * exp_ref(-0.5f * x * x);
    return cdf + x * pdf;
}
template <> inline double gelu_grad<double>(double x) {
    double cdf = 0.5 * (1.0 + std::erf(x * 0.70710678118654752440));
    double pdf = 0.39894228040143267794 * std::exp(-0.5 * x * x);
    return cdf + x * pdf;
}

// MathF.Exp in the softmax (SimdOps.cs:286).
template <typename R> static inline R soft_exp(R x) { return std::exp(x); }

// --------------------------------------------------------------------- small vector helpers

// SimdOps.Dot (SimdOps.cs:61-81): two 8-lane FMA accumulators, then lane sums.
template <typename R> static inline R dot(const R* a, const R* b, int n) {
    R s0[8] = {}, s1[8] = {};
    int i = 0;
    for (; i + 16 <= n; i += 16) {
        for (int l = 0; l < 8; ++l) {
            s0[l] = std::fma(a[i + l], b[i + l], s0[l]);
            s1[l] = std::fma(a[i + 8 + l], b[i + 8 + l], s1[l]);
        }
    }
    for (; i + 8 <= n; i += 8)
        for (int l = 0; l < 8; ++l) s0[l] = std::fma(a[i + l], b[i + l], s0[l]);
    R x = 0, y = 0;
    for (int l = 0; l < 8; ++l) x += s0[l];
    for (int l = 0; l < 8; ++l) y += s1[l];
    R sum = x + y;
    for (; i < n; ++i) sum += a[i] * b[i];
    return sum;
}

// SimdOps.AddScaled (SimdOps.cs:137-149): destination += source * scale, fused.
template <typename R> static inline void add_scaled(R* dst, const R* src, int n, R scale) {
    for (int i = 0; i < n; ++i) dst[i] = std::fma(src[i], scale, dst[i]);
}

template <typename R> static inline void add(R* dst, const R* src, long n) {
    for (long i = 0; i < n; ++i) dst[i] += src[i];
}

// SimdOps.Softmax (SimdOps.cs:275-291).
template <typename R> static void softmax(R* v, int n) {
    if (n == 0) return;
    R mx = v[0];
    for (int i = 1; i < n; ++i) mx = std::max(mx, v[i]);
    if (std::isinf(mx) && mx < 0) {
        std::fill(v, v + n, R(0));
        return;
    }
    R total = 0;
    for (int i = 0; i < n; ++i) {
        R e = soft_exp<R>(v[i] - mx);
        v[i] = e;
        total += e;
    }
    R s = total > 0 ? R(1) / total : R(0);
    for (int i = 0; i < n; ++i) v[i] *= s;
}

// ----------------------------------------------------------------------------- rotary (Ops.cs:446-504)

template <typename R> struct Rotary {
    int head_dim = 0, positions = 0;
    double theta = 0;
    std::vector<R> cos_, sin_;
    Rotary() = default;
    Rotary(int hd, double th) : head_dim(hd), theta(th) { grow(1024); }
    void grow(int p) {
        if (p <= positions) return;
        int half = head_dim / 2;
        cos_.assign((size_t)p * half, R(0));
        sin_.assign((size_t)p * half, R(0));
        for (int i = 0; i < half; ++i) {
            double inv = 1.0 / std::pow(theta, 2.0 * i / head_dim);
            for (int q = 0; q < p; ++q) {
                double angle = q * inv;
                cos_[(size_t)q * half + i] = (R)std::cos(angle);
                sin_[(size_t)q * half + i] = (R)std::sin(angle);
            }
        }
        positions = p;
    }
    void apply(R* v, int pos, bool inverse) const {
        int half = head_dim / 2;
        const R* c = cos_.data() + (size_t)pos * half;
        const R* s0 = sin_.data() + (size_t)pos * half;
        for (int i = 0; i < half; ++i) {
            R a = v[i], b = v[i + half];
            R s = inverse ? -s0[i] : s0[i];
            v[i] = a * c[i] - b * s;
            v[i + half] = b * c[i] + a * s;
        }
    }
};

// ------------------------------------------------------------------------- attention (Ops.cs:263-438)

struct Segment {
    int start, length;
};

template <typename R> struct AttentionShape {
    int hidden, heads;
    R scale;
    int half_window;  // INT32_MAX: no window
    const Rotary<R>* rotary;
    float dropout;
    u64 seed;
    int head_dim() const { return hidden / heads; }
};

template <typename R>
static void gather(const R* qkv, const Segment& seg, int head, const AttentionShape<R>& s, R* q, R* k, R* v) {
    int hidden = s.hidden, d = s.head_dim();
    long stride = 3L * hidden;
    for (int t = 0; t < seg.length; ++t) {
        const R* row = qkv + (long)(seg.start + t) * stride + head * d;
        std::memcpy(q + (long)t * d, row, sizeof(R) * d);
        std::memcpy(k + (long)t * d, row + hidden, sizeof(R) * d);
        std::memcpy(v + (long)t * d, row + 2 * hidden, sizeof(R) * d);
        if (s.rotary) {
            s.rotary->apply(q + (long)t * d, t, false);
            s.rotary->apply(k + (long)t * d, t, false);
        }
    }
}

static inline void window(int t, int length, int half, int& first, int& last) {
    if (half == INT32_MAX) {
        first = 0;
        last = length - 1;
    } else {
        first = std::max(0, t - half);
        last = std::min(length - 1, t + half);
    }
}

template <typename R>
static void probabilities(const R* q, const R* k, int t, int first, int count, int d, R scale, R* p) {
    const R* query = q + (long)t * d;
    for (int j = 0; j < count; ++j) p[j] = scale * dot(query, k + (long)(first + j) * d, d);
    softmax(p, count);
}

template <typename R>
static void forward_unit(const R* qkv, const Segment& seg, int head, const AttentionShape<R>& s, R* context) {
    int L = seg.length, d = s.head_dim(), hidden = s.hidden;
    std::vector<R> buf(3L * L * d + L);
    R *q = buf.data(), *k = q + (long)L * d, *v = k + (long)L * d, *p = v + (long)L * d;
    gather(qkv, seg, head, s, q, k, v);
    R keep = R(1) / (R(1) - R(s.dropout));
    for (int t = 0; t < L; ++t) {
        int first, last;
        window(t, L, s.half_window, first, last);
        int count = last - first + 1;
        probabilities(q, k, t, first, count, d, s.scale, p);
        R* out = context + (long)(seg.start + t) * hidden + head * d;
        std::fill(out, out + d, R(0));
        for (int j = 0; j < count; ++j) {
            R w = p[j];
            if (s.dropout > 0.0f)
                w = uniform(s.seed, dropout_index(head, seg.start + t, first + j)) < s.dropout ? R(0) : w * keep;
            if (w != R(0)) add_scaled(out, v + (long)(first + j) * d, d, w);
        }
    }
}

template <typename R>
static void backward_unit(const R* qkv, const Segment& seg, int head, const AttentionShape<R>& s, const R* dcontext,
                          R* dqkv) {
    int L = seg.length, d = s.head_dim(), hidden = s.hidden;
    long stride = 3L * hidden;
    std::vector<R> buf(6L * L * d + 3L * L, R(0));
    R *q = buf.data(), *k = q + (long)L * d, *v = k + (long)L * d;
    R *dq = v + (long)L * d, *dk = dq + (long)L * d, *dv = dk + (long)L * d;
    R *p = dv + (long)L * d, *dp = p + L, *mask = dp + L;
    gather(qkv, seg, head, s, q, k, v);
    R keep = R(1) / (R(1) - R(s.dropout));
    for (int t = 0; t < L; ++t) {
        int first, last;
        window(t, L, s.half_window, first, last);
        int count = last - first + 1;
        probabilities(q, k, t, first, count, d, s.scale, p);
        const R* up = dcontext + (long)(seg.start + t) * hidden + head * d;
        for (int j = 0; j < count; ++j) {
            mask[j] = s.dropout > 0.0f
                          ? (uniform(s.seed, dropout_index(head, seg.start + t, first + j)) < s.dropout ? R(0) : keep)
                          : R(1);
            R dropped = p[j] * mask[j];
            if (dropped != R(0)) add_scaled(dv + (long)(first + j) * d, up, d, dropped);
            dp[j] = dot(up, v + (long)(first + j) * d, d) * mask[j];
        }
        R c = 0;
        for (int j = 0; j < count; ++j) c += p[j] * dp[j];
        R* dquery = dq + (long)t * d;
        const R* query = q + (long)t * d;
        for (int j = 0; j < count; ++j) {
            R ds = s.scale * p[j] * (dp[j] - c);
            if (ds == R(0)) continue;
            add_scaled(dquery, k + (long)(first + j) * d, d, ds);
            add_scaled(dk + (long)(first + j) * d, query, d, ds);
        }
    }
    for (int t = 0; t < L; ++t) {
        if (s.rotary) {
            s.rotary->apply(dq + (long)t * d, t, true);
            s.rotary->apply(dk + (long)t * d, t, true);
        }
        R* row = dqkv + (long)(seg.start + t) * stride + head * d;
        std::memcpy(row, dq + (long)t * d, sizeof(R) * d);
        std::memcpy(row + hidden, dk + (long)t * d, sizeof(R) * d);
        std::memcpy(row + 2 * hidden, dv + (long)t * d, sizeof(R) * d);
    }
}

// Ops.RunUnits (Ops.cs:284-294): one unit per (segment, head), in parallel.
template <typename R>
static void attention_forward(const R* qkv, const std::vector<Segment>& segs, const AttentionShape<R>& s, R* context) {
    long units = (long)segs.size() * s.heads;
#pragma omp parallel for schedule(dynamic, 1)
    for (long u = 0; u < units; ++u) forward_unit(qkv, segs[u / s.heads], (int)(u % s.heads), s, context);
}

template <typename R>
static void attention_backward(const R* qkv, const std::vector<Segment>& segs, const AttentionShape<R>& s,
                               const R* dcontext, R* dqkv) {
    long units = (long)segs.size() * s.heads;
#pragma omp parallel for schedule(dynamic, 1)
    for (long u = 0; u < units; ++u) backward_unit(qkv, segs[u / s.heads], (int)(u % s.heads), s, dcontext, dqkv);
}

// ---------------------------------------------------------------------------- dense ops (Ops.cs)

// Ops.Linear (Ops.cs:22-27): y = x · Wᵀ + b.
template <typename R> static void linear(const R* x, int rows, int in, const R* W, int out, const R* b, R* y) {
    gemm<R>(rows, out, in, x, in, 1, W, 1, in, y, out, false);
    if (b) {
#pragma omp parallel for schedule(static)
        for (int r = 0; r < rows; ++r) add(y + (long)r * out, b, out);
    }
}

// Ops.LinearBackward (Ops.cs:33-69): dx = dy·W (overwrite), dW += dyᵀ·x (a fresh product, then added,
// as AddParallel does), db += Σ_rows dy.
template <typename R>
static void linear_backward(const R* x, const R* dy, int rows, int in, int out, const R* W, R* dx, R* dW, R* db) {
    if (dx) gemm<R>(rows, in, out, dy, out, 1, W, in, 1, dx, in, false);
    if (dW) {
        std::vector<R> product((size_t)out * in);
        gemm<R>(out, in, rows, dy, 1, out, x, in, 1, product.data(), in, false);
        long n = (long)out * in;
#pragma omp parallel for schedule(static)
        for (long i = 0; i < n; ++i) dW[i] += product[i];
    }
    if (db) {
        for (int r = 0; r < rows; ++r) add(db, dy + (long)r * out, out);
    }
}

// SimdOps.LayerNorm (SimdOps.cs:234-272) per row, Ops.LayerNorm (Ops.cs:103-110) over rows.
template <typename R> static void layernorm_row(const R* in, const R* w, const R* b, R eps, R* out, int n) {
    R lanes[8] = {};
    int i = 0;
    for (; i + 8 <= n; i += 8)
        for (int l = 0; l < 8; ++l) lanes[l] += in[i + l];
    R sum = 0;
    for (int l = 0; l < 8; ++l) sum += lanes[l];
    for (; i < n; ++i) sum += in[i];
    R mean = sum / n;
    R vl[8] = {};
    i = 0;
    for (; i + 8 <= n; i += 8)
        for (int l = 0; l < 8; ++l) {
            R dd = in[i + l] - mean;
            vl[l] = std::fma(dd, dd, vl[l]);
        }
    R var = 0;
    for (int l = 0; l < 8; ++l) var += vl[l];
    for (; i < n; ++i) {
        R dd = in[i] - mean;
        var += dd * dd;
    }
    var /= n;
    R inv = R(1) / std::sqrt(var + eps);
    for (i = 0; i < n; ++i) {
        R v = (in[i] - mean) * inv * w[i];
        out[i] = b ? v + b[i] : v;
    }
}

template <typename R>
static void layernorm(const R* x, int rows, int n, const R* w, const R* b, R eps, R* y) {
#pragma omp parallel for schedule(static)
    for (int r = 0; r < rows; ++r) layernorm_row(x + (long)r * n, w, b, eps, y + (long)r * n, n);
}

// Ops.LayerNormBackward (Ops.cs:117-186): stats recomputed in double, dx added, dγ/dβ accumulated.
template <typename R>
static void layernorm_backward(const R* x, int rows, int n, const R* gamma, R eps, const R* dy, R* dx, R* dgamma,
                               R* dbeta) {
    std::vector<R> mean(rows), rstd(rows);
#pragma omp parallel for schedule(static)
    for (int r = 0; r < rows; ++r) {
        const R* row = x + (long)r * n;
        double sum = 0;
        for (int i = 0; i < n; ++i) sum += row[i];
        double mu = sum / n;
        double variance = 0;
        for (int i = 0; i < n; ++i) variance += (row[i] - mu) * (row[i] - mu);
        variance /= n;
        R m = (R)mu;
        R inv = (R)(1.0 / std::sqrt(variance + (double)eps));
        mean[r] = m;
        rstd[r] = inv;
        const R* g = dy + (long)r * n;
        R* out = dx + (long)r * n;
        double sum_g = 0, sum_gx = 0;
        for (int i = 0; i < n; ++i) {
            double gi = g[i] * gamma[i];
            double xhat = (row[i] - m) * inv;
            sum_g += gi;
            sum_gx += gi * xhat;
        }
        R mean_g = (R)(sum_g / n), mean_gx = (R)(sum_gx / n);
        for (int i = 0; i < n; ++i) {
            R xhat = (row[i] - m) * inv;
            out[i] += inv * (g[i] * gamma[i] - mean_g - xhat * mean_gx);
        }
    }
    if (!dgamma && !dbeta) return;
    const int block = 64;
    int blocks = (n + block - 1) / block;
#pragma omp parallel for schedule(static)
    for (int bk = 0; bk < blocks; ++bk) {
        int c0 = bk * block, c1 = std::min(n, c0 + block);
        double ga[64] = {}, ba[64] = {};
        for (int r = 0; r < rows; ++r) {
            long off = (long)r * n;
            for (int c = c0; c < c1; ++c) {
                R g = dy[off + c];
                ga[c - c0] += g * (x[off + c] - mean[r]) * rstd[r];
                ba[c - c0] += g;
            }
        }
        for (int c = c0; c < c1; ++c) {
            if (dgamma) dgamma[c] += (R)ga[c - c0];
            if (dbeta) dbeta[c] += (R)ba[c - c0];
        }
    }
}

// Ops.Dropout (Ops.cs:244-258): inverted dropout in place; its own backward.
template <typename R> static void dropout(R* values, long n, float p, u64 seed) {
    if (p <= 0.0f) return;
    R scale = R(1) / (R(1) - R(p));
#pragma omp parallel for schedule(static)
    for (long i = 0; i < n; ++i) values[i] = uniform(seed, (u64)i) < p ? R(0) : values[i] * scale;
}

// GeGLU (TrainableDecisionModel.cs:390-398 and 564-579): halves [input | gate].
template <typename R> static void geglu(const R* wide, int rows, int inter, R* act) {
#pragma omp parallel for schedule(static)
    for (int t = 0; t < rows; ++t) {
        const R* row = wide + (long)t * 2 * inter;
        R* out = act + (long)t * inter;
        for (int i = 0; i < inter; ++i) out[i] = gelu<R>(row[i]) * row[inter + i];
    }
}

template <typename R> static void geglu_backward(const R* wide, const R* dact, int rows, int inter, R* dwide) {
#pragma omp parallel for schedule(static)
    for (int t = 0; t < rows; ++t) {
        const R* row = wide + (long)t * 2 * inter;
        const R* up = dact + (long)t * inter;
        R* di = dwide + (long)t * 2 * inter;
        R* dg = di + inter;
        for (int i = 0; i < inter; ++i) {
            dg[i] = gelu<R>(row[i]) * up[i];
            di[i] = up[i] * row[inter + i] * gelu_grad<R>(row[i]);
        }
    }
}

// ------------------------------------------------------------ model (TrainableDecisionModel.cs)

struct ParamInfo {
    std::string name;
    std::vector<int> shape;
    size_t offset = 0, numel = 0;
    bool trainable = true, touched = false;
};

struct ModelBase {
    virtual ~ModelBase() = default;
    std::vector<ParamInfo> params;
    std::map<std::string, int> by_name;
    orc_config cfg{};
    std::vector<int> kinds;  // 0 global, 1 sliding
    int first_trainable = 0;
    bool embeddings_trainable = true;
    float head_dropout = 0.1f;
    int steps = 0;
    // Diagnostics for the parity tests: when set, each head layer's linear1 output (the ReLU's input) of the
    // last forward is kept here in double.
    bool capture_head = false;
    std::vector<std::vector<double>> captured_head;
    virtual void set_param(int i, const float* d) = 0;
    virtual void get_param(int i, double* out) = 0;
    virtual void get_grad(int i, double* out) = 0;
    virtual void forward(int n_items, const int* lengths, const int* tokens, const int* n_options, const int* markers,
                         const int* qtypes, bool training, bool keep_tape, u64 seed, double* logits) = 0;
    virtual void backward(const float* dlogits) = 0;
    virtual void readout(float* act_probs, float* features, double* pooled) = 0;
    virtual void zero_grad() = 0;
    virtual double clip(double max_norm) = 0;
    virtual void adamw(double lr_enc, double lr_head, double b1, double b2, double eps, double wd) = 0;

    int add_param(const std::string& name, std::vector<int> shape, size_t& total) {
        ParamInfo p;
        p.name = name;
        p.shape = std::move(shape);
        p.numel = 1;
        for (int s : p.shape) p.numel *= (size_t)s;
        p.offset = total;
        total += p.numel;
        by_name[name] = (int)params.size();
        params.push_back(p);
        return (int)params.size() - 1;
    }
    int find(const std::string& name) const {
        auto it = by_name.find(name);
        return it == by_name.end() ? -1 : it->second;
    }
    int required(const std::string& name) const {
        int i = find(name);
        if (i < 0) throw std::runtime_error("the checkpoint has no '" + name + "' tensor");
        return i;
    }

    // SetTrainableEncoderLayers (TrainableDecisionModel.cs:206-231).
    void set_trainable_encoder_layers(int n) {
        int count = cfg.layers;
        int trainable = n < 0 ? count : std::clamp(n, 0, count);
        first_trainable = count - trainable;
        bool all = n < 0 || (trainable == count && n >= count);
        for (auto& p : params) {
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
            else {
                int layer = std::stoi(p.name.substr(15, p.name.find('.', 15) - 15));
                train = layer >= first_trainable;
            }
            p.trainable = train;
            if (!train) p.touched = false;
        }
        embeddings_trainable = params[find("encoder.embeddings.tok_embeddings.weight")].trainable;
        release_frozen();
    }
    virtual void release_frozen() = 0;
};

template <typename R> struct Model : ModelBase {
    std::vector<R> data, grad, m1, m2;
    Rotary<R> global_rot, local_rot;
    int hidden, head_heads;

    struct EncLayer {
        int attn_norm = -1, attn_norm_b = -1, wqkv, wqkv_b = -1, wo, wo_b = -1, mlp_norm, mlp_norm_b = -1, wi,
            wi_b = -1, mlp_wo, mlp_wo_b = -1, kind;
    };
    struct HeadLayer {
        int norm1, norm1_b, in_proj, in_proj_b, out_proj, out_proj_b, norm2, norm2_b, linear1, linear1_b, linear2,
            linear2_b;
    };
    std::vector<EncLayer> enc;
    std::vector<HeadLayer> head;
    int tok_emb, emb_norm, emb_norm_b = -1, final_norm, final_norm_b = -1, type_emb, sc_norm, sc_norm_b, sc1, sc1_b,
        sc2, sc2_b;

    // ForwardTape (TrainableDecisionModel.cs:31-54)
    struct Tape {
        bool valid = false, training = false;
        u64 seed = 0;
        std::vector<Segment> segs;
        std::vector<int> tokens, marker_rows, qtypes, n_options;
        std::vector<std::vector<R>> enc_inputs, head_inputs;
        std::vector<R> final_norm_input, embedding_input;
        bool has_final = false, has_embedding = false;
        std::vector<R> scorer_input, scorer_normed, scorer_pre, scorer_act;
    } tape;
    // What the read-out needs from the last forward: each item's first head-output row and option logits.
    std::vector<R> last_pooled, last_scores;
    std::vector<int> last_opts;
    int act1 = -1, act1_b = -1, act2 = -1, act2_b = -1;

    explicit Model(const orc_config& c) {
        cfg = c;
        hidden = c.hidden;
        head_heads = std::max(1, hidden / 64);
        size_t total = 0;
        int d = c.hidden, I = c.intermediate;
        kinds.resize(c.layers);
        for (int l = 0; l < c.layers; ++l)
            kinds[l] = c.layer_kinds ? c.layer_kinds[l] : (l % c.global_every == 0 ? 0 : 1);
        const std::string e = "encoder.";
        tok_emb = add_param(e + "embeddings.tok_embeddings.weight", {c.vocab, d}, total);
        emb_norm = add_param(e + "embeddings.norm.weight", {d}, total);
        if (c.norm_bias) emb_norm_b = add_param(e + "embeddings.norm.bias", {d}, total);
        for (int l = 0; l < c.layers; ++l) {
            std::string p = e + "layers." + std::to_string(l) + ".";
            EncLayer L;
            if (l > 0) {
                L.attn_norm = add_param(p + "attn_norm.weight", {d}, total);
                if (c.norm_bias) L.attn_norm_b = add_param(p + "attn_norm.bias", {d}, total);
            }
            L.wqkv = add_param(p + "attn.Wqkv.weight", {3 * d, d}, total);
            if (c.attention_bias) L.wqkv_b = add_param(p + "attn.Wqkv.bias", {3 * d}, total);
            L.wo = add_param(p + "attn.Wo.weight", {d, d}, total);
            if (c.attention_bias) L.wo_b = add_param(p + "attn.Wo.bias", {d}, total);
            L.mlp_norm = add_param(p + "mlp_norm.weight", {d}, total);
            if (c.norm_bias) L.mlp_norm_b = add_param(p + "mlp_norm.bias", {d}, total);
            L.wi = add_param(p + "mlp.Wi.weight", {2 * I, d}, total);
            if (c.mlp_bias) L.wi_b = add_param(p + "mlp.Wi.bias", {2 * I}, total);
            L.mlp_wo = add_param(p + "mlp.Wo.weight", {d, I}, total);
            if (c.mlp_bias) L.mlp_wo_b = add_param(p + "mlp.Wo.bias", {d}, total);
            L.kind = kinds[l];
            enc.push_back(L);
        }
        final_norm = add_param(e + "final_norm.weight", {d}, total);
        if (c.norm_bias) final_norm_b = add_param(e + "final_norm.bias", {d}, total);
        for (int l = 0; l < c.head_layers; ++l) {
            std::string p = "head.layers." + std::to_string(l) + ".";
            HeadLayer H;
            H.in_proj = add_param(p + "self_attn.in_proj_weight", {3 * d, d}, total);
            H.in_proj_b = add_param(p + "self_attn.in_proj_bias", {3 * d}, total);
            H.out_proj = add_param(p + "self_attn.out_proj.weight", {d, d}, total);
            H.out_proj_b = add_param(p + "self_attn.out_proj.bias", {d}, total);
            H.linear1 = add_param(p + "linear1.weight", {c.head_ff, d}, total);
            H.linear1_b = add_param(p + "linear1.bias", {c.head_ff}, total);
            H.linear2 = add_param(p + "linear2.weight", {d, c.head_ff}, total);
            H.linear2_b = add_param(p + "linear2.bias", {d}, total);
            H.norm1 = add_param(p + "norm1.weight", {d}, total);
            H.norm1_b = add_param(p + "norm1.bias", {d}, total);
            H.norm2 = add_param(p + "norm2.weight", {d}, total);
            H.norm2_b = add_param(p + "norm2.bias", {d}, total);
            head.push_back(H);
        }
        type_emb = add_param("type_emb.weight", {3, d}, total);
        sc_norm = add_param("scorer.0.weight", {d}, total);
        sc_norm_b = add_param("scorer.0.bias", {d}, total);
        sc1 = add_param("scorer.1.weight", {d, d}, total);
        sc1_b = add_param("scorer.1.bias", {d}, total);
        sc2 = add_param("scorer.3.weight", {1, d}, total);
        sc2_b = add_param("scorer.3.bias", {1}, total);
        act1 = add_param("act_head.0.weight", {256, d + 4}, total);
        act1_b = add_param("act_head.0.bias", {256}, total);
        act2 = add_param("act_head.2.weight", {c.n_act, 256}, total);
        act2_b = add_param("act_head.2.bias", {c.n_act}, total);
        int temp = add_param("temperature", {3}, total);
        params[temp].trainable = false;
        data.assign(total, R(0));
        grad.assign(total, R(0));
        global_rot = Rotary<R>(d / c.heads, c.theta_global);
        local_rot = Rotary<R>(d / c.heads, c.theta_local);
    }

    R* P(int i) { return data.data() + params[i].offset; }
    R* G(int i) {  // Parameter.GradientBuffer (Parameter.cs:177)
        params[i].touched = true;
        return grad.data() + params[i].offset;
    }
    R* Gt(int i) { return (i >= 0 && params[i].trainable) ? G(i) : nullptr; }
    const R* Pn(int i) { return i >= 0 ? P(i) : nullptr; }

    void release_frozen() override {
        for (auto& p : params)
            if (!p.trainable) std::fill(grad.begin() + p.offset, grad.begin() + p.offset + p.numel, R(0));
    }
    void set_param(int i, const float* d) override {
        for (size_t k = 0; k < params[i].numel; ++k) data[params[i].offset + k] = (R)d[k];
    }
    void get_param(int i, double* out) override {
        for (size_t k = 0; k < params[i].numel; ++k) out[k] = (double)data[params[i].offset + k];
    }
    void get_grad(int i, double* out) override {
        for (size_t k = 0; k < params[i].numel; ++k) out[k] = (double)grad[params[i].offset + k];
    }
    void zero_grad() override { std::fill(grad.begin(), grad.end(), R(0)); }

    AttentionShape<R> shape(const EncLayer& L) {
        int hd = cfg.hidden / cfg.heads;
        R scale = R(1) / std::sqrt((R)hd);
        return {hidden, cfg.heads, scale, L.kind == 1 ? cfg.local_attention / 2 : INT32_MAX,
                L.kind == 0 ? &global_rot : &local_rot, 0.0f, 0};
    }
    u64 salt(u64 seed, int layer, int site) { return mix(seed, (u64)(layer * 16 + site + 1)); }
    AttentionShape<R> head_shape(int index, float dropout, u64 seed) {
        R scale = R(1) / std::sqrt((R)(hidden / head_heads));
        return {hidden, head_heads, scale, INT32_MAX, nullptr, dropout, salt(seed, index, 0)};
    }

    struct EncTape {
        std::vector<R> normed, qkv, context, residual, mlp_normed, wide, activated;
    };

    // EncoderLayerForward (TrainableDecisionModel.cs:361-414).
    std::vector<R> encoder_layer_forward(const EncLayer& L, const std::vector<R>& x, const std::vector<Segment>& segs,
                                         EncTape* t) {
        int rows = (int)(x.size() / hidden), d = hidden, I = cfg.intermediate;
        R eps = (R)cfg.norm_eps;
        std::vector<R> normed;
        if (L.attn_norm < 0)
            normed = x;
        else {
            normed.resize(x.size());
            layernorm(x.data(), rows, d, P(L.attn_norm), Pn(L.attn_norm_b), eps, normed.data());
        }
        std::vector<R> qkv((size_t)rows * 3 * d);
        linear(normed.data(), rows, d, P(L.wqkv), 3 * d, Pn(L.wqkv_b), qkv.data());
        std::vector<R> context((size_t)rows * d);
        attention_forward(qkv.data(), segs, shape(L), context.data());
        std::vector<R> residual((size_t)rows * d);
        linear(context.data(), rows, d, P(L.wo), d, Pn(L.wo_b), residual.data());
        add(residual.data(), x.data(), (long)residual.size());
        std::vector<R> mlp_normed((size_t)rows * d);
        layernorm(residual.data(), rows, d, P(L.mlp_norm), Pn(L.mlp_norm_b), eps, mlp_normed.data());
        std::vector<R> wide((size_t)rows * 2 * I);
        linear(mlp_normed.data(), rows, d, P(L.wi), 2 * I, Pn(L.wi_b), wide.data());
        std::vector<R> activated((size_t)rows * I);
        geglu(wide.data(), rows, I, activated.data());
        std::vector<R> output((size_t)rows * d);
        linear(activated.data(), rows, I, P(L.mlp_wo), d, Pn(L.mlp_wo_b), output.data());
        add(output.data(), residual.data(), (long)output.size());
        if (t) {
            t->normed = std::move(normed);
            t->qkv = std::move(qkv);
            t->context = std::move(context);
            t->residual = std::move(residual);
            t->mlp_normed = std::move(mlp_normed);
            t->wide = std::move(wide);
            t->activated = std::move(activated);
        }
        return output;
    }

    struct HeadTape {
        std::vector<R> normed, qkv, context, residual, ff_normed, wide, dropped;
    };

    // HeadLayerForward (TrainableDecisionModel.cs:428-468).
    std::vector<R> head_layer_forward(const HeadLayer& H, int index, const std::vector<R>& x,
                                      const std::vector<Segment>& segs, bool training, u64 seed, HeadTape* t) {
        int rows = (int)(x.size() / hidden), d = hidden, ff = cfg.head_ff;
        float dr = training ? head_dropout : 0.0f;
        R eps = (R)1e-5f;
        std::vector<R> normed(x.size());
        layernorm(x.data(), rows, d, P(H.norm1), P(H.norm1_b), eps, normed.data());
        std::vector<R> qkv((size_t)rows * 3 * d);
        linear(normed.data(), rows, d, P(H.in_proj), 3 * d, P(H.in_proj_b), qkv.data());
        std::vector<R> context((size_t)rows * d);
        attention_forward(qkv.data(), segs, head_shape(index, dr, seed), context.data());
        std::vector<R> residual((size_t)rows * d);
        linear(context.data(), rows, d, P(H.out_proj), d, P(H.out_proj_b), residual.data());
        dropout(residual.data(), (long)residual.size(), dr, salt(seed, index, 1));
        add(residual.data(), x.data(), (long)residual.size());
        std::vector<R> ff_normed((size_t)rows * d);
        layernorm(residual.data(), rows, d, P(H.norm2), P(H.norm2_b), eps, ff_normed.data());
        std::vector<R> wide((size_t)rows * ff);
        linear(ff_normed.data(), rows, d, P(H.linear1), ff, P(H.linear1_b), wide.data());
        if (capture_head) {
            if ((int)captured_head.size() < cfg.head_layers) captured_head.resize(cfg.head_layers);
            captured_head[index].assign(wide.begin(), wide.end());
        }
        std::vector<R> dropped = wide;
        for (auto& v : dropped) v = std::max(v, R(0));
        dropout(dropped.data(), (long)dropped.size(), dr, salt(seed, index, 2));
        std::vector<R> output((size_t)rows * d);
        linear(dropped.data(), rows, ff, P(H.linear2), d, P(H.linear2_b), output.data());
        dropout(output.data(), (long)output.size(), dr, salt(seed, index, 3));
        add(output.data(), residual.data(), (long)output.size());
        if (t) {
            t->normed = std::move(normed);
            t->qkv = std::move(qkv);
            t->context = std::move(context);
            t->residual = std::move(residual);
            t->ff_normed = std::move(ff_normed);
            t->wide = std::move(wide);
            t->dropped = std::move(dropped);
        }
        return output;
    }

    // Forward (TrainableDecisionModel.cs:248-353).
    void forward(int n_items, const int* lengths, const int* tokens_in, const int* n_options, const int* markers,
                 const int* qtypes, bool training, bool keep_tape, u64 seed, double* logits) override {
        int d = hidden;
        std::vector<Segment> segs(n_items);
        int total = 0, nmark = 0, longest = 0;
        for (int i = 0; i < n_items; ++i) {
            segs[i] = {total, lengths[i]};
            total += lengths[i];
            nmark += n_options[i];
            longest = std::max(longest, lengths[i]);
        }
        global_rot.grow(longest);
        local_rot.grow(longest);
        std::vector<int> tokens(tokens_in, tokens_in + total);
        std::vector<int> marker_rows(nmark);
        for (int i = 0, m = 0; i < n_items; ++i)
            for (int o = 0; o < n_options[i]; ++o, ++m) marker_rows[m] = segs[i].start + std::max(0, markers[m]);

        std::vector<R> embedded((size_t)total * d);
        for (int t = 0; t < total; ++t) {
            int id = tokens[t];
            if ((unsigned)id >= (unsigned)cfg.vocab)
                throw std::out_of_range("token id " + std::to_string(id) + " is outside the vocabulary.");
            std::memcpy(embedded.data() + (size_t)t * d, P(tok_emb) + (size_t)id * d, sizeof(R) * d);
        }
        std::vector<R> states((size_t)total * d);
        layernorm(embedded.data(), total, d, P(emb_norm), Pn(emb_norm_b), (R)cfg.norm_eps, states.data());

        std::vector<std::vector<R>> enc_inputs(cfg.layers);
        for (int l = 0; l < cfg.layers; ++l) {
            if (keep_tape && l >= first_trainable) enc_inputs[l] = states;
            states = encoder_layer_forward(enc[l], states, segs, nullptr);
        }
        bool has_final = keep_tape && first_trainable < cfg.layers;
        std::vector<R> final_in;
        if (has_final) final_in = states;
        std::vector<R> normed((size_t)total * d);
        layernorm(states.data(), total, d, P(final_norm), Pn(final_norm_b), (R)cfg.norm_eps, normed.data());
        states = std::move(normed);
        for (int i = 0; i < n_items; ++i) {
            const R* tv = P(type_emb) + (size_t)qtypes[i] * d;
            for (int t = segs[i].start; t < segs[i].start + segs[i].length; ++t) add(states.data() + (size_t)t * d, tv, d);
        }
        std::vector<std::vector<R>> head_inputs(cfg.head_layers);
        for (int l = 0; l < cfg.head_layers; ++l) {
            if (keep_tape) head_inputs[l] = states;
            states = head_layer_forward(head[l], l, states, segs, training, seed, nullptr);
        }
        std::vector<R> sin_((size_t)nmark * d), snormed((size_t)nmark * d), pre((size_t)nmark * d);
        for (int r = 0; r < nmark; ++r)
            std::memcpy(sin_.data() + (size_t)r * d, states.data() + (size_t)marker_rows[r] * d, sizeof(R) * d);
        layernorm(sin_.data(), nmark, d, P(sc_norm), P(sc_norm_b), (R)1e-5f, snormed.data());
        linear(snormed.data(), nmark, d, P(sc1), d, P(sc1_b), pre.data());
        std::vector<R> act = pre;
        for (auto& v : act) v = gelu<R>(v);
        std::vector<R> scores(nmark);
        linear(act.data(), nmark, d, P(sc2), 1, P(sc2_b), scores.data());
        for (int r = 0; r < nmark; ++r) logits[r] = (double)scores[r];
        last_scores = scores;
        last_opts.assign(n_options, n_options + n_items);
        last_pooled.resize((size_t)n_items * d);
        for (int i = 0; i < n_items; ++i)
            std::memcpy(last_pooled.data() + (size_t)i * d, states.data() + (size_t)segs[i].start * d, sizeof(R) * d);

        tape = Tape{};
        if (keep_tape) {
            tape.valid = true;
            tape.training = training;
            tape.seed = seed;
            tape.segs = segs;
            tape.tokens = std::move(tokens);
            tape.marker_rows = std::move(marker_rows);
            tape.qtypes.assign(qtypes, qtypes + n_items);
            tape.n_options.assign(n_options, n_options + n_items);
            tape.enc_inputs = std::move(enc_inputs);
            tape.head_inputs = std::move(head_inputs);
            tape.has_final = has_final;
            tape.final_norm_input = std::move(final_in);
            tape.has_embedding = embeddings_trainable;
            if (embeddings_trainable) tape.embedding_input = std::move(embedded);
            tape.scorer_input = std::move(sin_);
            tape.scorer_normed = std::move(snormed);
            tape.scorer_pre = std::move(pre);
            tape.scorer_act = std::move(act);
        }
    }

    // DecisionModel.ReadOut (src/StructuredDecisions.Laya/Models/DecisionModel.cs:170-226) for every item of
    // the last forward: the untempered softmax of the option logits (SimdOps.Softmax), its entropy over
    // log(max(2, K)) with p clamped to ≥ 1e-9 inside the log, the top probability and its margin over the
    // second (strict comparisons, in option order), then the act head on [h[start], top1, top1 − top2,
    // entropy, k/255]: Linear → GELU → Linear (SimdOps.Linear: a Dot per output plus the bias) → softmax.
    // act_probs [n_items][n_act]; features [n_items][4]; pooled (may be null) [n_items][d] as doubles.
    void readout(float* act_probs, float* features, double* pooled) override {
        const int d = hidden, n_items = (int)last_opts.size();
        const int a1 = (int)params[act1_b].numel, na = (int)params[act2_b].numel;
        std::vector<R> x(d + 4), hid(a1), out(na);
        for (int i = 0, off = 0; i < n_items; off += last_opts[i], ++i) {
            const int K = last_opts[i];
            std::vector<R> p(last_scores.begin() + off, last_scores.begin() + off + K);
            softmax(p.data(), K);
            const R k = (R)std::max(2, K);
            R entropy = 0;
            for (R v : p) entropy -= v * std::log(std::max(v, (R)1e-9f));
            entropy /= std::log(k);
            R top1 = 0, top2 = 0;
            for (R v : p) {
                if (v > top1) {
                    top2 = top1;
                    top1 = v;
                } else if (v > top2) {
                    top2 = v;
                }
            }
            std::memcpy(x.data(), last_pooled.data() + (size_t)i * d, sizeof(R) * d);
            x[d] = top1;
            x[d + 1] = top1 - top2;
            x[d + 2] = entropy;
            x[d + 3] = k / (R)255;
            for (int o = 0; o < a1; ++o) hid[o] = gelu<R>(dot(x.data(), P(act1) + (size_t)o * (d + 4), d + 4) + P(act1_b)[o]);
            for (int o = 0; o < na; ++o) out[o] = dot(hid.data(), P(act2) + (size_t)o * a1, a1) + P(act2_b)[o];
            softmax(out.data(), na);
            for (int o = 0; o < na; ++o) act_probs[(size_t)i * na + o] = (float)out[o];
            for (int f = 0; f < 4; ++f) features[(size_t)i * 4 + f] = (float)x[d + f];
            if (pooled)
                for (int c = 0; c < d; ++c) pooled[(size_t)i * d + c] = (double)x[c];
        }
    }

    // Backward (TrainableDecisionModel.cs:479-549).
    void backward(const float* dlogits) override {
        if (!tape.valid) throw std::runtime_error("no tape: run forward with keep_tape first");
        int d = hidden, tokens = (int)tape.tokens.size(), nmark = (int)tape.marker_rows.size();
        std::vector<R> dscores(nmark);
        for (int r = 0; r < nmark; ++r) dscores[r] = (R)dlogits[r];
        std::vector<R> dact((size_t)nmark * d);
        linear_backward(tape.scorer_act.data(), dscores.data(), nmark, d, 1, P(sc2), dact.data(), Gt(sc2), Gt(sc2_b));
        for (size_t i = 0; i < dact.size(); ++i) dact[i] *= gelu_grad<R>(tape.scorer_pre[i]);
        std::vector<R> dnormed((size_t)nmark * d);
        linear_backward(tape.scorer_normed.data(), dact.data(), nmark, d, d, P(sc1), dnormed.data(), Gt(sc1),
                        Gt(sc1_b));
        std::vector<R> dmarkers((size_t)nmark * d, R(0));
        layernorm_backward(tape.scorer_input.data(), nmark, d, P(sc_norm), (R)1e-5f, dnormed.data(), dmarkers.data(),
                           Gt(sc_norm), Gt(sc_norm_b));
        std::vector<R> dstates((size_t)tokens * d, R(0));
        for (int r = 0; r < nmark; ++r)
            add(dstates.data() + (size_t)tape.marker_rows[r] * d, dmarkers.data() + (size_t)r * d, d);

        for (int l = cfg.head_layers - 1; l >= 0; --l)
            dstates = head_layer_backward(head[l], l, tape.head_inputs[l], dstates);

        if (params[type_emb].trainable) {
            R* g = G(type_emb);
            for (size_t i = 0; i < tape.segs.size(); ++i) {
                R* row = g + (size_t)tape.qtypes[i] * d;
                for (int t = tape.segs[i].start; t < tape.segs[i].start + tape.segs[i].length; ++t)
                    add(row, dstates.data() + (size_t)t * d, d);
            }
        }
        if (!tape.has_final) return;

        std::vector<R> denc((size_t)tokens * d, R(0));
        layernorm_backward(tape.final_norm_input.data(), tokens, d, P(final_norm), (R)cfg.norm_eps, dstates.data(),
                           denc.data(), Gt(final_norm), Gt(final_norm_b));
        dstates = std::move(denc);
        for (int l = cfg.layers - 1; l >= first_trainable; --l) {
            bool need = l > first_trainable || embeddings_trainable;
            dstates = encoder_layer_backward(enc[l], tape.enc_inputs[l], dstates, need);
        }
        if (embeddings_trainable && first_trainable == 0 && tape.has_embedding) {
            std::vector<R> demb((size_t)tokens * d, R(0));
            layernorm_backward(tape.embedding_input.data(), tokens, d, P(emb_norm), (R)cfg.norm_eps, dstates.data(),
                               demb.data(), Gt(emb_norm), Gt(emb_norm_b));
            R* g = G(tok_emb);
            for (int t = 0; t < tokens; ++t) add(g + (size_t)tape.tokens[t] * d, demb.data() + (size_t)t * d, d);
        }
    }

    // EncoderLayerBackward (TrainableDecisionModel.cs:551-603).
    std::vector<R> encoder_layer_backward(const EncLayer& L, const std::vector<R>& x, const std::vector<R>& dout,
                                          bool need_input) {
        int rows = (int)(x.size() / hidden), d = hidden, I = cfg.intermediate;
        R eps = (R)cfg.norm_eps;
        EncTape t;
        encoder_layer_forward(L, x, tape.segs, &t);
        std::vector<R> dres = dout;
        std::vector<R> dact((size_t)rows * I);
        linear_backward(t.activated.data(), dout.data(), rows, I, d, P(L.mlp_wo), dact.data(), Gt(L.mlp_wo),
                        Gt(L.mlp_wo_b));
        std::vector<R> dwide((size_t)rows * 2 * I);
        geglu_backward(t.wide.data(), dact.data(), rows, I, dwide.data());
        std::vector<R> dmlpn((size_t)rows * d);
        linear_backward(t.mlp_normed.data(), dwide.data(), rows, d, 2 * I, P(L.wi), dmlpn.data(), Gt(L.wi),
                        Gt(L.wi_b));
        layernorm_backward(t.residual.data(), rows, d, P(L.mlp_norm), eps, dmlpn.data(), dres.data(), Gt(L.mlp_norm),
                           Gt(L.mlp_norm_b));
        std::vector<R> dctx((size_t)rows * d);
        linear_backward(t.context.data(), dres.data(), rows, d, d, P(L.wo), dctx.data(), Gt(L.wo), Gt(L.wo_b));
        std::vector<R> dqkv((size_t)rows * 3 * d);
        attention_backward(t.qkv.data(), tape.segs, shape(L), dctx.data(), dqkv.data());
        if (!need_input) {
            linear_backward(t.normed.data(), dqkv.data(), rows, d, 3 * d, P(L.wqkv), (R*)nullptr, Gt(L.wqkv),
                            Gt(L.wqkv_b));
            return dres;
        }
        std::vector<R> dnormed((size_t)rows * d);
        linear_backward(t.normed.data(), dqkv.data(), rows, d, 3 * d, P(L.wqkv), dnormed.data(), Gt(L.wqkv),
                        Gt(L.wqkv_b));
        if (L.attn_norm < 0)
            add(dres.data(), dnormed.data(), (long)dres.size());
        else
            layernorm_backward(x.data(), rows, d, P(L.attn_norm), eps, dnormed.data(), dres.data(), Gt(L.attn_norm),
                               Gt(L.attn_norm_b));
        return dres;
    }

    // HeadLayerBackward (TrainableDecisionModel.cs:605-640).
    std::vector<R> head_layer_backward(const HeadLayer& H, int index, const std::vector<R>& x,
                                       const std::vector<R>& dout) {
        int rows = (int)(x.size() / hidden), d = hidden, ff = cfg.head_ff;
        float dr = tape.training ? head_dropout : 0.0f;
        u64 seed = tape.seed;
        HeadTape t;
        head_layer_forward(H, index, x, tape.segs, tape.training, seed, &t);
        std::vector<R> dres = dout, dy = dout;
        dropout(dy.data(), (long)dy.size(), dr, salt(seed, index, 3));
        std::vector<R> ddropped((size_t)rows * ff);
        linear_backward(t.dropped.data(), dy.data(), rows, ff, d, P(H.linear2), ddropped.data(), Gt(H.linear2),
                        Gt(H.linear2_b));
        dropout(ddropped.data(), (long)ddropped.size(), dr, salt(seed, index, 2));
        for (size_t i = 0; i < ddropped.size(); ++i)
            if (t.wide[i] <= R(0)) ddropped[i] = R(0);
        std::vector<R> dffn((size_t)rows * d);
        linear_backward(t.ff_normed.data(), ddropped.data(), rows, d, ff, P(H.linear1), dffn.data(), Gt(H.linear1),
                        Gt(H.linear1_b));
        layernorm_backward(t.residual.data(), rows, d, P(H.norm2), (R)1e-5f, dffn.data(), dres.data(), Gt(H.norm2),
                           Gt(H.norm2_b));
        std::vector<R> datt = dres;
        dropout(datt.data(), (long)datt.size(), dr, salt(seed, index, 1));
        std::vector<R> dctx((size_t)rows * d);
        linear_backward(t.context.data(), datt.data(), rows, d, d, P(H.out_proj), dctx.data(), Gt(H.out_proj),
                        Gt(H.out_proj_b));
        std::vector<R> dqkv((size_t)rows * 3 * d);
        attention_backward(t.qkv.data(), tape.segs, head_shape(index, dr, seed), dctx.data(), dqkv.data());
        std::vector<R> dnormed((size_t)rows * d);
        linear_backward(t.normed.data(), dqkv.data(), rows, d, 3 * d, P(H.in_proj), dnormed.data(), Gt(H.in_proj),
                        Gt(H.in_proj_b));
        layernorm_backward(x.data(), rows, d, P(H.norm1), (R)1e-5f, dnormed.data(), dres.data(), Gt(H.norm1),
                           Gt(H.norm1_b));
        return dres;
    }

    // Gradients.ClipByGlobalNorm (AdamW.cs:103-130).
    double clip(double max_norm) override {
        double sumsq = 0;
        for (auto& p : params) {
            if (!p.trainable || !p.touched) continue;
            const R* g = grad.data() + p.offset;
            double local = 0;
#pragma omp parallel for reduction(+ : local) schedule(static)
            for (long i = 0; i < (long)p.numel; ++i) local += (double)g[i] * g[i];
            sumsq += local;
        }
        double norm = std::sqrt(sumsq);
        double coefficient = max_norm / (norm + 1e-6);
        if (coefficient < 1.0) {
            R scale = (R)coefficient;
            for (auto& p : params) {
                if (!p.trainable || !p.touched) continue;
                R* g = grad.data() + p.offset;
                for (size_t i = 0; i < p.numel; ++i) g[i] *= scale;
            }
        }
        return norm;
    }

    // AdamW.Step (AdamW.cs:29-73) with the trainer's two groups (Trainer.cs:96-100): parameters whose
    // name contains "encoder." and the rest.
    void adamw(double lr_enc, double lr_head, double beta1, double beta2, double epsilon, double wd) override {
        if (m1.empty()) {
            m1.assign(data.size(), R(0));
            m2.assign(data.size(), R(0));
        }
        steps++;
        double c1 = 1.0 - std::pow(beta1, steps), c2 = 1.0 - std::pow(beta2, steps);
        R b1 = (R)beta1, b2 = (R)beta2;
        for (int group = 0; group < 2; ++group) {
            double lr = group == 0 ? lr_enc : lr_head;
            R decay = (R)(1.0 - lr * wd);
            R step_size = (R)(lr / c1);
            R sqrt_c2 = (R)std::sqrt(c2);
            R eps = (R)epsilon;
            for (auto& p : params) {
                if (!p.trainable) continue;
                bool is_enc = p.name.find("encoder.") != std::string::npos;
                if (is_enc != (group == 0)) continue;
                R* w = data.data() + p.offset;
                const R* g = grad.data() + p.offset;
                R* m = m1.data() + p.offset;
                R* v = m2.data() + p.offset;
#pragma omp parallel for schedule(static)
                for (long i = 0; i < (long)p.numel; ++i) {
                    R gi = p.touched ? g[i] : R(0);
                    w[i] *= decay;
                    m[i] = b1 * m[i] + (R(1) - b1) * gi;
                    v[i] = b2 * v[i] + (R(1) - b2) * gi * gi;
                    w[i] -= step_size * m[i] / (std::sqrt(v[i]) / sqrt_c2 + eps);
                }
            }
        }
    }
};

}  // namespace oracle

using namespace oracle;

// ======================================================================================== C ABI

extern "C" {

const char* orc_last_error(void) { return g_error.c_str(); }

void* orc_model_create(const orc_config* cfg, int use_double) {
    try {
        if (use_double) return static_cast<ModelBase*>(new Model<double>(*cfg));
        return static_cast<ModelBase*>(new Model<float>(*cfg));
    } catch (const std::exception& e) {
        g_error = e.what();
        return nullptr;
    }
}
void orc_model_destroy(void* m) { delete static_cast<ModelBase*>(m); }
static ModelBase* M_(void* m) { return static_cast<ModelBase*>(m); }
int orc_model_num_params(void* m) { return (int)M_(m)->params.size(); }
const char* orc_model_param_name(void* m, int i) { return M_(m)->params[i].name.c_str(); }
int orc_model_param_ndim(void* m, int i) { return (int)M_(m)->params[i].shape.size(); }
int orc_model_param_dim(void* m, int i, int d) { return M_(m)->params[i].shape[d]; }
long orc_model_param_numel(void* m, int i) { return (long)M_(m)->params[i].numel; }
int orc_model_param_trainable(void* m, int i) { return M_(m)->params[i].trainable ? 1 : 0; }
int orc_model_has_grad(void* m, int i) { return M_(m)->params[i].touched ? 1 : 0; }
int orc_model_set_param(void* m, int i, const float* d) {
    M_(m)->set_param(i, d);
    return 0;
}
int orc_model_get_param(void* m, int i, double* out) {
    M_(m)->get_param(i, out);
    return 0;
}
int orc_model_get_grad(void* m, int i, double* out) {
    M_(m)->get_grad(i, out);
    return 0;
}
void orc_model_set_trainable_encoder_layers(void* m, int n) { M_(m)->set_trainable_encoder_layers(n); }
void orc_model_set_head_dropout(void* m, float p) { M_(m)->head_dropout = p; }
int orc_model_forward(void* m, int n_items, const int* lengths, const int* tokens, const int* n_options,
                      const int* markers, const int* qtypes, int training, int keep_tape, uint64_t seed,
                      double* logits) {
    try {
        M_(m)->forward(n_items, lengths, tokens, n_options, markers, qtypes, training != 0, keep_tape != 0, seed,
                       logits);
        return 0;
    } catch (const std::exception& e) {
        g_error = e.what();
        return 1;
    }
}
int orc_model_readout(void* m, float* act_probs, float* features, double* pooled) {
    try {
        M_(m)->readout(act_probs, features, pooled);
        return 0;
    } catch (const std::exception& e) {
        g_error = e.what();
        return 1;
    }
}
int orc_model_backward(void* m, const float* dlogits) {
    try {
        M_(m)->backward(dlogits);
        return 0;
    } catch (const std::exception& e) {
        g_error = e.what();
        return 1;
    }
}
// ZeroGradients (TrainableDecisionModel.cs:237-240) clears the buffers but keeps them allocated.
void orc_model_zero_grad(void* m) { M_(m)->zero_grad(); }
double orc_model_clip(void* m, double max_norm) { return M_(m)->clip(max_norm); }
void orc_model_adamw(void* m, double lr_enc, double lr_head, double b1, double b2, double eps, double wd) {
    M_(m)->adamw(lr_enc, lr_head, b1, b2, eps, wd);
}
int orc_model_steps(void* m) { return M_(m)->steps; }
void orc_model_set_capture_head(void* m, int on) {
    M_(m)->capture_head = on != 0;
    if (!on) M_(m)->captured_head.clear();
}
long orc_model_head_preactivation(void* m, int layer, double* out) {
    auto& c = M_(m)->captured_head;
    if (layer < 0 || layer >= (int)c.size()) return -1;
    if (out) std::copy(c[layer].begin(), c[layer].end(), out);
    return (long)c[layer].size();
}

// The OpenMP thread count of the calls that follow (the CPU baseline's one-thread figure); returns the old one.
int orc_set_threads(int n) {
    const int old = omp_get_max_threads();
    if (n > 0) omp_set_num_threads(n);
    return old;
}
float orc_uniform(uint64_t seed, uint64_t index) { return uniform(seed, index); }
uint64_t orc_mix(uint64_t seed, uint64_t salt) { return mix(seed, salt); }
float orc_exp_f32(float x) { return exp_ref(x); }
float orc_erf_f32(float x) { return erf_ref(x); }

static std::vector<Segment> make_segs(int nseg, const int* start, const int* len) {
    std::vector<Segment> s(nseg);
    for (int i = 0; i < nseg; ++i) s[i] = {start[i], len[i]};
    return s;
}

#define ORC_DEFINE_OPS(R, S)                                                                                      \
    void orc_gemm_##S(int M, int N, int K, const R* A, long sam, long sak, const R* B, long sbk, long sbn, R* C,   \
                      long ldc, int accumulate) {                                                                 \
        gemm<R>(M, N, K, A, sam, sak, B, sbk, sbn, C, ldc, accumulate != 0);                                      \
    }                                                                                                             \
    void orc_linear_##S(const R* x, int rows, int in, const R* W, int out, const R* b, R* y) {                    \
        linear<R>(x, rows, in, W, out, b, y);                                                                     \
    }                                                                                                             \
    void orc_linear_backward_##S(const R* x, const R* dy, int rows, int in, int out, const R* W, R* dx, R* dW,    \
                                 R* db) {                                                                         \
        linear_backward<R>(x, dy, rows, in, out, W, dx, dW, db);                                                  \
    }                                                                                                             \
    void orc_layernorm_##S(const R* x, int rows, int n, const R* w, const R* b, float eps, R* y) {                \
        layernorm<R>(x, rows, n, w, b, (R)eps, y);                                                                \
    }                                                                                                             \
    void orc_layernorm_backward_##S(const R* x, int rows, int n, const R* w, float eps, const R* dy, R* dx,       \
                                    R* dgamma, R* dbeta) {                                                        \
        layernorm_backward<R>(x, rows, n, w, (R)eps, dy, dx, dgamma, dbeta);                                      \
    }                                                                                                             \
    void orc_gelu_##S(R* x, long n) {                                                                             \
        for (long i = 0; i < n; ++i) x[i] = gelu<R>(x[i]);                                                        \
    }                                                                                                             \
    void orc_gelu_backward_##S(const R* u, R* grad, long n) {                                                     \
        for (long i = 0; i < n; ++i) grad[i] *= gelu_grad<R>(u[i]);                                               \
    }                                                                                                             \
    void orc_geglu_##S(const R* wide, int rows, int inter, R* act) { geglu<R>(wide, rows, inter, act); }          \
    void orc_geglu_backward_##S(const R* wide, const R* dact, int rows, int inter, R* dwide) {                    \
        geglu_backward<R>(wide, dact, rows, inter, dwide);                                                        \
    }                                                                                                             \
    void orc_dropout_##S(R* values, long n, float p, uint64_t seed) { dropout<R>(values, n, p, seed); }          \
    void orc_rotary_apply_##S(double theta, int head_dim, R* vec, int position, int inverse) {                    \
        Rotary<R> r(head_dim, theta);                                                                             \
        r.grow(position + 1);                                                                                     \
        r.apply(vec, position, inverse != 0);                                                                     \
    }                                                                                                             \
    void orc_attention_forward_##S(const R* qkv, int nseg, const int* seg_start, const int* seg_len, int hidden,   \
                                   int heads, float scale, int half_window, double theta, float dr,               \
                                   uint64_t seed, R* context) {                                                   \
        auto segs = make_segs(nseg, seg_start, seg_len);                                                          \
        int longest = 1;                                                                                          \
        for (auto& s : segs) longest = std::max(longest, s.length);                                               \
        Rotary<R> rot;                                                                                            \
        if (theta > 0) {                                                                                          \
            rot = Rotary<R>(hidden / heads, theta);                                                               \
            rot.grow(longest);                                                                                    \
        }                                                                                                         \
        AttentionShape<R> sh{hidden, heads, (R)scale, half_window < 0 ? INT32_MAX : half_window,                  \
                             theta > 0 ? &rot : nullptr, dr, seed};                                               \
        attention_forward<R>(qkv, segs, sh, context);                                                             \
    }                                                                                                             \
    void orc_attention_backward_##S(const R* qkv, int nseg, const int* seg_start, const int* seg_len,             \
                                    int hidden, int heads, float scale, int half_window, double theta, float dr,  \
                                    uint64_t seed, const R* dcontext, R* dqkv) {                                  \
        auto segs = make_segs(nseg, seg_start, seg_len);                                                          \
        int longest = 1;                                                                                          \
        for (auto& s : segs) longest = std::max(longest, s.length);                                               \
        Rotary<R> rot;                                                                                            \
        if (theta > 0) {                                                                                          \
            rot = Rotary<R>(hidden / heads, theta);                                                               \
            rot.grow(longest);                                                                                    \
        }                                                                                                         \
        AttentionShape<R> sh{hidden, heads, (R)scale, half_window < 0 ? INT32_MAX : half_window,                  \
                             theta > 0 ? &rot : nullptr, dr, seed};                                               \
        attention_backward<R>(qkv, segs, sh, dcontext, dqkv);                                                     \
    }                                                                                                             \
    void orc_adamw_tensor_##S(R* p, const R* g, R* m, R* v, long n, double lr, double beta1, double beta2,        \
                              double epsilon, double wd, int step) {                                              \
        double c1 = 1.0 - std::pow(beta1, step), c2 = 1.0 - std::pow(beta2, step);                               \
        R b1 = (R)beta1, b2 = (R)beta2, decay = (R)(1.0 - lr * wd), step_size = (R)(lr / c1);                     \
        R sqrt_c2 = (R)std::sqrt(c2), eps = (R)epsilon;                                                           \
        for (long i = 0; i < n; ++i) {                                                                            \
            R gi = g ? g[i] : R(0);                                                                               \
            p[i] *= decay;                                                                                        \
            m[i] = b1 * m[i] + (R(1) - b1) * gi;                                                                  \
            v[i] = b2 * v[i] + (R(1) - b2) * gi * gi;                                                             \
            p[i] -= step_size * m[i] / (std::sqrt(v[i]) / sqrt_c2 + eps);                                         \
        }                                                                                                         \
    }

ORC_DEFINE_OPS(float, f32)
ORC_DEFINE_OPS(double, f64)

// Gradients.ClipByGlobalNorm (AdamW.cs:103-130) over a list of fp32 arrays.
double orc_clip_f32(int n, float** grads, const long* lens, double max_norm) {
    double sumsq = 0;
    for (int t = 0; t < n; ++t)
        for (long i = 0; i < lens[t]; ++i) sumsq += (double)grads[t][i] * grads[t][i];
    double norm = std::sqrt(sumsq);
    double coefficient = max_norm / (norm + 1e-6);
    if (coefficient < 1.0) {
        float scale = (float)coefficient;
        for (int t = 0; t < n; ++t)
            for (long i = 0; i < lens[t]; ++i) grads[t][i] *= scale;
    }
    return norm;
}

// RlcdObjective.Compute (RlcdObjective.cs:57-155) soft cross-entropy term (139-148), groups = 0.
double orc_cross_entropy(int n_items, const int* n_options, const float* logits, const float* targets,
                         double ce_weight, double scale, float* grad_out) {
    double ce = 0;
    int off = 0;
    for (int i = 0; i < n_items; ++i) {
        int k = n_options[i];
        std::vector<float> p(logits + off, logits + off + k);
        softmax<float>(p.data(), k);
        double mass = 0;
        for (int o = 0; o < k; ++o) mass += targets[off + o];
        for (int o = 0; o < k; ++o) {
            ce -= targets[off + o] * std::log(std::max((double)p[o], 1e-30)) / n_items;
            double g = ce_weight * (p[o] * mass - targets[off + o]) / n_items;
            grad_out[off + o] = (float)(g * scale);
        }
        off += k;
    }
    return ce;
}

// Calibration.ProperReward (src/StructuredDecisions.Laya/Runtime/Calibration.cs:76-119), all options unmasked.
double orc_proper_reward(int n, const float* reported, const float* target, int qtype, double sph, double rpsw) {
    double log_score = 0, dotv = 0, norm2 = 0;
    for (int i = 0; i < n; ++i) {
        double q = reported[i];
        double lq = std::max(std::log(std::max(q, 1e-12)), -9.21);
        log_score += target[i] * lq;
        dotv += target[i] * q;
        norm2 += q * q;
    }
    double reward = log_score + sph * (dotv / std::max(std::sqrt(norm2), 1e-9));
    if (qtype != 1) return reward;
    int k = std::max(n, 2);
    double cq = 0, ct = 0, rps = 0;
    for (int i = 0; i < n; ++i) {
        cq += reported[i];
        ct += target[i];
        double delta = cq - ct;
        rps += delta * delta;
    }
    return reward - rpsw * rps / (k - 1);
}

// RlcdObjective.Compute with supplied draws (RlcdObjective.cs:57-155).
int orc_rlcd(int n, const int* n_options, const int* qtypes, const float* logits, const float* targets, int groups,
             const double* draws, double sigma, double sph, double rpsw, double cew, double scale, float* grad_out,
             double* loss_out) {
    std::vector<int> off(n + 1, 0);
    for (int i = 0; i < n; ++i) off[i + 1] = off[i] + n_options[i];
    int per_group = off[n];
    std::vector<double> eps((size_t)groups * per_group), reward((size_t)groups * n);
    for (int g = 0; g < groups; ++g) {
        for (int i = 0; i < n; ++i) {
            int k = n_options[i];
            double* e = eps.data() + (size_t)g * per_group + off[i];
            double mean = 0;
            for (int o = 0; o < k; ++o) {
                e[o] = draws[(size_t)g * per_group + off[i] + o] * sigma;
                mean += e[o];
            }
            mean /= k;
            for (int o = 0; o < k; ++o) e[o] -= mean;
            std::vector<float> q(k);
            for (int o = 0; o < k; ++o) q[o] = (float)(logits[off[i] + o] + e[o]);
            softmax<float>(q.data(), k);
            reward[(size_t)g * n + i] = orc_proper_reward(k, q.data(), targets + off[i], qtypes[i], sph, rpsw);
        }
    }
    std::vector<double> adv((size_t)groups * n);
    double total = 0;
    for (int i = 0; i < n; ++i) {
        double mean = 0;
        for (int g = 0; g < groups; ++g) mean += reward[(size_t)g * n + i];
        mean /= groups;
        for (int g = 0; g < groups; ++g) {
            adv[(size_t)g * n + i] = reward[(size_t)g * n + i] - mean;
            total += adv[(size_t)g * n + i];
        }
    }
    int count = groups * n;
    double gmean = total / count, var = 0;
    for (int g = 0; g < groups; ++g)
        for (int i = 0; i < n; ++i) var += (adv[(size_t)g * n + i] - gmean) * (adv[(size_t)g * n + i] - gmean);
    double sd = count > 1 ? std::sqrt(var / (count - 1)) : 0.0;
    for (auto& a : adv) a /= sd + 1e-6;
    double policy = 0, ce = 0, rsum = 0, s2 = sigma * sigma;
    for (int i = 0; i < n; ++i) {
        int k = n_options[i];
        std::vector<double> grad(k, 0.0);
        for (int g = 0; g < groups; ++g) {
            double logp = 0;
            for (int o = 0; o < k; ++o) {
                double e = eps[(size_t)g * per_group + off[i] + o];
                logp -= e * e / (2 * s2);
                grad[o] -= adv[(size_t)g * n + i] * e / s2 / count;
            }
            policy -= adv[(size_t)g * n + i] * logp / count;
            rsum += reward[(size_t)g * n + i];
        }
        std::vector<float> p(logits + off[i], logits + off[i] + k);
        softmax<float>(p.data(), k);
        double mass = 0;
        for (int o = 0; o < k; ++o) mass += targets[off[i] + o];
        for (int o = 0; o < k; ++o) {
            ce -= targets[off[i] + o] * std::log(std::max((double)p[o], 1e-30)) / n;
            grad[o] += cew * (p[o] * mass - targets[off[i] + o]) / n;
        }
        for (int o = 0; o < k; ++o) grad_out[off[i] + o] = (float)(grad[o] * scale);
    }
    loss_out[0] = policy + cew * ce;
    loss_out[1] = policy;
    loss_out[2] = ce;
    loss_out[3] = rsum / count;
    return 0;
}

}  // extern "C"
