// Shared definitions of liblaya_hip: status handling, the context, and device helpers.
#pragma once

#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdint>
#include <cstdio>
#include <stdexcept>
#include <string>
#include <unordered_map>
#include <vector>

#include "../../include/laya_hip.h"

namespace laya {

// A failure carried up to the C-ABI boundary, where it becomes a status code plus laya_last_error().
struct Error : std::runtime_error {
    int code;
    Error(int c, const std::string& m) : std::runtime_error(m), code(c) {}
};

void set_last_error(const std::string& msg);

#define LAYA_HIP(expr)                                                                                   \
    do {                                                                                                 \
        hipError_t e_ = (expr);                                                                          \
        if (e_ != hipSuccess)                                                                            \
            throw ::laya::Error(LAYA_ERR_HIP, std::string(#expr) + ": " + hipGetErrorString(e_));        \
    } while (0)

#define LAYA_REQUIRE(cond, msg)                                                                          \
    do {                                                                                                 \
        if (!(cond)) throw ::laya::Error(LAYA_ERR_ARGUMENT, msg);                                        \
    } while (0)

// Runs a body at the C-ABI boundary and turns exceptions into status codes.
template <typename F> int guarded(F&& f) {
    try {
        f();
        return LAYA_OK;
    } catch (const Error& e) {
        set_last_error(e.what());
        return e.code;
    } catch (const std::bad_alloc&) {
        set_last_error("host allocation failed");
        return LAYA_ERR_MEMORY;
    } catch (const std::exception& e) {
        set_last_error(e.what());
        return LAYA_ERR_ARGUMENT;
    }
}

// After a launch: surfaces launch-configuration errors immediately.
inline void check_launch(const char* what) {
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) throw Error(LAYA_ERR_HIP, std::string(what) + ": " + hipGetErrorString(e));
}

// Workspace that grows on demand and is reused across calls on one context.
struct Workspace {
    void* ptr = nullptr;
    size_t bytes = 0;
};

// One profiled launch: events around it on the context's stream and its algorithmic work
// (flops for matrix-core kernels, compulsory HBM bytes for memory-bound ones).
struct LaunchRecord {
    const char* name;
    int start, stop;    // indices into the context's event pool: the scope's markers
    int kstart, kstop;  // the first and last kernel's own events (-1: time the scope by its markers)
    double flops, bytes;
};

}  // namespace laya

// One context: a device, one stream, an allocation ledger and reusable scratch.
struct laya_ctx {
    int device = 0;
    hipStream_t stream = nullptr;
    size_t cap = 0, in_use = 0;
    std::unordered_map<void*, size_t> allocations;
    laya::Workspace scratch[9];
    hipEvent_t timers[16][2] = {};
    int cu_count = 256;
    bool profiling = false;
    // Products with bf16 operands on the bf16 MFMA (fp32 accumulation) instead of fp32 MFMA, per product
    // class: bit 0 the forward products (NT), bit 1 the input gradients (NN), bit 2 the weight gradients (TN).
    int matmul_bf16 = 0;
    // fp32 products from three-piece bf16 splits (fp32-accurate, on the bf16 MFMA), same class bits.
    int matmul_split = LAYA_MATMUL_SPLIT_ALL;
    // Of those, the classes whose 256-wide kernels take two-piece fp16 products instead (fp32-accurate,
    // three fp16 MFMA products per fp32 one, operands scaled by powers of two), same class bits.
    int matmul_pair = LAYA_MATMUL_SPLIT_ALL;
    // Attention's split products as two-piece fp16 products too (the default).
    bool attention_pair = true;
    // max|operand| words of the two-piece products that no caller keeps: a ring of AMAX_RING word groups, each
    // measurement taking the next; each half is cleared (one launch) as the measurements enter it. A product
    // measures its operands one after another, so clearing only the half being entered keeps the group just
    // measured for the same product; stream order does the rest: every product that read a group of the
    // half being cleared was launched before the clear.
    unsigned* amax = nullptr;
    int amax_next = 0;
    std::vector<hipEvent_t> event_pool;
    std::vector<laya::LaunchRecord> launches;
    int next_event = 0;
    // Non-finite flag of the last laya_grad_norm on this context (device int, allocated on first use).
    int* nonfinite = nullptr;

    // Device scratch slot `slot` of at least `bytes`, reallocated (not preserved) when it grows.
    void* workspace(int slot, size_t bytes);
    void* alloc(size_t bytes);
    void release(void* p);
};

// A segment list (ModernBertEncoder.cs:30-33: Segment(Start, Length)) uploaded once: device tables the
// attention kernels read, and the host copy that sizes launches without reading the device back.
struct laya_segments {
    int nseg = 0, max_len = 0, rows = 0;
    std::vector<int> start, length, blocks;  // blocks: the attention block list (attention_block_list)
    int* d_start = nullptr;
    int* d_len = nullptr;
    int* d_blocks = nullptr;
};

// Rotary tables on the device (Ops.cs:446-504).
struct laya_rotary {
    int head_dim = 0, positions = 0;
    double theta = 0;
    float* cos_t = nullptr;
    float* sin_t = nullptr;
};

namespace laya {

// ------------------------------------------------------------------------------ device helpers

// Ops.Uniform (Ops.cs:227-234): SplitMix64 finaliser over seed + (index + 1)·φ, top 24 bits.
__host__ __device__ inline float uniform01(uint64_t seed, uint64_t index) {
    uint64_t z = seed + (index + 1ull) * 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    z ^= z >> 31;
    return (float)(z >> 40) * (1.0f / 16777216.0f);
}

// Ops.Mix (Ops.cs:236-241).
__host__ __device__ inline uint64_t mix64(uint64_t seed, uint64_t salt) {
    uint64_t z = seed ^ (salt * 0xD1B54A32D192ED03ull + 0x8CB92BA72F3D8DD7ull);
    z = (z ^ (z >> 33)) * 0xFF51AFD7ED558CCDull;
    return z ^ (z >> 33);
}

// Ops.DropoutIndex (Ops.cs:318).
__host__ __device__ inline uint64_t attn_dropout_index(int head, int row, int key) {
    return ((uint64_t)head << 42) | ((uint64_t)(uint32_t)row << 21) | (uint64_t)(uint32_t)key;
}

// erf as the reference's float GELU evaluates it (SimdOps.cs:329-356): the Numerical Recipes rational form of
// erfc (Press et al., Numerical Recipes in C, 2nd ed., §6.2, erfcc; fractional error below 1.2e-7),
// erf = sign(x)·(1 − t·exp(P(t) − x²)) with t = 1 / (1 + |x|/2), and ±1 beyond |x| = 6. Branch-free: one
// reciprocal, ten FMAs and one base-2 hardware exponential, each within an ulp or two, so the result stays
// within a few 1e-7 of erf (ROCm's erff evaluates two polynomial branches, both where a wave's lanes differ).
__device__ inline float erf_nr(float x) {
    const float ax = fabsf(x);
    const float t = __builtin_amdgcn_rcpf(fmaf(0.5f, ax, 1.0f));
    float p = 0.17087277f;
    p = fmaf(p, t, -0.82215223f);
    p = fmaf(p, t, 1.48851587f);
    p = fmaf(p, t, -1.13520398f);
    p = fmaf(p, t, 0.27886807f);
    p = fmaf(p, t, -0.18628806f);
    p = fmaf(p, t, 0.09678418f);
    p = fmaf(p, t, 0.37409196f);
    p = fmaf(p, t, 1.00002368f);
    p = fmaf(p, t, -1.26551223f);
    p = fmaf(-ax, ax, p);
    const float y = t * __builtin_amdgcn_exp2f(p * 1.44269504088896341f);
    return copysignf(ax > 6.0f ? 1.0f : 1.0f - y, x);
}

// Exact GELU x·Φ(x) and its derivative Φ(x) + x·φ(x) (SimdOps.cs:305-323, Ops.cs:194-218).
__device__ inline float gelu_f(float x) { return 0.5f * x * (1.0f + erf_nr(x * 0.70710678118654752f)); }
__device__ inline float gelu_grad_f(float x) {
    float cdf = 0.5f * (1.0f + erf_nr(x * 0.70710678118654752f));
    float pdf = 0.39894228040143268f * __expf(-0.5f * x * x);
    return cdf + x * pdf;
}

__device__ inline float wave_sum(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}

__device__ inline double wave_sum_d(double v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}

// The two-piece fp16 products take each operand's scale from max|x| over its finite elements, kept as
// fp32 bit patterns (non-negative patterns order as their values) in a group of AMAX_SPREAD device words
// that the kernels producing the operand fold their outputs into: amax_bits of each value, then one
// atomicMax per block into word blockIdx mod AMAX_SPREAD; the maximum is the largest word of the group.
// The words lie AMAX_STRIDE words (256 bytes) apart, so that the thousands of blocks of a launch meet on
// sixteen memory lines rather than one (on one line the atomics serialise: a LayerNorm forward measured
// 2.6 times slower); a group spans AMAX_GROUP words.
constexpr int AMAX_SPREAD = 16, AMAX_STRIDE = 64, AMAX_GROUP = AMAX_SPREAD * AMAX_STRIDE;
constexpr int AMAX_RING = 128;  // operand word groups the context measures into in turn (512 KB)
__device__ inline unsigned amax_bits(float x) {
    const unsigned a = __builtin_bit_cast(unsigned, x) & 0x7fffffffu;
    return a < 0x7f800000u ? a : 0u;  // infinities and NaNs left out
}
template <class V>
__device__ inline unsigned amax_bits4(V v) {
    return max(max(amax_bits(v[0]), amax_bits(v[1])), max(amax_bits(v[2]), amax_bits(v[3])));
}
// Every thread of the block calls it (it synchronises the block); out may be null.
__device__ inline void block_amax_fold(unsigned m, unsigned* out) {
    if (!out) return;
    __shared__ unsigned red[16];
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) m = max(m, (unsigned)__shfl_xor((int)m, o, 64));
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = m;
    __syncthreads();
    if (threadIdx.x == 0) {
        unsigned t = red[0];
        for (int w = 1; w < (int)((blockDim.x + 63) >> 6); ++w) t = max(t, red[w]);
        atomicMax(out + (blockIdx.x & (AMAX_SPREAD - 1)) * AMAX_STRIDE, t);
    }
}

// The largest word of a magnitude word group.
__device__ inline unsigned amax_group_max(const unsigned* w) {
    unsigned m = w[0];
#pragma unroll
    for (int i = 1; i < AMAX_SPREAD; ++i) m = max(m, w[i * AMAX_STRIDE]);
    return m;
}

inline unsigned blocks_for(size_t n, unsigned per_block, unsigned cap = 65535u * 16u) {
    size_t b = (n + per_block - 1) / per_block;
    if (b == 0) b = 1;
    return (unsigned)(b > cap ? cap : b);
}

// Brackets one kernel launch with events when the context is profiling (laya_profile_begin).
struct ProfileScope {
    laya_ctx* ctx;
    int start = -1;
    int kstart = -1, kstop = -1;  // events carried by the scope's own kernel dispatches (LAYA_LAUNCH)
    bool nested = false;          // a scope inside this one launched kernels: time by the markers
    const char* name;
    double flops, bytes;
    ProfileScope* outer;
    ProfileScope(laya_ctx* c, const char* n, double f, double b);
    ~ProfileScope();
};

// The events the next kernel dispatch carries while a live profile runs (both null otherwise): the innermost
// open scope's first dispatch records the scope's start, each dispatch its end.
void profile_kernel_events(hipEvent_t* start, hipEvent_t* stop);

// Every kernel launch goes through LAYA_LAUNCH: while a live profile runs, the innermost open profile scope's
// dispatches carry its start and stop events in the dispatch itself (hipExtLaunchKernelGGL), so a scope is
// timed by its kernels alone, without the dispatch gaps separate event packets would add.
#define LAYA_LAUNCH(kernel, grid, block, shmem, stream, ...)                                               \
    do {                                                                                                 \
        hipEvent_t laya_ls_ = nullptr, laya_le_ = nullptr;                                               \
        ::laya::profile_kernel_events(&laya_ls_, &laya_le_);                                             \
        if (laya_le_)                                                                                    \
            hipExtLaunchKernelGGL(kernel, grid, block, shmem, stream, laya_ls_, laya_le_, 0, __VA_ARGS__); \
        else                                                                                             \
            hipLaunchKernelGGL(kernel, grid, block, shmem, stream, __VA_ARGS__);                         \
    } while (0)

// Renames the innermost open profile scope of this thread: a launcher that picks a kernel variant
// below the scope's opener (the 256 × 256 tiles) tags the launch with that variant's name.
void profile_rename(const char* name);

// ------------------------------------------------------------------------ internal launchers

enum class GemmLayout {
    NT,  // C[M,N] = A[M,K] · B[N,K]ᵀ          (forward:  y  = x · Wᵀ)
    NN,  // C[M,N] = A[M,K] · B[K,N]           (backward: dx = dy · W)
    TN,  // C[M,N] = A[K,M]ᵀ · B[K,N]          (backward: dW = dyᵀ · x)
};

enum class GemmEpilogue {
    Store,       // C = acc (+ bias[n]) (+ R[m, n])
    Accumulate,  // C += acc, deterministically (split-K partials reduced in a fixed order)
};

// A16 / B16: optional bf16 copies of A / B (rounded to nearest even, same leading dimensions) that a bf16
// product reads instead of rounding A / B itself; the result is the same.
// amax_c / amax_dx (optional): the output's magnitude word group, folded in by the two-piece kernels'
// epilogues or measured after the product.
// A max|operand| word group (AMAX_GROUP words) kept by a caller for the two-piece fp16 products: `word`
// on the device, `*known` on the host says whether it holds the operand's current value. A product that
// needs it and finds it unknown measures the operand into it (and sets *known): an unknown group must
// hold zeros. A null word makes the product measure into the context's own words on every call.
struct AmaxRef {
    unsigned* word = nullptr;
    unsigned char* known = nullptr;
    // The operand's values are bf16 values held in fp32 (a bf16-weights product's weights): a two-piece
    // product takes them as one fp16 piece.
    bool bf16 = false;
};

void gemm(laya_ctx* ctx, GemmLayout layout, GemmEpilogue ep, int M, int N, int K, const float* A, long lda,
          const float* B, long ldb, float* C, long ldc, const float* bias = nullptr, const float* R = nullptr,
          long ldr = 0, const __bf16* A16 = nullptr, const __bf16* B16 = nullptr, AmaxRef amax_a = {},
          AmaxRef amax_b = {}, unsigned* amax_c = nullptr);

// GeGLU's input product and GeGLU (TrainableDecisionModel.cs:388-397: Ops.Linear, then SimdOps.Gelu of each
// row's first half times its second half): wide = x·Wᵀ + b for x [M, K], W [2·inter, K] (the first half's
// rows, then the second's), and act = gelu(first half)·(second half) [M, inter] with its bf16 copy act16 and
// magnitude amax_act (both optional): one launch where the product runs as two-piece products on 256-wide
// tiles (the GeGLU in its epilogue), else the product and geglu_fwd. Both forms take the same operand scales
// and the same GeGLU arithmetic; the products' K order (a tile's starting stage) may differ between them,
// which moves a value by fp32 rounding only.
void gemm_geglu(laya_ctx* ctx, int M, int inter, int K, const float* x, const float* W, const float* bias, float* wide,
                float* act, __bf16* act16, const __bf16* x16 = nullptr, const __bf16* W16 = nullptr,
                AmaxRef amax_x = {}, AmaxRef amax_W = {}, unsigned* amax_act = nullptr);

// y = x·Wᵀ + b for x [M, K], W [N, K] with RoPE applied in the epilogue to output columns [0, rope_cols)
// taken as heads of 64 (d and d + 32 rotated at position pos[row]; tables [positions][32]). The fused
// QKV projection: q and k leave the GEMM already rotated (Ops.cs:297-313).
void gemm_rope(laya_ctx* ctx, int M, int N, int K, const float* A, const float* B, float* C, const float* bias,
               const int* pos, const float* cos_t, const float* sin_t, int rope_cols, const __bf16* A16 = nullptr,
               const __bf16* B16 = nullptr, AmaxRef amax_a = {}, AmaxRef amax_b = {}, unsigned* amax_c = nullptr);

// The two products of Ops.LinearBackward in one launch: dx = dy·W (+ dx_residual) and dW += dyᵀ·x,
// for dy [rows, out], W [out, in], x [rows, in]; split-K partials of dW reduced in a fixed order.
void gemm_backward_pair(laya_ctx* ctx, int rows, int in, int out, const float* dy, const float* W, const float* x,
                        float* dx, const float* dx_residual, float* dW, const __bf16* W16 = nullptr,
                        const __bf16* x16 = nullptr, AmaxRef amax_dy = {}, AmaxRef amax_W = {},
                        AmaxRef amax_x = {}, unsigned* amax_dx = nullptr);
void gemm_backward_pair_body(laya_ctx* ctx, int rows, int in, int out, const float* dy, const float* W,
                             const float* x, float* dx, const float* dx_residual, float* dW, const __bf16* W16,
                             const __bf16* x16, AmaxRef amax_dy, AmaxRef amax_W, AmaxRef amax_x, unsigned* amax_dx,
                             bool* folded);

// max|x| over the finite elements of a rows x cols operand (row stride ld), folded into the word group
// at out by atomicMax as fp32 bit patterns (the two-piece products' operand scales).
void absmax_into(laya_ctx* ctx, const float* x, int rows, int cols, long ld, unsigned* out);
// Several tensors' magnitudes in one launch: block b folds max|arena[off[b] … off[b] + len[b])| (offsets 16-byte
// aligned, device arrays of `blocks` entries) into word group word[b] of `words`; `bytes` for the profile.
void absmax_multi(laya_ctx* ctx, const float* arena, const long* off, const int* len, const int* word, int blocks,
                  unsigned* words, double bytes);
// An operand's magnitude word group: the caller's r (measured now if not known yet), or the context's
// group `slot` (0 … 5), measured now.
const unsigned* operand_amax_ref(laya_ctx* ctx, AmaxRef r, int slot, const float* x, int rows, int cols, long ld);

// Σ over rows of a [rows, n] matrix added into out[n], deterministic (bias gradients); amax (optional): max|x|
// folded into that word group too, in the same pass where the sums take the float4 path.
void column_sum_add(laya_ctx* ctx, const float* x, int rows, int n, float* out, unsigned* amax = nullptr);
// The context's next operand word group, cleared (the ring operand_amax_ref measures into when the caller keeps
// no word), for a caller that folds an operand's magnitude into it itself.
unsigned* operand_ring_word(laya_ctx* ctx);

// y16 (optional): a bf16 copy of y (nearest even), for the bf16 products that read it; amax (optional):
// max|y| folded into a magnitude word group (absmax_into).
void layernorm_fwd(laya_ctx* ctx, const float* x, int rows, int n, const float* w, const float* b, float eps, float* y,
                   float* mean, float* rstd, const int* gather_ids = nullptr, const float* add_table = nullptr,
                   const int* add_index = nullptr, __bf16* y16 = nullptr, unsigned* amax = nullptr);
// Column sums whose reduction is deferred: `count` partial rows of `n` floats in `part`, added into `out`.
struct ColumnSumJob {
    const float* part;
    float* out;
    int count, n;
};
constexpr int MAX_COLUMN_JOBS = 96;  // 2.3 KB of kernel arguments
struct ColumnSumJobs {
    int n = 0;
    ColumnSumJob job[MAX_COLUMN_JOBS];
};

// LayerNorm backward whose dγ/dβ partials go to `ws` (2 · ln_bwd_partial_rows(rows) · n floats) and whose
// reduction is appended to `jobs` instead of launched (the caller runs column_reduce_batch later; a full
// list is flushed first). Falls back to the immediate reduction when a gradient is not 16-byte aligned.
int ln_bwd_partial_rows(int rows);
// amax (optional): max|dx| (after the addition) folded into a magnitude word group.
void layernorm_bwd_deferred(laya_ctx* ctx, const float* x, int rows, int n, const float* w, float eps,
                            const float* dy, float* dx, float* dgamma, float* dbeta, const float* mean,
                            const float* rstd, const int* gather_ids, float* ws, ColumnSumJobs& jobs,
                            unsigned* amax = nullptr);
void layernorm_bwd(laya_ctx* ctx, const float* x, int rows, int n, const float* w, float eps, const float* dy,
                   float* dx, float* dgamma, float* dbeta, const float* mean, const float* rstd,
                   const int* gather_ids = nullptr, unsigned* amax = nullptr);

// The allocation-free LayerNorm backward: partials in a static device array whose per-device address
// noalloc_scratch_init resolves once (laya_ctx_create calls it with the device current).
void noalloc_scratch_init(int device);
void layernorm_bwd_noalloc(laya_ctx* ctx, const float* x, int rows, int n, const float* w, float eps,
                           const float* dy, float* dx, float* dgamma, float* dbeta, const float* mean,
                           const float* rstd);

struct AttentionArgs {
    const float* qkv;
    const int* seg_start;
    const int* seg_len;
    int nseg, max_len, hidden, heads, head_dim, half_window;
    float scale, p_drop;
    uint64_t seed;
    const float* cos_table;  // [positions, head_dim/2] or null
    const float* sin_table;
    int positions;
    bool rotated = false;  // q and k in qkv already carry RoPE (the model's fused projection)
    int rows = -1;         // rows of qkv, needed to rotate a copy when !rotated
    double keys;           // Σ over queries of the keys each one attends to (for the profile's flop count)
    // Optional device list of the batch's row blocks of ATTENTION_BLOCK_ROWS rows, segment · 2¹⁶ + block as
    // an unsigned 32-bit pattern, every block of every segment once (attention_block_list): the kernels then
    // take one workgroup per entry and head, in list order. Null: a (max_len blocks, segments, heads) grid.
    const int* blocks = nullptr;
    int n_blocks = 0;
};

constexpr int ATTENTION_BLOCK_ROWS = 128;  // query or key rows per attention workgroup

// The block list of segments of lengths len[0 .. n): the segments in decreasing length (ties in index
// order), each segment's blocks in row order, so that a launch starts with its longest work. Segments
// beyond 65535 or of 2²³ rows or more have no encoding; attention refuses such batches anyway.
inline std::vector<int> attention_block_list(const std::vector<int>& len) {
    std::vector<int> order(len.size());
    for (size_t i = 0; i < order.size(); ++i) order[i] = (int)i;
    std::stable_sort(order.begin(), order.end(), [&](int a, int b) { return len[a] > len[b]; });
    std::vector<int> out;
    if (len.size() > 65536) return out;
    for (int s : order)
        for (int b = 0; b * ATTENTION_BLOCK_ROWS < len[s] && b < 65536; ++b)
            out.push_back((int)((unsigned)s << 16 | (unsigned)b));
    return out;
}

// Σ_q |window(q) ∩ segment| for one segment (Ops.cs:315-316).
inline double window_keys(int L, int hw) {
    if (hw < 0 || hw >= L) return (double)L * L;
    double s = 0;
    for (int q = 0; q < L; ++q) s += std::min(L - 1, q + hw) - std::max(0, q - hw) + 1;
    return s;
}
// context16 (optional): a bf16 copy of the context (nearest even), for the bf16 products that read it;
// amax (optional): max|context| folded into a magnitude word group.
void attention_fwd(laya_ctx* ctx, const AttentionArgs& a, float* context, float* lse, __bf16* context16 = nullptr,
                   unsigned* amax = nullptr, AmaxRef amax_qkv = {});

// RlcdObjective.Compute (RlcdObjective.cs:57-155) with supplied standard-normal draws [groups][Σ K], all
// operands on the device; grad [Σ K]; losses [4] = total, policy, cross-entropy, mean reward.
void rlcd_objective(laya_ctx* ctx, const float* logits, const float* targets, const int* offsets, const int* qtypes,
                    int n_items, int total_options, int max_options, int groups, const double* draws, double sigma,
                    double spherical, double rps, double ce_weight, double scale, float* grad, double* losses);
// DecisionModel.ReadOut (DecisionModel.cs:170-226) per item: probs [n_items][na], features [n_items][4]
// (may be null); states are the head output rows, opt_off [n_items + 1] the items' option offsets.
void decision_readout(laya_ctx* ctx, const float* scores, const int* opt_off, const int* seg_start, int n_items,
                      const float* states, int d, const float* w1, const float* b1, int a1, const float* w2,
                      const float* b2, int na, float* probs, float* features);
// rows: the number of rows of qkv / context / dcontext (the dO·O row constants span all of them); amax
// (optional): max|dqkv| folded into a magnitude word group.
void attention_bwd(laya_ctx* ctx, const AttentionArgs& a, int rows, const float* context, const float* lse,
                   const float* dcontext, float* dqkv, unsigned* amax = nullptr, AmaxRef amax_qkv = {},
                   AmaxRef amax_do = {});

}  // namespace laya
