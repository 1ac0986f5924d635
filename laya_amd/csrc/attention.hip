// Attention forward and backward on CDNA4 matrix cores (fp32, v_mfma_f32_32x32x2_f32).
//
// Restates Ops.AttentionForward / Ops.AttentionBackward (src/StructuredDecisions.Laya.Training/Ops.cs:263-438)
// flash-style: per (segment, head), q·k scores over the window [t − w, t + w] clipped to the segment
// (Ops.cs:315-316), softmax with an online max and sum, probability dropout regenerated from the counter
// RNG at head<<42 | row<<21 | key (Ops.cs:318, 355, 401), and the inverse RoPE on dq and dk
// (Ops.cs:421-427). The kernels read q and k with RoPE (segment-local positions, Gather, Ops.cs:297-313)
// already applied: the model's QKV projection applies it in its epilogue, and the op-level entry points
// rotate a copy first (`rope_rows_kernel`).
// The forward saves each row's base-2 log-sum-exp; the backward recomputes P from it instead of
// re-running the row softmax.
//
// Layout trick: the forward computes Sᵀ = K·Qᵀ, so in the 32×32 accumulator a lane owns one query
// (its column) and 16 keys (its rows). Those registers are exactly the B operand of Oᵀ = Vᵀ·Pᵀ, so
// P never leaves registers, and each query's running max / sum live in one lane pair.
// The backward runs two kernels, both without atomics (deterministic):
//   dkv: each wave owns 32 keys and sweeps the query tiles: S = Q·Kᵀ,
//        dVᵀ += dOᵀ·P, dP = dO·Vᵀ, dS, dKᵀ += Qᵀ·dS;
//   dq:  each wave owns 32 queries (Q, dO in registers) and sweeps the key tiles: Sᵀ, dPᵀ, dSᵀ,
//        dQᵀ += Kᵀ·dSᵀ.
#include "common.hpp"
#include "elementwise.hpp"
#include "split.hpp"

namespace laya {
namespace {

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int THREADS = 256;
constexpr int WAVE_ROWS = 32;   // queries (or keys) owned by one wave
constexpr int BLOCK_ROWS = ATTENTION_BLOCK_ROWS;  // 4 waves
constexpr int TILE = 64;        // rows of the streamed operand per LDS tile
constexpr float NEG_INF = -__builtin_huge_valf();
constexpr float LAZY_RESCALE = 8.0f;  // log2 headroom of the split-product forward's running max

struct Params {
    const float* qkv;
    const int* seg_start;
    const int* seg_len;
    int hidden, heads, half_window;  // half_window < 0: no window
    float scale, scale_log2, p_drop, keep;
    uint64_t seed;
    const float* cos_t;
    const float* sin_t;
    float* context;
    __bf16* context16;  // optional bf16 copy of the context (nearest even)
    float* lse;
    const float* dcontext;
    float* dots;  // Σ_d dO·O per (row, head)
    float* dqkv;
    unsigned* amax;  // optional magnitude word group of the output (context, or dqkv), folded per block
    // Two-piece products: the magnitude word groups of qkv and (backward) dO, from which q, k, v and dO
    // take their power-of-two scales.
    const unsigned* amax_qkv;
    const unsigned* amax_do;
    // Optional block list (AttentionArgs::blocks): the launch is one-dimensional, heads fastest.
    const int* blocks;
};

// A workgroup's segment, head and first row (query or key). With a block list, workgroup i takes entry
// i / heads (segment · 2¹⁶ + row block, unsigned), head i mod heads: every workgroup has rows, the longest segments'
// blocks are dispatched first, and the row blocks of one (segment, head) fall heads apart in dispatch order
// (on two XCDs for 12 heads rather than all eight). Without one, the grid is (row block, segment, head).
struct BlockCoord {
    int seg, head, row0;
};
__device__ __forceinline__ BlockCoord block_coord(const Params& p) {
    if (p.blocks) {
        const unsigned i = blockIdx.x / (unsigned)p.heads;
        const unsigned e = (unsigned)p.blocks[i];
        return {(int)(e >> 16), (int)(blockIdx.x - i * (unsigned)p.heads), (int)(e & 0xffffu) * BLOCK_ROWS};
    }
    return {(int)blockIdx.y, (int)blockIdx.z, (int)blockIdx.x * BLOCK_ROWS};
}

template <int D> struct Shape {
    static constexpr int G = D / 8;     // float4 groups per lane (the lane's half of d)
    static constexpr int ND = D / 32;   // 32-row d tiles of an accumulator
    static constexpr int FP = D / 4;    // flat accumulator offset of the rotary partner
    static constexpr int KS = D + 4;    // LDS stride of tiles read as b128 fragments
    static constexpr int VS = D + 8;    // LDS stride of tiles read as b32 columns
};

__device__ __forceinline__ f32x4 ld4(const float* p) { return *reinterpret_cast<const f32x4*>(p); }
__device__ __forceinline__ void st4(float* p, f32x4 v) { *reinterpret_cast<f32x4*>(p) = v; }

__device__ __forceinline__ f32x16 mfma(float a, float b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ bool in_window(int q, int key, int L, int hw) {
    return q < L && key >= 0 && key < L && (hw < 0 || (key - q <= hw && q - key <= hw));
}

// Wave-uniform: every (query, key) pair of the 32 queries from q0 and 32 keys from k0 lies inside the
// segment and the window, so the subtile needs no per-element test.
__device__ __forceinline__ bool subtile_inside(int q0, int k0, int L, int hw) {
    return q0 + 32 <= L && k0 >= 0 && k0 + 32 <= L && (hw < 0 || (k0 + 31 - q0 <= hw && q0 + 31 - k0 <= hw));
}

// The partners (keys of a query, or queries of a key) that row t may pair with under in_window, as
// one unsigned range test: partner i qualifies iff (unsigned)(i − lo) ≤ span. A row past the segment
// end gets a range nothing falls in. Lets a partial subtile mask its 16 elements with an add, a compare
// and a select each, instead of a branch per element.
struct WindowRange {
    int lo;
    unsigned span;
};
__device__ __forceinline__ WindowRange window_range(int t, int L, int hw) {
    if (t >= L) return {1 << 30, 0u};
    const int lo = hw < 0 ? 0 : max(0, t - hw);
    const int hi = hw < 0 ? L - 1 : min(L - 1, t + hw);
    return {lo, (unsigned)(hi - lo)};
}
__device__ __forceinline__ bool in_range(const WindowRange& w, int rel) { return (unsigned)rel <= w.span; }

// 2^x on the hardware exponential (v_exp_f32): arguments here are finite or −inf (→ 0), and results
// below the normal range only arise for probabilities far under the fp32 parity tolerance.
__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// A TILE-row slice of one head staged in registers between its global fetch and its LDS commit, so
// the next tile's loads are in flight while the current tile is computed. Rows outside [0, L) are zeros.
template <int D> struct PlainStage {
    static constexpr int U = TILE * (D / 4) / THREADS;
    f32x4 v[U];
};

template <int D>
__device__ __forceinline__ void fetch_plain(PlainStage<D>& st, const float* base, long stride, int L, int row0) {
#pragma unroll
    for (int i = 0; i < PlainStage<D>::U; ++i) {
        const int u = threadIdx.x + i * THREADS;
        const int r = u / (D / 4), j = (u % (D / 4)) * 4;
        const int t = row0 + r;
        st.v[i] = (t >= 0 && t < L) ? ld4(base + (long)t * stride + j) : f32x4{0, 0, 0, 0};
    }
}

template <int D, int S>
__device__ __forceinline__ void commit_plain(const PlainStage<D>& st, float* lds) {
#pragma unroll
    for (int i = 0; i < PlainStage<D>::U; ++i) {
        const int u = threadIdx.x + i * THREADS;
        st4(lds + (u / (D / 4)) * S + (u % (D / 4)) * 4, st.v[i]);
    }
}

// Loads the lane's own row (d = 8g + 4h + c) into registers (zeros when !valid).
template <int D>
__device__ __forceinline__ void load_lane_row(const float* src, bool valid, int h, f32x4 (&v)[Shape<D>::G]) {
#pragma unroll
    for (int g = 0; g < Shape<D>::G; ++g) v[g] = valid ? ld4(src + 8 * g + 4 * h) : f32x4{0, 0, 0, 0};
}

// Inverse RoPE on an accumulator whose column is the lane's row t and whose rows are d.
template <int D>
__device__ __forceinline__ void inverse_rope_acc(f32x16 (&acc)[Shape<D>::ND], const Params& p, int t, int h) {
    using S = Shape<D>;
#pragma unroll
    for (int f = 0; f < S::FP; ++f) {
        const int dt = f >> 4, r = f & 15;
        const int pf = f + S::FP, pdt = pf >> 4, pr = pf & 15;
        const int i = dt * 32 + 8 * (r >> 2) + 4 * h + (r & 3);
        const float c = p.cos_t[(long)t * (D / 2) + i], s = p.sin_t[(long)t * (D / 2) + i];
        const float a = acc[dt][r], b = acc[pdt][pr];
        acc[dt][r] = a * c + b * s;
        acc[pdt][pr] = b * c - a * s;
    }
}

// Writes an accumulator (rows d, column = the lane's row) into row `row` of dst at column `col`.
template <int D>
// Returns max|stored value| (amax_bits) for the output's magnitude word.
__device__ __forceinline__ unsigned store_acc(const f32x16 (&acc)[Shape<D>::ND], float* dst_row, int h, float scale) {
    unsigned m = 0;
#pragma unroll
    for (int dt = 0; dt < Shape<D>::ND; ++dt)
#pragma unroll
        for (int r4 = 0; r4 < 4; ++r4) {
            const f32x4 v = {acc[dt][4 * r4] * scale, acc[dt][4 * r4 + 1] * scale, acc[dt][4 * r4 + 2] * scale,
                             acc[dt][4 * r4 + 3] * scale};
            st4(dst_row + dt * 32 + 8 * r4 + 4 * h, v);
            m = max(m, amax_bits4(v));
        }
    return m;
}

// store_acc's values, also as bf16 (nearest even) into row `row` of a bf16 copy.
template <int D>
__device__ __forceinline__ void store_acc16(const f32x16 (&acc)[Shape<D>::ND], __bf16* dst_row, int h, float scale) {
    typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
#pragma unroll
    for (int dt = 0; dt < Shape<D>::ND; ++dt)
#pragma unroll
        for (int r4 = 0; r4 < 4; ++r4) {
            const f32x4 v = {acc[dt][4 * r4] * scale, acc[dt][4 * r4 + 1] * scale, acc[dt][4 * r4 + 2] * scale,
                             acc[dt][4 * r4 + 3] * scale};
            *reinterpret_cast<bf16x4*>(dst_row + dt * 32 + 8 * r4 + 4 * h) = __builtin_convertvector(v, bf16x4);
        }
}

// ------------------------------------------------------------------------------------ forward

template <int D>
__global__ __launch_bounds__(THREADS) void attn_fwd_kernel(Params p) {
    using S = Shape<D>;
    __shared__ __attribute__((aligned(16))) float Ks[TILE * S::KS];
    __shared__ __attribute__((aligned(16))) float Vs[TILE * S::VS];

    const BlockCoord bc = block_coord(p);
    const int seg = bc.seg, head = bc.head;
    const int start = p.seg_start[seg], L = p.seg_len[seg];
    const int qb0 = bc.row0;
    if (qb0 >= L) return;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, h = lane >> 5, lr = lane & 31;
    const int q0w = qb0 + wave * WAVE_ROWS;
    const int q = q0w + lr;
    const bool qvalid = q < L;
    const int hw = p.half_window;
    const long stride = 3L * p.hidden;
    const int qcol = head * D, kcol = p.hidden + head * D, vcol = 2 * p.hidden + head * D;

    f32x4 qv[S::G];
    load_lane_row<D>(p.qkv + (long)(start + (qvalid ? q : 0)) * stride + qcol, qvalid, h, qv);

    int kbeg = 0, kend = L;
    int wbeg = 0, wend = L;
    if (hw >= 0) {
        kbeg = max(0, qb0 - hw);
        kend = min(L, qb0 + BLOCK_ROWS + hw);
        wbeg = max(0, q0w - hw);
        wend = min(L, q0w + WAVE_ROWS + hw);
    }

    f32x16 o[S::ND];
#pragma unroll
    for (int dt = 0; dt < S::ND; ++dt) o[dt] = f32x16{};
    float m = -1e30f, l = 0.0f;

    const float* kbase = p.qkv + (long)start * stride + kcol;
    const float* vbase = p.qkv + (long)start * stride + vcol;
    PlainStage<D> kst, vst;
    fetch_plain<D>(kst, kbase, stride, L, kbeg);
    fetch_plain<D>(vst, vbase, stride, L, kbeg);
    for (int kt0 = kbeg; kt0 < kend; kt0 += TILE) {
        __syncthreads();
        commit_plain<D, S::KS>(kst, Ks);
        commit_plain<D, S::VS>(vst, Vs);
        __syncthreads();
        if (kt0 + TILE < kend) {  // block-uniform: the next tile's loads overlap this tile's products
            fetch_plain<D>(kst, kbase, stride, L, kt0 + TILE);
            fetch_plain<D>(vst, vbase, stride, L, kt0 + TILE);
        }
#pragma unroll
        for (int st = 0; st < TILE / 32; ++st) {
            const int kbs = kt0 + 32 * st;
            // Wave-uniform: outside this wave's window, or a wave whose rows all lie past the segment end.
            if (kbs >= wend || kbs + 32 <= wbeg || kbs >= kend || q0w >= L) continue;
            f32x16 s = f32x16{};
            const float* krow = Ks + (32 * st + lr) * S::KS + 4 * h;
#pragma unroll
            for (int g = 0; g < S::G; ++g) {
                const f32x4 kf = ld4(krow + 8 * g);
#pragma unroll
                for (int c = 0; c < 4; ++c) s = mfma(kf[c], qv[g][c], s);
            }
            float t[16];
            float mx = -1e30f;
            if (subtile_inside(q0w, kbs, L, hw)) {
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    t[r] = s[r] * p.scale_log2;
                    mx = fmaxf(mx, t[r]);
                }
            } else {
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const int key = kbs + 8 * (r >> 2) + 4 * h + (r & 3);
                    t[r] = in_window(q, key, L, hw) ? s[r] * p.scale_log2 : NEG_INF;
                    mx = fmaxf(mx, t[r]);
                }
            }
            mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
            const float mnew = fmaxf(m, mx);
            const float alpha = fast_exp2(m - mnew);
            float pr[16];
            float sum = 0.0f;
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                pr[r] = fast_exp2(t[r] - mnew);
                sum += pr[r];
            }
            l = l * alpha + sum;
            m = mnew;
#pragma unroll
            for (int dt = 0; dt < S::ND; ++dt) o[dt] *= alpha;
            if (p.p_drop > 0.0f) {
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const int key = kbs + 8 * (r >> 2) + 4 * h + (r & 3);
                    const float u = uniform01(p.seed, attn_dropout_index(head, start + q, key));
                    pr[r] = u < p.p_drop ? 0.0f : pr[r] * p.keep;
                }
            }
#pragma unroll
            for (int dt = 0; dt < S::ND; ++dt) {
                const float* vcolp = Vs + (32 * st + 4 * h) * S::VS + dt * 32 + lr;
#pragma unroll
                for (int r = 0; r < 16; ++r) o[dt] = mfma(vcolp[(8 * (r >> 2) + (r & 3)) * S::VS], pr[r], o[dt]);
            }
        }
    }

    const float lt = l + __shfl_xor(l, 32, 64);
    unsigned am = 0;
    if (qvalid) {
        const float inv = lt > 0.0f ? 1.0f / lt : 0.0f;
        am = store_acc<D>(o, p.context + (long)(start + q) * p.hidden + qcol, h, inv);
        if (h == 0) p.lse[(long)(start + q) * p.heads + head] = lt > 0.0f ? m + log2f(lt) : __builtin_huge_valf();
    }
    block_amax_fold(am, p.amax);
}

// ------------------------------------------------------------------------------------ split products
//
// The products on the bf16 matrix cores (v_mfma_f32_32x32x16_bf16) from exact three-piece splits of every
// fp32 operand (split.hpp): six piece products per fp32 product with fp32 accumulation, so the results
// carry fp32 rounding only. A tile streamed through LDS is split once, as it is committed, into three bf16
// planes; a wave's own rows are split once into registers; P (and dS) are split in registers.
// In a 32×32×16 product a lane supplies 8 consecutive k of its row or column. The scores' accumulator
// gives a lane the keys 8(r/4) + 4h + r%4 of its column, so a product over keys takes, per 16 keys, the
// key order {4h … 4h+3, 8+4h … 8+4h+3} for both operands: P stays in the registers it was computed in and
// the other operand is read from its [key][d] plane as two runs of 4 keys by transposing LDS reads.

__device__ __forceinline__ f32x16 mfma16(bf16x8 a, bf16x8 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

// c += a·b over one 16-k step from the pieces, the smallest products first.
__device__ __forceinline__ f32x16 mma6(const bf16x8 (&a)[3], const bf16x8 (&b)[3], f32x16 c) {
    c = mfma16(a[2], b[0], c);
    c = mfma16(a[0], b[2], c);
    c = mfma16(a[1], b[1], c);
    c = mfma16(a[1], b[0], c);
    c = mfma16(a[0], b[1], c);
    return mfma16(a[0], b[0], c);
}

template <class V4>
__device__ __forceinline__ auto cat8(V4 lo, V4 hi) {
    return __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
}

// The pieces an operand is split into: NP = 3, exact three-piece bf16 splits and six products per block
// (split.hpp); NP = 2, two fp16 pieces of the operand scaled by a power of two (split2h_4) and three
// products per block, the smallest first. Both feed the same 32×32×16 fragment layouts.
template <int NP> struct Pieces;
template <> struct Pieces<3> {
    typedef bf16x8 V8;
    typedef bf16x4 V4;
    static __device__ __forceinline__ void split4(f32x4 x, float, V4 (&o)[3]) { split3_4(x, o[0], o[1], o[2]); }
    static __device__ __forceinline__ void split4u(f32x4 x, float, V4 (&o)[3]) { split3_4(x, o[0], o[1], o[2]); }
    static __device__ __forceinline__ f32x16 mma(const V8 (&a)[3], const V8 (&b)[3], f32x16 c) { return mma6(a, b, c); }
};
template <> struct Pieces<2> {
    typedef f16x8 V8;
    typedef f16x4 V4;
    static __device__ __forceinline__ void split4(f32x4 x, float sc, V4 (&o)[2]) { split2h_4(x, sc, o[0], o[1]); }
    static __device__ __forceinline__ void split4u(f32x4 x, float one, V4 (&o)[2]) { split2h_4u(x, one, o[0], o[1]); }
    static __device__ __forceinline__ f32x16 mma(const V8 (&a)[2], const V8 (&b)[2], f32x16 c) {
        c = __builtin_amdgcn_mfma_f32_32x32x16_f16(a[1], b[0], c, 0, 0, 0);
        c = __builtin_amdgcn_mfma_f32_32x32x16_f16(a[0], b[1], c, 0, 0, 0);
        return __builtin_amdgcn_mfma_f32_32x32x16_f16(a[0], b[0], c, 0, 0, 0);
    }
};

// The operands computed in registers (P, dS) take a per-lane power-of-two scale for the two-piece
// products: a lane's 16 values, with its partner lane's (lanes l and l + 32 feed the same output column),
// set the exponent 14 − ⌊log₂ max⌋; it only decreases over the tiles, and when it does the column's
// accumulators are rescaled by the same exact power of two, so they always carry one factor 2^e.
// The operand is c·v for a positive constant c that the split applies (c·max|v| rounds to the largest
// |c·v|, rounding being monotone). Returns the new exponent (e0 = 126 before the first tile).
// (A NaN is passed over by the maximum; an infinity gives a tiny scale that keeps it infinite.)
template <int N>
__device__ __forceinline__ int lane_scale_update(const float (&v)[16], int e, f32x16 (&acc)[N], float c = 1.0f) {
    float m = 0.0f;
#pragma unroll
    for (int r = 0; r < 16; ++r) m = fmaxf(m, fabsf(v[r]));
    m = fmaxf(m, __shfl_xor(m, 32, 64)) * c;
    const int et = pair_scale_exp(__builtin_bit_cast(unsigned, m));
    if (et < e) {
        const float f = ldexpf(1.0f, et - e);
#pragma unroll
        for (int i = 0; i < N; ++i) acc[i] *= f;
        e = et;
    }
    return e;
}

// The pieces of 8 values (two float4), scaled by sc (two-piece products).
template <int NP>
__device__ __forceinline__ void split8(f32x4 lo, f32x4 hi, typename Pieces<NP>::V8 (&out)[NP], float sc = 1.0f) {
    typename Pieces<NP>::V4 a[NP], b[NP];
    Pieces<NP>::split4(lo, sc, a);
    Pieces<NP>::split4(hi, sc, b);
#pragma unroll
    for (int pl = 0; pl < NP; ++pl) out[pl] = cat8(a[pl], b[pl]);
}

// split8 at unit scale (split2h_4u for two-piece products).
template <int NP>
__device__ __forceinline__ void split8u(f32x4 lo, f32x4 hi, typename Pieces<NP>::V8 (&out)[NP], float one) {
    typename Pieces<NP>::V4 a[NP], b[NP];
    Pieces<NP>::split4u(lo, one, a);
    Pieces<NP>::split4u(hi, one, b);
#pragma unroll
    for (int pl = 0; pl < NP; ++pl) out[pl] = cat8(a[pl], b[pl]);
}

// An R × 64 slice of one head (R = 32, 64 or 128 rows) in registers between its global fetch and its LDS
// commit: thread t holds rows (R/16)·(t/16) + i (i < R/16) at d = 4·(t%16) … +3.
template <int R>
struct RowStage {
    static constexpr int N = R / 16;
    f32x4 v[N];
};

// Rows row0 … row0 + R − 1 (row0 ≥ 0, block-uniform) of a segment of L rows. The loads go through a buffer
// resource that spans rows row0 … L − 1 only: a row at or past L lies beyond its record count and reads
// as zeros, so no lane computes a 64-bit address or takes a branch (the host keeps L · stride · 4 < 2³¹).
template <int R>
__device__ __forceinline__ void fetch_rows(RowStage<R>& st, const float* base, long stride, int L, int row0) {
    constexpr int N = RowStage<R>::N;
    const int q = threadIdx.x >> 4, j = (threadIdx.x & 15) * 4;
    const int bytes = row0 < L ? (L - row0) * (int)stride * 4 : 0;
    const __amdgpu_buffer_rsrc_t rs =
        __builtin_amdgcn_make_buffer_rsrc((void*)(base + (long)row0 * stride), (short)0, bytes, 0x00020000);
#pragma unroll
    for (int i = 0; i < N; ++i) {
        const int off = ((N * q + i) * (int)stride + j) * 4;
        st.v[i] = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(rs, off, 0, 0));
    }
}

// The lane's own row (d = 16s + 8h … +7 for s < 4), loaded, and split later: a kernel issues its first tile's
// loads in between, so the two loads' latencies overlap. src is always a row of the segment (a lane past the
// segment's end reads row 0): such a lane's column of every product is its own and is never stored, so its
// values need no zeroing, and the loads need no predicate.
struct LaneRow {
    f32x4 v[8];
    __device__ __forceinline__ void load(const float* src, int h) {
#pragma unroll
        for (int s = 0; s < 4; ++s) {
            v[2 * s] = ld4(src + 16 * s + 8 * h);
            v[2 * s + 1] = ld4(src + 16 * s + 8 * h + 4);
        }
    }
    template <int NP>
    __device__ __forceinline__ void split(typename Pieces<NP>::V8 (&out)[4][NP], float sc = 1.0f) const {
#pragma unroll
        for (int s = 0; s < 4; ++s) split8<NP>(v[2 * s], v[2 * s + 1], out[s], sc);
    }
};

// The lane's own row (d = 16s + 8h … +7 for s < 4), split.
template <int NP>
__device__ __forceinline__ void split_lane_row(const float* src, bool valid, int h,
                                               typename Pieces<NP>::V8 (&out)[4][NP], float sc = 1.0f) {
#pragma unroll
    for (int s = 0; s < 4; ++s) {
        const f32x4 lo = valid ? ld4(src + 16 * s + 8 * h) : f32x4{0, 0, 0, 0};
        const f32x4 hi = valid ? ld4(src + 16 * s + 8 * h + 4) : f32x4{0, 0, 0, 0};
        split8<NP>(lo, hi, out[s], sc);
    }
}

// 16 values of a lane's accumulator column as the pieces of two 16-row k-steps (in the key order above).
template <int NP>
__device__ __forceinline__ void split_col16(const float (&v)[16], int u, typename Pieces<NP>::V8 (&out)[NP],
                                            float sc = 1.0f) {
    split8<NP>(f32x4{v[8 * u], v[8 * u + 1], v[8 * u + 2], v[8 * u + 3]},
               f32x4{v[8 * u + 4], v[8 * u + 5], v[8 * u + 6], v[8 * u + 7]}, out, sc);
}

template <int NP>
__device__ __forceinline__ void split_col16u(const float (&v)[16], int u, typename Pieces<NP>::V8 (&out)[NP], float one) {
    split8u<NP>(f32x4{v[8 * u], v[8 * u + 1], v[8 * u + 2], v[8 * u + 3]},
                f32x4{v[8 * u + 4], v[8 * u + 5], v[8 * u + 6], v[8 * u + 7]}, out, one);
}

// One LDS layout for every staged tile.
//
// Planes of 64 bf16 per row (128 bytes) with the 16-byte chunks of row r XOR-swizzled by
// g(r) = 4·(r/2 mod 2) + (r/4 mod 4). The LDS serves a b128 read 16 lanes (256 bytes, 64 banks) at a time:
// 16 consecutive rows at one chunk then take 16 distinct (row parity, chunk) bank groups. A transposing
// read is served 32 lanes at a time, four consecutive rows at four adjacent chunks: rows r and r + 2 differ
// in bit 2 of g, so their aligned groups of four chunks do not meet. A product over rows (queries)
// reads its operand from the [row][d] plane with ds_read_b64_tr_b16: in each 16-lane group, lane j names
// the 4-element chunk (row r0 + j/4, columns c0 + 4(j mod 4)) and lane i receives element i mod 4 of the
// chunks named by lanes i/4, 4 + i/4, 8 + i/4, 12 + i/4 — i.e. 4 consecutive rows of its column.
__device__ __forceinline__ int swz(int row, int col) {
    return row * 64 + ((((col >> 3) ^ ((((row >> 1) & 1) << 2) | ((row >> 2) & 3)))) << 3) + (col & 7);
}

__device__ __forceinline__ bf16x4 ds_read_tr(const __bf16* p) {
    typedef short i16x4 __attribute__((ext_vector_type(4)));
    typedef __attribute__((address_space(3))) i16x4* lds_i16x4;
    return __builtin_bit_cast(bf16x4, __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4)(p)));
}

// NP swizzled [row][d] planes of R rows (plane stride R·64, 16-bit pieces) from a staged tile.
template <int R, int NP = 3>
__device__ __forceinline__ void commit_swz(const RowStage<R>& st, __bf16* planes, float sc = 1.0f) {
    typedef typename Pieces<NP>::V4 V4;
    constexpr int N = RowStage<R>::N;
    const int q = threadIdx.x >> 4, j = (threadIdx.x & 15) * 4;
#pragma unroll
    for (int i = 0; i < N; ++i) {
        V4 h[NP];
        Pieces<NP>::split4(st.v[i], sc, h);
        const int o = swz(N * q + i, j);
#pragma unroll
        for (int pl = 0; pl < NP; ++pl) *reinterpret_cast<V4*>(planes + pl * R * 64 + o) = h[pl];
    }
}

// Row fragments (8 consecutive d of row `row` at k-step s) of NP swizzled planes of R rows.
template <int R, int NP = 3>
__device__ __forceinline__ void swz_row_frag(const __bf16* planes, int row, int s, int h,
                                             typename Pieces<NP>::V8 (&f)[NP]) {
    typedef typename Pieces<NP>::V8 V8;
    const int o = swz(row, 16 * s + 8 * h);
#pragma unroll
    for (int pl = 0; pl < NP; ++pl) f[pl] = *reinterpret_cast<const V8*>(planes + pl * R * 64 + o);
}

// The A fragments of d-rows 32·dt + lane mod 32 over the 16 rows from r0, in the key order of the score
// accumulators (rows r0 + 4h … +3, then r0 + 8 + 4h … +3), from NP swizzled planes of R rows.
template <int R, int NP = 3>
__device__ __forceinline__ void swz_col_frag(const __bf16* planes, int r0, int dt, int lane,
                                             typename Pieces<NP>::V8 (&f)[NP]) {
    typedef typename Pieces<NP>::V4 V4;
    const int G = lane >> 4, j = lane & 15;
    const int row = r0 + 4 * (G >> 1) + (j >> 2), col = 32 * dt + 16 * (G & 1) + 4 * (j & 3);
    const int o0 = swz(row, col), o1 = swz(row + 8, col);
#pragma unroll
    for (int pl = 0; pl < NP; ++pl)
        f[pl] = cat8(__builtin_bit_cast(V4, ds_read_tr(planes + pl * R * 64 + o0)),
                     __builtin_bit_cast(V4, ds_read_tr(planes + pl * R * 64 + o1)));
}

// NP = 3: three-piece bf16 split products; NP = 2: two-piece fp16 products of scaled operands.
template <int D, bool DROP, int NP = 3>
__global__ __launch_bounds__(THREADS, 2) void attn_fwd_x6_kernel(Params p) {
    static_assert(D == 64, "split-product attention is written for head_dim 64");
    __shared__ __attribute__((aligned(16))) __bf16 Ks[NP * TILE * 64];  // K tile, swizzled [key][d]
    __shared__ __attribute__((aligned(16))) __bf16 Vs[NP * TILE * 64];  // V tile, swizzled [key][d]

    const BlockCoord bc = block_coord(p);
    const int seg = bc.seg, head = bc.head;
    const int start = p.seg_start[seg], L = p.seg_len[seg];
    const int qb0 = bc.row0;
    if (qb0 >= L) return;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, h = lane >> 5, lr = lane & 31;
    const int q0w = qb0 + wave * WAVE_ROWS;
    const int q = q0w + lr;
    const bool qvalid = q < L;
    const int hw = p.half_window;
    const long stride = 3L * p.hidden;
    const int qcol = head * D, kcol = p.hidden + head * D, vcol = 2 * p.hidden + head * D;

    typedef typename Pieces<NP>::V8 V8;
    // Two-piece products: q, k and v scaled by 2^eq (from the qkv magnitude), P by the lane's running 2^ep:
    // a subtile's largest probability is 2^(mx − m) (times keep), so ep = 14 − ⌊mx − m⌋ − ⌈log₂ keep⌉ goes
    // into the exponential's argument, and the row sum l is kept in the same units as the output's
    // accumulator (both rescaled when ep drops), so the final o/l needs only q's factor out.
    int eq = 0, ep = 126, ek = 0;
    if constexpr (NP == 2) {
        eq = pair_scale_exp(amax_group_max(p.amax_qkv));
        if (DROP) {
            const unsigned kb = __builtin_bit_cast(unsigned, p.keep);
            ek = (int)(kb >> 23) - 127 + ((kb & 0x7fffffu) != 0u);
        }
    }
    const float sq = exp2_int(eq);
    const float scale_log2 = NP == 2 ? ldexpf(p.scale_log2, -2 * eq) : p.scale_log2;
    float one = 1.0f;
    asm volatile("" : "+s"(one));  // 1.0 that the compiler cannot fold (split2h_4u)
    LaneRow qrow;
    qrow.load(p.qkv + (long)(start + (qvalid ? q : 0)) * stride + qcol, h);

    int kbeg = 0, kend = L;
    int wbeg = 0, wend = L;
    if (hw >= 0) {
        kbeg = max(0, qb0 - hw);
        kend = min(L, qb0 + BLOCK_ROWS + hw);
        wbeg = max(0, q0w - hw);
        wend = min(L, q0w + WAVE_ROWS + hw);
    }

    const WindowRange win = window_range(q, L, hw);
    f32x16 o[2];
    o[0] = f32x16{};
    o[1] = f32x16{};
    float m = -1e30f, l = 0.0f;

    const float* kbase = p.qkv + (long)start * stride + kcol;
    const float* vbase = p.qkv + (long)start * stride + vcol;
    RowStage<TILE> kst, vst;
    fetch_rows<TILE>(kst, kbase, stride, L, kbeg);
    fetch_rows<TILE>(vst, vbase, stride, L, kbeg);
    __builtin_amdgcn_sched_barrier(0);  // the tile's loads are issued before q's split waits for q
    V8 qh[4][NP];
    qrow.split<NP>(qh, sq);
    for (int kt0 = kbeg; kt0 < kend; kt0 += TILE) {
        __syncthreads();
        commit_swz<TILE, NP>(kst, Ks, sq);
        commit_swz<TILE, NP>(vst, Vs, sq);
        __syncthreads();
        if (kt0 + TILE < kend) {  // block-uniform: the next tile's loads overlap this tile's products
            fetch_rows<TILE>(kst, kbase, stride, L, kt0 + TILE);
            fetch_rows<TILE>(vst, vbase, stride, L, kt0 + TILE);
        }
#pragma unroll
        for (int st = 0; st < TILE / 32; ++st) {
            const int kbs = kt0 + 32 * st;
            // Wave-uniform: outside this wave's window, or a wave whose rows all lie past the segment end.
            if (kbs >= wend || kbs + 32 <= wbeg || kbs >= kend || q0w >= L) continue;
            // Sᵀ = K·Qᵀ: lane column = its query, rows = 16 keys.
            f32x16 s = f32x16{};
#pragma unroll
            for (int ks = 0; ks < 4; ++ks) {
                V8 kf[NP];
                swz_row_frag<TILE, NP>(Ks, 32 * st + lr, ks, h, kf);
                s = Pieces<NP>::mma(kf, qh[ks], s);
            }
            // The maximum is taken over the raw scores and scaled once (the scale is positive and rounding
            // monotone, so it is the largest scaled score); each exponent is one fused s·scale − mm.
            float mx = -1e30f;
            if (!subtile_inside(q0w, kbs, L, hw)) {
                const int rel0 = kbs + 4 * h - win.lo;  // key − lo of the lane's row r = 0
#pragma unroll
                for (int r = 0; r < 16; ++r)
                    if (!in_range(win, rel0 + 8 * (r >> 2) + (r & 3))) s[r] = NEG_INF;
            }
#pragma unroll
            for (int r = 0; r < 16; ++r) mx = fmaxf(mx, s[r]);
            mx = fmaxf(mx, __shfl_xor(mx, 32, 64)) * scale_log2;
            // The running max moves only when a score passes it by more than 2^LAZY_RESCALE (the
            // probabilities then stay below 2^LAZY_RESCALE): most subtiles rescale nothing.
            const bool grow = mx > m + LAZY_RESCALE;
            if (__any(grow)) {  // wave-uniform
                const float mnew = grow ? mx : m;
                const float alpha = fast_exp2(m - mnew);  // exactly 1 where the max stays
                l *= alpha;
                o[0] *= alpha;
                o[1] *= alpha;
                m = mnew;
            }
            float mm = m;  // pr = 2^(t − mm): the probabilities, times 2^ep for two-piece products
            if constexpr (NP == 2) {
                const float d = mx - m;
                const int et = d > -200.0f ? min(126, 14 - (int)floorf(d) - ek) : 126;
                if (et < ep) {
                    const float f = ldexpf(1.0f, et - ep);
                    l *= f;
                    o[0] *= f;
                    o[1] *= f;
                    ep = et;
                }
                mm = m - (float)ep;
            }
            float pr[16];
            float sum = 0.0f;
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                pr[r] = fast_exp2(__builtin_fmaf(s[r], scale_log2, -mm));
                sum += pr[r];
            }
            l += sum;
            if (DROP) {
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const int key = kbs + 8 * (r >> 2) + 4 * h + (r & 3);
                    const float u = uniform01(p.seed, attn_dropout_index(head, start + q, key));
                    pr[r] = u < p.p_drop ? 0.0f : pr[r] * p.keep;
                }
            }
            // Oᵀ += Vᵀ·Pᵀ over the subtile's 32 keys in two 16-key steps.
#pragma unroll
            for (int u = 0; u < 2; ++u) {
                V8 ph[NP];
                split_col16u<NP>(pr, u, ph, one);
#pragma unroll
                for (int dt = 0; dt < 2; ++dt) {
                    V8 vf[NP];
                    swz_col_frag<TILE, NP>(Vs, 32 * st + 16 * u, dt, lane, vf);
                    o[dt] = Pieces<NP>::mma(vf, ph, o[dt]);
                }
            }
        }
    }

    const float lt = l + __shfl_xor(l, 32, 64);
    unsigned am = 0;
    if (qvalid) {
        const float inv = lt > 0.0f ? (NP == 2 ? ldexpf(1.0f / lt, -eq) : 1.0f / lt) : 0.0f;
        am = store_acc<D>(o, p.context + (long)(start + q) * p.hidden + qcol, h, inv);
        if (p.context16) store_acc16<D>(o, p.context16 + (long)(start + q) * p.hidden + qcol, h, inv);
        if (h == 0) p.lse[(long)(start + q) * p.heads + head] = lt > 0.0f ? (m + log2f(lt)) - (NP == 2 ? (float)ep : 0.0f)
                                                                     : __builtin_huge_valf();
    }
    block_amax_fold(am, p.amax);
}

// ------------------------------------------------------------------------------------ backward

// dots[row, head] = Σ_d dO · O: the row constant c = Σ_j p_j·dp_j of Ops.cs:408-409.
template <int D>
__global__ __launch_bounds__(THREADS) void attn_dot_kernel(const float* __restrict__ dctx, const float* __restrict__ ctx,
                                                           int rows, int hidden, int heads, float* __restrict__ dots) {
    const long i = blockIdx.x * (long)THREADS + threadIdx.x;
    const long total = (long)rows * hidden;
    float v = i < total ? dctx[i] * ctx[i] : 0.0f;
#pragma unroll
    for (int o = D / 2; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    if (i < total && (i % D) == 0) {
        const long row = i / hidden;
        const int head = (int)((i - row * hidden) / D);
        dots[row * heads + head] = v;
    }
}

// Two waves per SIMD: the block's keys sit in LDS (read back as b128 fragments by the wave that owns them)
// and each query tile is loaded straight into LDS, which keeps the kernel under 256 registers without
// spills; the other resident block hides the tile loads.
template <int D>
__global__ __launch_bounds__(THREADS, 2) void attn_bwd_dkv_kernel(Params p) {
    using S = Shape<D>;
    __shared__ __attribute__((aligned(16))) float Qs[TILE * S::KS];
    __shared__ __attribute__((aligned(16))) float Os[TILE * S::VS];  // dO rows
    __shared__ float lse_s[TILE], dot_s[TILE];
    __shared__ __attribute__((aligned(16))) float Ks[BLOCK_ROWS * S::KS];  // the block's keys

    const BlockCoord bc = block_coord(p);
    const int seg = bc.seg, head = bc.head;
    const int start = p.seg_start[seg], L = p.seg_len[seg];
    const int kb0 = bc.row0;
    if (kb0 >= L) return;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, h = lane >> 5, lr = lane & 31;
    const int k0w = kb0 + wave * WAVE_ROWS;
    const int key = k0w + lr;
    const bool kvalid = key < L;
    const bool rope = p.cos_t != nullptr;
    const int hw = p.half_window;
    const long stride = 3L * p.hidden;
    const int qcol = head * D, kcol = p.hidden + head * D, vcol = 2 * p.hidden + head * D;

    f32x4 vv[S::G];
    const long krow = (long)(start + (kvalid ? key : 0)) * stride;
    load_lane_row<D>(p.qkv + krow + vcol, kvalid, h, vv);
    {
        f32x4 kv[S::G];
        load_lane_row<D>(p.qkv + krow + kcol, kvalid, h, kv);
#pragma unroll
        for (int g = 0; g < S::G; ++g) st4(Ks + (wave * WAVE_ROWS + lr) * S::KS + 8 * g + 4 * h, kv[g]);
    }
    const float* krow_s = Ks + (wave * WAVE_ROWS + lr) * S::KS + 4 * h;

    int qbeg = 0, qend = L, wbeg = 0, wend = L;
    if (hw >= 0) {
        qbeg = max(0, kb0 - hw);
        qend = min(L, kb0 + BLOCK_ROWS + hw);
        wbeg = max(0, k0w - hw);
        wend = min(L, k0w + WAVE_ROWS + hw);
    }

    f32x16 dk[S::ND], dv[S::ND];
#pragma unroll
    for (int dt = 0; dt < S::ND; ++dt) {
        dk[dt] = f32x16{};
        dv[dt] = f32x16{};
    }

    // Q rows, dO rows from dcontext [rows, hidden], and the per-row lse / dots, fetched one tile ahead
    // of the products.
    const float* qbase = p.qkv + (long)start * stride + qcol;
    const float* obase = p.dcontext + (long)start * p.hidden + qcol;
    for (int qt0 = qbeg; qt0 < qend; qt0 += TILE) {
        __syncthreads();
        {
            PlainStage<D> qst, ost;
            fetch_plain<D>(qst, qbase, stride, L, qt0);
            fetch_plain<D>(ost, obase, p.hidden, L, qt0);
            const int t = qt0 + (int)threadIdx.x;
            if (threadIdx.x < TILE) {
                lse_s[threadIdx.x] = t < L ? p.lse[(long)(start + t) * p.heads + head] : __builtin_huge_valf();
                dot_s[threadIdx.x] = t < L ? p.dots[(long)(start + t) * p.heads + head] : 0.0f;
            }
            commit_plain<D, S::KS>(qst, Qs);
            commit_plain<D, S::VS>(ost, Os);
        }
        __syncthreads();
#pragma unroll
        for (int st = 0; st < TILE / 32; ++st) {
            const int qbs = qt0 + 32 * st;
            // Wave-uniform: outside this wave's window, or a wave whose keys all lie past the segment end.
            if (qbs >= wend || qbs + 32 <= wbeg || qbs >= qend || k0w >= L) continue;
            // S[q][key] = Q·Kᵀ: lane column = its key, rows = 16 queries.
            f32x16 s = f32x16{}, dp = f32x16{};
            const float* qrow = Qs + (32 * st + lr) * S::KS + 4 * h;
            const float* orow = Os + (32 * st + lr) * S::VS + 4 * h;
#pragma unroll
            for (int g = 0; g < S::G; ++g) {
                const f32x4 qf = ld4(qrow + 8 * g);
                const f32x4 of = ld4(orow + 8 * g);
                const f32x4 kf = ld4(krow_s + 8 * g);
#pragma unroll
                for (int c = 0; c < 4; ++c) {
                    s = mfma(qf[c], kf[c], s);
                    dp = mfma(of[c], vv[g][c], dp);
                }
            }
            float pm[16], ds[16];
            if (p.p_drop == 0.0f && subtile_inside(qbs, k0w, L, hw)) {
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const int ql = 32 * st + 8 * (r >> 2) + 4 * h + (r & 3);
                    const float pr = fast_exp2(s[r] * p.scale_log2 - lse_s[ql]);
                    pm[r] = pr;
                    ds[r] = pr * (dp[r] - dot_s[ql]) * p.scale;
                }
            } else {
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const int ql = 32 * st + 8 * (r >> 2) + 4 * h + (r & 3);
                    const int qq = qt0 + ql;
                    const bool ok = in_window(qq, key, L, hw) && kvalid;
                    const float pr = ok ? fast_exp2(s[r] * p.scale_log2 - lse_s[ql]) : 0.0f;
                    float mask = 1.0f;
                    if (p.p_drop > 0.0f && ok)
                        mask = uniform01(p.seed, attn_dropout_index(head, start + qq, key)) < p.p_drop ? 0.0f : p.keep;
                    pm[r] = pr * mask;
                    ds[r] = pr * (dp[r] * mask - dot_s[ql]) * p.scale;
                }
            }
            // dVᵀ += dOᵀ·(P∘M) and dKᵀ += Qᵀ·dS, reducing over the 32 queries of this subtile.
#pragma unroll
            for (int dt = 0; dt < S::ND; ++dt) {
                const float* ocol = Os + (32 * st + 4 * h) * S::VS + dt * 32 + lr;
                const float* qcolp = Qs + (32 * st + 4 * h) * S::KS + dt * 32 + lr;
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const int rr = 8 * (r >> 2) + (r & 3);
                    dv[dt] = mfma(ocol[rr * S::VS], pm[r], dv[dt]);
                    dk[dt] = mfma(qcolp[rr * S::KS], ds[r], dk[dt]);
                }
            }
        }
    }

    unsigned am = 0;
    if (kvalid) {
        if (rope) inverse_rope_acc<D>(dk, p, key, h);
        float* dst = p.dqkv + (long)(start + key) * stride;
        am = max(store_acc<D>(dk, dst + kcol, h, 1.0f), store_acc<D>(dv, dst + vcol, h, 1.0f));
    }
    block_amax_fold(am, p.amax);
}

template <int D>
__global__ __launch_bounds__(THREADS, 2) void attn_bwd_dq_kernel(Params p) {
    using S = Shape<D>;
    __shared__ __attribute__((aligned(16))) float Ks[TILE * S::KS];
    __shared__ __attribute__((aligned(16))) float Vs[TILE * S::KS];

    const BlockCoord bc = block_coord(p);
    const int seg = bc.seg, head = bc.head;
    const int start = p.seg_start[seg], L = p.seg_len[seg];
    const int qb0 = bc.row0;
    if (qb0 >= L) return;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, h = lane >> 5, lr = lane & 31;
    const int q0w = qb0 + wave * WAVE_ROWS;
    const int q = q0w + lr;
    const bool qvalid = q < L;
    const bool rope = p.cos_t != nullptr;
    const int hw = p.half_window;
    const long stride = 3L * p.hidden;
    const int qcol = head * D, kcol = p.hidden + head * D, vcol = 2 * p.hidden + head * D;

    f32x4 qv[S::G], ov[S::G];
    const int qs = start + (qvalid ? q : 0);
    load_lane_row<D>(p.qkv + (long)qs * stride + qcol, qvalid, h, qv);
    load_lane_row<D>(p.dcontext + (long)qs * p.hidden + qcol, qvalid, h, ov);
    const float lse = qvalid ? p.lse[(long)qs * p.heads + head] : __builtin_huge_valf();
    const float dot = qvalid ? p.dots[(long)qs * p.heads + head] : 0.0f;

    int kbeg = 0, kend = L, wbeg = 0, wend = L;
    if (hw >= 0) {
        kbeg = max(0, qb0 - hw);
        kend = min(L, qb0 + BLOCK_ROWS + hw);
        wbeg = max(0, q0w - hw);
        wend = min(L, q0w + WAVE_ROWS + hw);
    }

    f32x16 dq[S::ND];
#pragma unroll
    for (int dt = 0; dt < S::ND; ++dt) dq[dt] = f32x16{};

    const float* kbase = p.qkv + (long)start * stride + kcol;
    const float* vbase = p.qkv + (long)start * stride + vcol;
    PlainStage<D> kst, vst;
    fetch_plain<D>(kst, kbase, stride, L, kbeg);
    fetch_plain<D>(vst, vbase, stride, L, kbeg);
    for (int kt0 = kbeg; kt0 < kend; kt0 += TILE) {
        __syncthreads();
        commit_plain<D, S::KS>(kst, Ks);
        commit_plain<D, S::KS>(vst, Vs);
        __syncthreads();
        if (kt0 + TILE < kend) {  // block-uniform
            fetch_plain<D>(kst, kbase, stride, L, kt0 + TILE);
            fetch_plain<D>(vst, vbase, stride, L, kt0 + TILE);
        }
#pragma unroll
        for (int st = 0; st < TILE / 32; ++st) {
            const int kbs = kt0 + 32 * st;
            // Wave-uniform: outside this wave's window, or a wave whose rows all lie past the segment end.
            if (kbs >= wend || kbs + 32 <= wbeg || kbs >= kend || q0w >= L) continue;
            f32x16 s = f32x16{}, dp = f32x16{};
            const float* krow = Ks + (32 * st + lr) * S::KS + 4 * h;
            const float* vrow = Vs + (32 * st + lr) * S::KS + 4 * h;
#pragma unroll
            for (int g = 0; g < S::G; ++g) {
                const f32x4 kf = ld4(krow + 8 * g);
                const f32x4 vf = ld4(vrow + 8 * g);
#pragma unroll
                for (int c = 0; c < 4; ++c) {
                    s = mfma(kf[c], qv[g][c], s);
                    dp = mfma(vf[c], ov[g][c], dp);
                }
            }
            float ds[16];
            if (p.p_drop == 0.0f && subtile_inside(q0w, kbs, L, hw)) {
#pragma unroll
                for (int r = 0; r < 16; ++r) ds[r] = fast_exp2(s[r] * p.scale_log2 - lse) * (dp[r] - dot) * p.scale;
            } else {
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const int key = kbs + 8 * (r >> 2) + 4 * h + (r & 3);
                    const bool ok = in_window(q, key, L, hw);
                    const float pr = ok ? fast_exp2(s[r] * p.scale_log2 - lse) : 0.0f;
                    float mask = 1.0f;
                    if (p.p_drop > 0.0f && ok)
                        mask = uniform01(p.seed, attn_dropout_index(head, start + q, key)) < p.p_drop ? 0.0f : p.keep;
                    ds[r] = pr * (dp[r] * mask - dot) * p.scale;
                }
            }
#pragma unroll
            for (int dt = 0; dt < S::ND; ++dt) {
                const float* kcolp = Ks + (32 * st + 4 * h) * S::KS + dt * 32 + lr;
#pragma unroll
                for (int r = 0; r < 16; ++r) dq[dt] = mfma(kcolp[(8 * (r >> 2) + (r & 3)) * S::KS], ds[r], dq[dt]);
            }
        }
    }

    unsigned am = 0;
    if (qvalid) {
        if (rope) inverse_rope_acc<D>(dq, p, q, h);
        am = store_acc<D>(dq, p.dqkv + (long)(start + q) * stride + qcol, h, 1.0f);
    }
    block_amax_fold(am, p.amax);
}

// The backward on split products, tiles of 32 query or key rows: with the dK/dV kernel's V planes (the
// block's 128 keys), 64-row tiles would not leave room for two blocks per CU.
constexpr int BT = 32;

// Each wave owns 32 keys: K split once into registers, V split once into the block's LDS planes. The
// query tiles are committed to one swizzled layout each (Q and dO), the next tile's rows load while the
// current one is multiplied, and the products over queries read Qᵀ and dOᵀ with the transposing reads.
template <int D, bool DROP, int NP = 3>
__global__ __launch_bounds__(THREADS, 2) void attn_bwd_dkv_x6_kernel(Params p) {
    static_assert(D == 64, "split-product attention is written for head_dim 64");
    __shared__ __attribute__((aligned(16))) __bf16 Qs[NP * BT * 64];
    __shared__ __attribute__((aligned(16))) __bf16 Os[NP * BT * 64];
    __shared__ __attribute__((aligned(16))) __bf16 Vs[NP * BLOCK_ROWS * 64];
    __shared__ __attribute__((aligned(16))) float lse_s[BT];
    __shared__ __attribute__((aligned(16))) float dot_s[BT];

    const BlockCoord bc = block_coord(p);
    const int seg = bc.seg, head = bc.head;
    const int start = p.seg_start[seg], L = p.seg_len[seg];
    const int kb0 = bc.row0;
    if (kb0 >= L) return;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, h = lane >> 5, lr = lane & 31;
    const int k0w = kb0 + wave * WAVE_ROWS;
    const int key = k0w + lr;
    const bool kvalid = key < L;
    const bool rope = p.cos_t != nullptr;
    const int hw = p.half_window;
    const long stride = 3L * p.hidden;
    const int qcol = head * D, kcol = p.hidden + head * D, vcol = 2 * p.hidden + head * D;

    typedef typename Pieces<NP>::V8 V8;
    // Two-piece products: q, k and v scaled by 2^eq (from the qkv magnitude), dO by 2^eo, P and dS by the
    // lane's running 2^ep and 2^eds (lane_scale_update). The scores' and dP's accumulators carry the
    // operand factors, taken out with the softmax scale and as dP is used; the gradients' accumulators
    // at their store.
    int eq = 0, eo = 0, ep = 126, eds = 126;
    if constexpr (NP == 2) {
        eq = pair_scale_exp(amax_group_max(p.amax_qkv));
        eo = pair_scale_exp(amax_group_max(p.amax_do));
    }
    const float sq = exp2_int(eq), so = exp2_int(eo);
    const float scale_log2 = NP == 2 ? ldexpf(p.scale_log2, -2 * eq) : p.scale_log2;
    const float udp = NP == 2 ? ldexpf(1.0f, -(eo + eq)) : 1.0f;
    const float dsc = p.scale * udp;
    const float dmul = NP == 2 ? 1.0f : dsc;
    V8 kh[4][NP];
    const long krow = (long)(start + (kvalid ? key : 0)) * stride;
    split_lane_row<NP>(p.qkv + krow + kcol, kvalid, h, kh, sq);
    {
        RowStage<BLOCK_ROWS> vst;
        fetch_rows<BLOCK_ROWS>(vst, p.qkv + (long)start * stride + vcol, stride, L, kb0);
        commit_swz<BLOCK_ROWS, NP>(vst, Vs, sq);
    }

    int qbeg = 0, qend = L, wbeg = 0, wend = L;
    if (hw >= 0) {
        qbeg = max(0, kb0 - hw);
        qend = min(L, kb0 + BLOCK_ROWS + hw);
        wbeg = max(0, k0w - hw);
        wend = min(L, k0w + WAVE_ROWS + hw);
    }

    const WindowRange win = window_range(key, L, hw);
    f32x16 dk[2], dv[2];
#pragma unroll
    for (int dt = 0; dt < 2; ++dt) {
        dk[dt] = f32x16{};
        dv[dt] = f32x16{};
    }

    const float* qbase = p.qkv + (long)start * stride + qcol;
    const float* obase = p.dcontext + (long)start * p.hidden + qcol;
    RowStage<BT> qst, ost;
    float lse_n = __builtin_huge_valf(), dot_n = 0.0f;
    auto fetch = [&](int t0) {
        fetch_rows<BT>(qst, qbase, stride, L, t0);
        fetch_rows<BT>(ost, obase, p.hidden, L, t0);
        const int t = t0 + (int)threadIdx.x;
        if (threadIdx.x < BT) {
            lse_n = t < L ? p.lse[(long)(start + t) * p.heads + head] : __builtin_huge_valf();
            dot_n = t < L ? p.dots[(long)(start + t) * p.heads + head] : 0.0f;
        }
    };
    if (qbeg < qend) fetch(qbeg);
    for (int qt0 = qbeg; qt0 < qend; qt0 += BT) {
        __syncthreads();  // the previous tile's fragments (and, first time round, V's commit) are read
        commit_swz<BT, NP>(qst, Qs, sq);
        commit_swz<BT, NP>(ost, Os, so);
        if (threadIdx.x < BT) {
            lse_s[threadIdx.x] = lse_n;
            dot_s[threadIdx.x] = NP == 2 ? ldexpf(dot_n, eo + eq) : dot_n;  // in dP's scaled units
        }
        __syncthreads();
        if (qt0 + BT < qend) fetch(qt0 + BT);  // block-uniform
        // Wave-uniform: outside this wave's window, or a wave whose keys all lie past the segment end.
        if (qt0 >= wend || qt0 + BT <= wbeg || k0w >= L) continue;
        // S[q][key] = Q·Kᵀ and dP = dO·Vᵀ: lane column = its key, rows = 16 queries.
        f32x16 s = f32x16{}, dp = f32x16{};
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) {
            V8 f[NP], vh[NP];
            swz_row_frag<BT, NP>(Qs, lr, ks, h, f);
            s = Pieces<NP>::mma(f, kh[ks], s);
            swz_row_frag<BT, NP>(Os, lr, ks, h, f);
            swz_row_frag<BLOCK_ROWS, NP>(Vs, wave * WAVE_ROWS + lr, ks, h, vh);
            dp = Pieces<NP>::mma(f, vh, dp);
        }
        // dP stays in its operands' scaled units (2^(eo + eq)), the row constants were staged in the same
        // units and the units' factor sits in the softmax scale dsc, which the two-piece split applies
        // (dmul = 1) and the three-piece form multiplies in (dmul = dsc).
        float pm[16], ds[16];
        const int rel0 = qt0 + 4 * h - win.lo;  // query − lo of the lane's row r = 0
        // Outside the window the exponent is −∞ and the probability exactly 0 (no branch per score).
        if constexpr (!DROP) {
            const bool inside = subtile_inside(qt0, k0w, L, hw);
            // The row constants of the lane's 16 queries, rows 8u + 4h … +3 for u < 4: one b128 read per u.
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const f32x4 lq = *reinterpret_cast<const f32x4*>(lse_s + 8 * u + 4 * h);
                const f32x4 dq4 = *reinterpret_cast<const f32x4*>(dot_s + 8 * u + 4 * h);
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const int r = 4 * u + i;
                    const bool ok = inside || in_range(win, rel0 + 8 * u + i);
                    pm[r] = fast_exp2(ok ? s[r] * scale_log2 - lq[i] : NEG_INF);
                    ds[r] = pm[r] * (dp[r] - dq4[i]) * dmul;
                }
            }
        } else {
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int ql = 8 * (r >> 2) + 4 * h + (r & 3);
                const bool ok = in_range(win, rel0 + 8 * (r >> 2) + (r & 3));
                const float pr = fast_exp2(ok ? s[r] * scale_log2 - lse_s[ql] : NEG_INF);
                const float drop =
                    uniform01(p.seed, attn_dropout_index(head, start + qt0 + ql, key)) < p.p_drop ? 0.0f : p.keep;
                const float mask = ok ? drop : 1.0f;
                pm[r] = pr * mask;
                ds[r] = pr * (dp[r] * mask - dot_s[ql]) * dmul;
            }
        }
        // dVᵀ += dOᵀ·(P∘M) and dKᵀ += Qᵀ·dS over the tile's 32 queries in two 16-query steps; dS is
        // ds·dsc, the constant applied by the split together with the lane's scale.
        if constexpr (NP == 2) {
            ep = lane_scale_update(pm, ep, dv);
            eds = lane_scale_update(ds, eds, dk, dsc);
        }
#pragma unroll
        for (int u = 0; u < 2; ++u) {
            V8 ph[NP], dh[NP];
            split_col16<NP>(pm, u, ph, exp2_int(NP == 2 ? ep : 0));
            split_col16<NP>(ds, u, dh, dsc * exp2_int(NP == 2 ? eds : 0));
#pragma unroll
            for (int dt = 0; dt < 2; ++dt) {
                V8 f[NP];
                swz_col_frag<BT, NP>(Os, 16 * u, dt, lane, f);
                dv[dt] = Pieces<NP>::mma(f, ph, dv[dt]);
                swz_col_frag<BT, NP>(Qs, 16 * u, dt, lane, f);
                dk[dt] = Pieces<NP>::mma(f, dh, dk[dt]);
            }
        }
    }

    // The epilogue's lane values are taken again after the loop rather than held across it.
    int te = threadIdx.x;
    asm volatile("" : "+v"(te));
    const int he = (te & 63) >> 5, keye = kb0 + (te >> 6) * WAVE_ROWS + (te & 31);
    unsigned am = 0;
    if (keye < L) {
        if (rope) inverse_rope_acc<D>(dk, p, keye, he);
        float* dst = p.dqkv + (long)(start + keye) * stride;
        const float uk = NP == 2 ? ldexpf(1.0f, -(eds + eq)) : 1.0f, uv = NP == 2 ? ldexpf(1.0f, -(ep + eo)) : 1.0f;
        am = max(store_acc<D>(dk, dst + kcol, he, uk), store_acc<D>(dv, dst + vcol, he, uv));
    }
    block_amax_fold(am, p.amax);
}

// Each wave owns 32 queries: q split once into registers, dO split once into the block's LDS planes (each
// wave reads back only its own rows), which keeps the two-piece form within three waves per SIMD.
template <int D, bool DROP, int NP = 3>
__global__ __launch_bounds__(THREADS, NP == 2 ? 3 : 2) void attn_bwd_dq_x6_kernel(Params p) {
    static_assert(D == 64, "split-product attention is written for head_dim 64");
    __shared__ __attribute__((aligned(16))) __bf16 Ks[NP * BT * 64];  // K tile, swizzled [key][d]
    __shared__ __attribute__((aligned(16))) __bf16 Vs[NP * BT * 64];  // V tile, swizzled [key][d]
    __shared__ __attribute__((aligned(16))) __bf16 Ob[NP * BLOCK_ROWS * 64];  // the block's dO rows, swizzled

    const BlockCoord bc = block_coord(p);
    const int seg = bc.seg, head = bc.head;
    const int start = p.seg_start[seg], L = p.seg_len[seg];
    const int qb0 = bc.row0;
    if (qb0 >= L) return;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, h = lane >> 5, lr = lane & 31;
    const int q0w = qb0 + wave * WAVE_ROWS;
    const int q = q0w + lr;
    const bool qvalid = q < L;
    const bool rope = p.cos_t != nullptr;
    const int hw = p.half_window;
    const long stride = 3L * p.hidden;
    const int qcol = head * D, kcol = p.hidden + head * D, vcol = 2 * p.hidden + head * D;

    typedef typename Pieces<NP>::V8 V8;
    // Two-piece products: q, k and v scaled by 2^eq (from the qkv magnitude), dO by 2^eo, P and dS by the
    // lane's running 2^ep and 2^eds (lane_scale_update). The scores' and dP's accumulators carry the
    // operand factors, taken out with the softmax scale and as dP is used; the gradients' accumulators
    // at their store.
    int eq = 0, eo = 0, ep = 126, eds = 126;
    if constexpr (NP == 2) {
        eq = pair_scale_exp(amax_group_max(p.amax_qkv));
        eo = pair_scale_exp(amax_group_max(p.amax_do));
    }
    const float sq = exp2_int(eq), so = exp2_int(eo);
    const float scale_log2 = NP == 2 ? ldexpf(p.scale_log2, -2 * eq) : p.scale_log2;
    const float udp = NP == 2 ? ldexpf(1.0f, -(eo + eq)) : 1.0f;
    // The lane's q, dO and context rows, then the first K/V tile: the loads overlap before anything waits.
    const int qs = start + (qvalid ? q : 0);
    LaneRow qrow, orow, crow;
    qrow.load(p.qkv + (long)qs * stride + qcol, h);
    orow.load(p.dcontext + (long)qs * p.hidden + qcol, h);
    crow.load(p.context + (long)qs * p.hidden + qcol, h);
    const float lse = qvalid ? p.lse[(long)qs * p.heads + head] : __builtin_huge_valf();

    int kbeg = 0, kend = L, wbeg = 0, wend = L;
    if (hw >= 0) {
        kbeg = max(0, qb0 - hw);
        kend = min(L, qb0 + BLOCK_ROWS + hw);
        wbeg = max(0, q0w - hw);
        wend = min(L, q0w + WAVE_ROWS + hw);
    }
    const float* kbase = p.qkv + (long)start * stride + kcol;
    const float* vbase = p.qkv + (long)start * stride + vcol;
    RowStage<BT> kst, vst;
    fetch_rows<BT>(kst, kbase, stride, L, kbeg);
    fetch_rows<BT>(vst, vbase, stride, L, kbeg);
    __builtin_amdgcn_sched_barrier(0);  // the tile's loads are issued before the rows' splits wait for them

    V8 qh[4][NP];
    qrow.split<NP>(qh, sq);
    {
        V8 oh[4][NP];
        orow.split<NP>(oh, so);
#pragma unroll
        for (int ks = 0; ks < 4; ++ks)
#pragma unroll
            for (int pl = 0; pl < NP; ++pl)
                *reinterpret_cast<V8*>(Ob + pl * BLOCK_ROWS * 64 + swz(wave * WAVE_ROWS + lr, 16 * ks + 8 * h)) = oh[ks][pl];
    }
    // The row constant Σ_d dO·O (Ops.cs:408-409) from the lane's half of the row and its partner's, written
    // for the dK/dV kernel, which runs after this one.
    float dot = 0.0f;
#pragma unroll
    for (int s4 = 0; s4 < 8; ++s4) {
        const f32x4 a = orow.v[s4], b = crow.v[s4];
        dot += a[0] * b[0] + a[1] * b[1] + a[2] * b[2] + a[3] * b[3];
    }
    dot += __shfl_xor(dot, 32, 64);
    if (qvalid && h == 0) p.dots[(long)qs * p.heads + head] = dot;
    const float dotu = NP == 2 ? ldexpf(dot, eo + eq) : dot;  // in dP's scaled units
    const float dsc = p.scale * udp;
    const float dmul = NP == 2 ? 1.0f : dsc;

    const WindowRange win = window_range(q, L, hw);
    f32x16 dq[2];
    dq[0] = f32x16{};
    dq[1] = f32x16{};

    for (int kt0 = kbeg; kt0 < kend; kt0 += BT) {
        __syncthreads();
        commit_swz<BT, NP>(kst, Ks, sq);
        commit_swz<BT, NP>(vst, Vs, sq);
        __syncthreads();
        if (kt0 + BT < kend) {  // block-uniform
            fetch_rows<BT>(kst, kbase, stride, L, kt0 + BT);
            fetch_rows<BT>(vst, vbase, stride, L, kt0 + BT);
        }
        // Wave-uniform: outside this wave's window, or a wave whose rows all lie past the segment end.
        if (kt0 >= wend || kt0 + BT <= wbeg || q0w >= L) continue;
        // Sᵀ = K·Qᵀ and dPᵀ = V·dOᵀ: lane column = its query, rows = 16 keys.
        f32x16 s = f32x16{}, dp = f32x16{};
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) {
            V8 f[NP];
            swz_row_frag<BT, NP>(Ks, lr, ks, h, f);
            s = Pieces<NP>::mma(f, qh[ks], s);
            V8 o[NP];
            swz_row_frag<BT, NP>(Vs, lr, ks, h, f);
            swz_row_frag<BLOCK_ROWS, NP>(Ob, wave * WAVE_ROWS + lr, ks, h, o);
            dp = Pieces<NP>::mma(f, o, dp);
        }
        // dP stays in its operands' scaled units (2^(eo + eq)); the row constant is taken into the same units
        // (dotu) and the units' factor into the softmax scale dsc, which the two-piece split applies
        // (dmul = 1) and the three-piece form multiplies in (dmul = dsc).
        float ds[16];
        const int rel0 = kt0 + 4 * h - win.lo;  // key − lo of the lane's row r = 0
        if (!DROP) {
            if (subtile_inside(q0w, kt0, L, hw)) {
#pragma unroll
                for (int r = 0; r < 16; ++r) ds[r] = fast_exp2(s[r] * scale_log2 - lse) * (dp[r] - dotu) * dmul;
            } else {
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const bool ok = in_range(win, rel0 + 8 * (r >> 2) + (r & 3));
                    const float pr = fast_exp2(ok ? s[r] * scale_log2 - lse : NEG_INF);
                    ds[r] = pr * (dp[r] - dotu) * dmul;
                }
            }
        } else {
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int key = kt0 + 8 * (r >> 2) + 4 * h + (r & 3);
                const bool ok = in_range(win, rel0 + 8 * (r >> 2) + (r & 3));
                const float pr = fast_exp2(ok ? s[r] * scale_log2 - lse : NEG_INF);
                const float drop =
                    uniform01(p.seed, attn_dropout_index(head, start + q, key)) < p.p_drop ? 0.0f : p.keep;
                const float mask = ok ? drop : 1.0f;
                ds[r] = pr * (dp[r] * mask - dotu) * dmul;
            }
        }
        // dQᵀ += Kᵀ·dSᵀ over the tile's 32 keys in two 16-key steps; dS is ds·dsc, the constant applied by
        // the split together with the lane's scale.
        if constexpr (NP == 2) eds = lane_scale_update(ds, eds, dq, dsc);
#pragma unroll
        for (int u = 0; u < 2; ++u) {
            V8 dh[NP];
            split_col16<NP>(ds, u, dh, dsc * exp2_int(NP == 2 ? eds : 0));
#pragma unroll
            for (int dt = 0; dt < 2; ++dt) {
                V8 f[NP];
                swz_col_frag<BT, NP>(Ks, 16 * u, dt, lane, f);
                dq[dt] = Pieces<NP>::mma(f, dh, dq[dt]);
            }
        }
    }

    unsigned am = 0;
    if (qvalid) {
        if (rope) inverse_rope_acc<D>(dq, p, q, h);
        am = store_acc<D>(dq, p.dqkv + (long)(start + q) * stride + qcol, h, NP == 2 ? ldexpf(1.0f, -(eds + eq)) : 1.0f);
    }
    block_amax_fold(am, p.amax);
}

// RoPE at segment-local positions on the q and k columns of one segment's qkv rows, written to `out`
// together with an unchanged copy of v (Gather, Ops.cs:297-313). One thread per float4 unit of a row:
// the first hidden/4 units are (d, d + D/2) pairs of q and then k, the next hidden/4 copy v.
// amax (optional): max|written value| folded into that word group (the magnitude the two-piece kernels take
// their scale from, in the same pass).
__global__ void rope_rows_kernel(const float* __restrict__ qkv, const int* __restrict__ seg_start,
                                 const int* __restrict__ seg_len, int hidden, int head_dim,
                                 const float* __restrict__ cos_t, const float* __restrict__ sin_t,
                                 float* __restrict__ out, unsigned* amax) {
    const int seg = blockIdx.y;
    const int start = seg_start[seg], L = seg_len[seg];
    const int units = hidden / 2;  // per row
    const long idx = (long)blockIdx.x * blockDim.x + threadIdx.x;
    const int t = (int)(idx / units), u = (int)(idx - (long)t * units);
    unsigned m = 0;
    if (t < L) {  // (no early return: the whole block reaches the fold)
        const long row = (long)(start + t) * 3 * hidden;
        const int half = head_dim / 2;
        if (u < hidden / 4) {
            const int per_part = hidden / 8;  // float4 pair units in q (or k)
            const int part = u / per_part, v = u - part * per_part;
            const int head = v / (half / 4), j = (v - head * (half / 4)) * 4;
            const long col = (long)part * hidden + head * head_dim + j;
            const f32x4 a = ld4(qkv + row + col), b = ld4(qkv + row + col + half);
            const f32x4 c = ld4(cos_t + (long)t * half + j), s = ld4(sin_t + (long)t * half + j);
            const f32x4 ra = a * c - b * s, rb = b * c + a * s;
            st4(out + row + col, ra);
            st4(out + row + col + half, rb);
            m = max(amax_bits4(ra), amax_bits4(rb));
        } else {
            const long col = 2L * hidden + (long)(u - hidden / 4) * 4;
            const f32x4 v = ld4(qkv + row + col);
            st4(out + row + col, v);
            m = amax_bits4(v);
        }
    }
    block_amax_fold(m, amax);
}

Params make_params(const AttentionArgs& a) {
    Params p{};
    p.qkv = a.qkv;
    p.seg_start = a.seg_start;
    p.seg_len = a.seg_len;
    p.blocks = a.blocks;
    p.hidden = a.hidden;
    p.heads = a.heads;
    p.half_window = a.half_window;
    p.scale = a.scale;
    p.scale_log2 = a.scale * 1.4426950408889634f;
    p.p_drop = a.p_drop;
    p.keep = a.p_drop > 0.0f ? 1.0f / (1.0f - a.p_drop) : 1.0f;
    p.seed = a.seed;
    p.cos_t = a.cos_table;
    p.sin_t = a.sin_table;
    return p;
}

// The qkv the kernels read: `a.qkv` itself when RoPE is already applied (or absent), else a rotated
// copy of its segment rows in workspace slot 4, its magnitude folded into `amax` when given.
const float* rotated_qkv(laya_ctx* ctx, const AttentionArgs& a, unsigned* amax = nullptr) {
    if (a.cos_table == nullptr || a.rotated) return a.qkv;
    LAYA_REQUIRE(a.rows >= 0, "attention: row count needed to rotate q and k");
    LAYA_REQUIRE(a.hidden % 8 == 0 && (a.head_dim / 2) % 4 == 0, "attention: RoPE needs head_dim % 8 == 0");
    float* out = static_cast<float*>(ctx->workspace(4, sizeof(float) * (size_t)std::max(a.rows, 1) * 3 * a.hidden));
    const long threads = (long)a.max_len * (a.hidden / 2);
    dim3 grid((unsigned)((threads + 255) / 256), a.nseg);
    ProfileScope scope(ctx, "attention_rope", 0.0, 4.0 * 3.0 * a.hidden * (double)a.rows * 2.0);
    LAYA_LAUNCH(rope_rows_kernel, grid, dim3(256), 0, ctx->stream, a.qkv, a.seg_start, a.seg_len, a.hidden,
                       a.head_dim, a.cos_table, a.sin_table, out, amax);
    check_launch("rope_rows_kernel");
    return out;
}

// The attention kernels' grid: one workgroup per listed block and head, else (row blocks, segments, heads).
dim3 block_grid(const AttentionArgs& a) {
    if (a.blocks) return dim3((unsigned)(a.n_blocks * a.heads));
    return dim3((a.max_len + BLOCK_ROWS - 1) / BLOCK_ROWS, a.nseg, a.heads);
}

void check_args(const AttentionArgs& a) {
    LAYA_REQUIRE(a.heads > 0 && a.hidden == a.heads * a.head_dim, "attention: hidden must equal heads × head_dim");
    LAYA_REQUIRE(a.head_dim == 32 || a.head_dim == 64, "attention: head_dim must be 32 or 64");
    LAYA_REQUIRE(a.max_len >= 0 && a.nseg >= 0, "attention: negative size");
    LAYA_REQUIRE(a.heads <= 65535 && a.nseg <= 65535, "attention: too many heads or segments for one launch");
    LAYA_REQUIRE(!a.blocks || (a.n_blocks > 0 && (long)a.n_blocks * a.heads < (1L << 31) &&
                               (a.max_len + BLOCK_ROWS - 1) / BLOCK_ROWS <= 65536),
                 "attention: bad block list");
    LAYA_REQUIRE(a.p_drop >= 0.0f && a.p_drop < 1.0f, "attention: dropout must be in [0, 1)");
    LAYA_REQUIRE(a.cos_table == nullptr || a.positions >= a.max_len, "attention: rotary table shorter than max_len");
    // The split-product kernels address a segment's rows through 32-bit buffer offsets.
    LAYA_REQUIRE(((long)a.max_len + BLOCK_ROWS) * 3L * a.hidden * 4L < (1L << 31),
                 "attention: a segment's qkv rows exceed 2 GiB");
}

// Attention takes split products (fp32 results) unless the context asked for the fp32 matrix cores; the
// bf16 product policies leave attention in fp32 arithmetic too.
bool split_attention(const laya_ctx* ctx) { return (ctx->matmul_split | ctx->matmul_bf16) != 0; }

// The two-piece form's scale input: qkv's magnitude (measured into the context's words unless the caller
// keeps it).
void pair_inputs(laya_ctx* ctx, const AttentionArgs& a, const float* qkv, AmaxRef r_qkv, Params& p) {
    LAYA_REQUIRE(a.rows >= 0, "attention: row count needed to measure qkv");
    p.amax_qkv = operand_amax_ref(ctx, qkv == a.qkv ? r_qkv : AmaxRef{}, 3, qkv, a.rows, 3 * a.hidden, 3L * a.hidden);
}

}  // namespace

void attention_fwd(laya_ctx* ctx, const AttentionArgs& a, float* context, float* lse, __bf16* context16,
                   unsigned* amax, AmaxRef amax_qkv) {
    check_args(a);
    if (a.nseg == 0 || a.max_len == 0) return;
    Params p = make_params(a);
    const bool split = a.head_dim == 64 && split_attention(ctx);
    const bool pair = split && ctx->attention_pair;
    // A rotated copy folds its own magnitude in as it is written (no pass to measure it).
    unsigned* rot_word = pair && a.cos_table && !a.rotated ? operand_ring_word(ctx) : nullptr;
    p.qkv = rotated_qkv(ctx, a, rot_word);
    p.context = context;
    p.lse = lse;
    p.amax = amax;
    const dim3 grid = block_grid(a);
    p.context16 = split ? context16 : nullptr;
    if (pair && rot_word)
        p.amax_qkv = rot_word;
    else if (pair)
        pair_inputs(ctx, a, p.qkv, amax_qkv, p);
    {
        ProfileScope scope(ctx, pair ? "attention_fwd_h2" : split ? "attention_fwd_x6" : "attention_fwd",
                           4.0 * a.hidden * a.keys, 0.0);
        if (pair && p.p_drop > 0.0f)
            LAYA_LAUNCH((attn_fwd_x6_kernel<64, true, 2>), grid, dim3(THREADS), 0, ctx->stream, p);
        else if (pair)
            LAYA_LAUNCH((attn_fwd_x6_kernel<64, false, 2>), grid, dim3(THREADS), 0, ctx->stream, p);
        else if (split && p.p_drop > 0.0f)
            LAYA_LAUNCH((attn_fwd_x6_kernel<64, true>), grid, dim3(THREADS), 0, ctx->stream, p);
        else if (split)
            LAYA_LAUNCH((attn_fwd_x6_kernel<64, false>), grid, dim3(THREADS), 0, ctx->stream, p);
        else if (a.head_dim == 64)
            LAYA_LAUNCH(attn_fwd_kernel<64>, grid, dim3(THREADS), 0, ctx->stream, p);
        else
            LAYA_LAUNCH(attn_fwd_kernel<32>, grid, dim3(THREADS), 0, ctx->stream, p);
        check_launch("attn_fwd_kernel");
    }
    if (context16 && !split) {
        LAYA_REQUIRE(a.rows >= 0, "attention: row count needed for the bf16 copy of the context");
        to_bf16(ctx, context, (size_t)a.rows * a.hidden, context16);
    }
}

void attention_bwd(laya_ctx* ctx, const AttentionArgs& a, int rows, const float* context, const float* lse,
                   const float* dcontext, float* dqkv, unsigned* amax, AmaxRef amax_qkv, AmaxRef amax_do) {
    check_args(a);
    if (a.nseg == 0 || a.max_len == 0 || rows == 0) return;
    Params p = make_params(a);
    p.amax = amax;
    AttentionArgs ar = a;
    if (ar.rows < 0) ar.rows = rows;
    const bool pair = a.head_dim == 64 && split_attention(ctx) && ctx->attention_pair;
    unsigned* rot_word = pair && a.cos_table && !a.rotated ? operand_ring_word(ctx) : nullptr;
    p.qkv = rotated_qkv(ctx, ar, rot_word);
    p.lse = const_cast<float*>(lse);
    p.dcontext = dcontext;
    p.dqkv = dqkv;
    float* dots = static_cast<float*>(ctx->workspace(3, sizeof(float) * (size_t)rows * a.heads));
    p.dots = dots;
    const long total = (long)rows * a.hidden;
    const unsigned dot_blocks = (unsigned)((total + THREADS - 1) / THREADS);
    const dim3 grid = block_grid(a);
    // Model flops of the backward, 8·d·Σkeys, split as the kernels do the work: dK/dV (4 products of
    // which 2 recompute the forward's) and dQ (3 products, 2 recomputed).
    const double fb = 2.0 * a.hidden * a.keys;
    if (pair) {
        p.context = const_cast<float*>(context);
        if (rot_word)
            p.amax_qkv = rot_word;
        else
            pair_inputs(ctx, ar, p.qkv, amax_qkv, p);
        p.amax_do = operand_amax_ref(ctx, amax_do, 4, dcontext, rows, a.hidden, a.hidden);
        {
            // dQ first: it forms each row's Σ dO·O and writes it for dK/dV.
            ProfileScope scope(ctx, "attention_bwd_dq_h2", 2.0 * fb, 0.0);
            if (p.p_drop > 0.0f)
                LAYA_LAUNCH((attn_bwd_dq_x6_kernel<64, true, 2>), grid, dim3(THREADS), 0, ctx->stream, p);
            else
                LAYA_LAUNCH((attn_bwd_dq_x6_kernel<64, false, 2>), grid, dim3(THREADS), 0, ctx->stream, p);
            check_launch("attn_bwd_dq_x6_kernel");
        }
        ProfileScope scope(ctx, "attention_bwd_dkv_h2", 2.0 * fb, 0.0);
        if (p.p_drop > 0.0f)
            LAYA_LAUNCH((attn_bwd_dkv_x6_kernel<64, true, 2>), grid, dim3(THREADS), 0, ctx->stream, p);
        else
            LAYA_LAUNCH((attn_bwd_dkv_x6_kernel<64, false, 2>), grid, dim3(THREADS), 0, ctx->stream, p);
        check_launch("attn_bwd_dkv_x6_kernel");
        return;
    }
    if (a.head_dim == 64 && split_attention(ctx)) {
        p.context = const_cast<float*>(context);
        {
            // dQ first: it forms each row's Σ dO·O and writes it for dK/dV.
            ProfileScope scope(ctx, "attention_bwd_dq_x6", 2.0 * fb, 0.0);
            if (p.p_drop > 0.0f)
                LAYA_LAUNCH((attn_bwd_dq_x6_kernel<64, true>), grid, dim3(THREADS), 0, ctx->stream, p);
            else
                LAYA_LAUNCH((attn_bwd_dq_x6_kernel<64, false>), grid, dim3(THREADS), 0, ctx->stream, p);
            check_launch("attn_bwd_dq_x6_kernel");
        }
        ProfileScope scope(ctx, "attention_bwd_dkv_x6", 2.0 * fb, 0.0);
        if (p.p_drop > 0.0f)
            LAYA_LAUNCH((attn_bwd_dkv_x6_kernel<64, true>), grid, dim3(THREADS), 0, ctx->stream, p);
        else
            LAYA_LAUNCH((attn_bwd_dkv_x6_kernel<64, false>), grid, dim3(THREADS), 0, ctx->stream, p);
        check_launch("attn_bwd_dkv_x6_kernel");
        return;
    }
    {
        ProfileScope scope(ctx, "attention_bwd_dots", 0.0, 8.0 * total);
        if (a.head_dim == 64)
            LAYA_LAUNCH(attn_dot_kernel<64>, dim3(dot_blocks), dim3(THREADS), 0, ctx->stream, dcontext, context,
                               rows, a.hidden, a.heads, dots);
        else
            LAYA_LAUNCH(attn_dot_kernel<32>, dim3(dot_blocks), dim3(THREADS), 0, ctx->stream, dcontext, context,
                               rows, a.hidden, a.heads, dots);
        check_launch("attn_dot_kernel");
    }
    {
        ProfileScope scope(ctx, "attention_bwd_dkv", 2.0 * fb, 0.0);
        if (a.head_dim == 64)
            LAYA_LAUNCH(attn_bwd_dkv_kernel<64>, grid, dim3(THREADS), 0, ctx->stream, p);
        else
            LAYA_LAUNCH(attn_bwd_dkv_kernel<32>, grid, dim3(THREADS), 0, ctx->stream, p);
        check_launch("attn_bwd_dkv_kernel");
    }
    {
        ProfileScope scope(ctx, "attention_bwd_dq", 2.0 * fb, 0.0);
        if (a.head_dim == 64)
            LAYA_LAUNCH(attn_bwd_dq_kernel<64>, grid, dim3(THREADS), 0, ctx->stream, p);
        else
            LAYA_LAUNCH(attn_bwd_dq_kernel<32>, grid, dim3(THREADS), 0, ctx->stream, p);
        check_launch("attn_bwd_dq_kernel");
    }
}

}  // namespace laya
