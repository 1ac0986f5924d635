// fp32 GEMM on CDNA4 matrix cores for the three products of backpropagation.
//
// Replaces the reference's panel GEMM (src/StructuredDecisions.Base/Numerics/PackedMatrix.cs:109-428)
// and the transposes/copies LinearBackward wraps around it (Ops.cs:47-61): each layout reads its
// operands in place, so no packed or transposed copy of a weight or activation is ever made.
//
//   NT  C = A·Bᵀ   y  = x·Wᵀ      A k-contiguous, B k-contiguous
//   NN  C = A·B    dx = dy·W      A k-contiguous, B n-contiguous
//   TN  C = Aᵀ·B   dW += dyᵀ·x    A m-contiguous, B n-contiguous  (K = tokens, split-K)
//
// Block tile 128×128×32, 256 threads = 4 waves in 2×2, each wave 64×64 = 2×2 tiles of
// v_mfma_f32_32x32x2_f32. Operand tiles are staged through LDS in their global orientation
// (k-contiguous rows read as b128 fragments of 4 k; mn-contiguous rows read as b64 pairs of
// neighbouring rows/columns, which then land in two interleaved MFMA tiles), double-buffered with a
// register prefetch of the next K tile. Split-K partials are reduced in a fixed order, so results
// never depend on timing.
//
// Two kernel families. The main one is branch-free in its K loop: rows and columns past the matrix
// edge are clamped to the last valid one (their products only reach outputs that are never stored),
// and a ragged final K tile is peeled off the loop and zero-filled with selects. It needs float4
// access (leading dimensions and the contiguous extent of each operand a multiple of 4, 16-byte
// aligned bases, fewer than 2³¹ elements per operand). Every other shape takes the generic kernel,
// which tests each element. Keeping each kernel to one loop and one store path matters: the same
// loop in a kernel that also carries unused boundary code and runtime epilogue branches measured a
// fifth slower on short-K products.
#include "common.hpp"
#include "elementwise.hpp"
#include "split.hpp"

namespace laya {
namespace {

constexpr int BM = 128, BN = 128, BK = 32, THREADS = 256;
constexpr int KPAD = BK + 4;   // row stride of a k-contiguous tile [mn][k]: b128 reads hit all 64 banks once
constexpr int MNPAD = BM + 8;  // row stride of an mn-contiguous tile [k][mn]: rows k and k+4 land 32 banks apart
constexpr int STAGE = BM * KPAD;  // ≥ BK * MNPAD

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

// Epilogue modes, fixed at compile time so each kernel carries only its own store path.
enum : int { STORE = 0, ACCUMULATE = 1, PARTIAL = 2, STORE_ROPE = 3, STORE_GEGLU = 4 };

struct GemmParams {
    const float* A;
    const float* B;
    float* C;
    const float* bias;
    const float* R;
    long lda, ldb, ldc, ldr;
    int M, N, K;
    int tiles_m, tiles_n, splits, k_per_split;
    int mode;  // STORE, ACCUMULATE in place (one writer per element), PARTIAL split-K slices, STORE_ROPE
    int vec_a, vec_b;
    // STORE_ROPE: RoPE on output columns [0, rope_cols) in heads of 64, position rope_pos[row]; tables
    // [positions][32].
    const int* rope_pos;
    const float* rope_cos;
    const float* rope_sin;
    int rope_cols;
    // Optional bf16 copies of A and B (same leading dimensions), rounded to nearest even as the kernels
    // would round A and B: a bf16 product whose kernel can read them streams half the bytes and skips the
    // conversion; the result is the same.
    const __bf16* A16;
    const __bf16* B16;
    // Two-piece fp16 products: the bit patterns of max|A| and max|B| (device words, written by
    // absmax_kernel before the product), from which each kernel takes its operands' power-of-two scales.
    const unsigned* amax_a;
    const unsigned* amax_b;
    // Optional magnitude word group of C, folded in by the two-piece kernels' epilogues (max|stored value|).
    unsigned* amax_c;
    // Two-piece NT products: B's values are bf16 values (fp32 holding a bf16), so sb·B is one fp16 piece
    // (see split1h_4) and the kernels that honour it skip B's low plane and its products.
    int b_one;
    // STORE_GEGLU (the 256-wide NT kernels): C is GeGLU's input [M, 2·inter] (both halves stored, from B's
    // rows taken in pairs, geglu_b_row), act [M, inter] receives gelu(first half)·(second half) beside it,
    // act16 (optional) its bf16 copy, amax_act (optional) its magnitude word group.
    float* act;
    __bf16* act16;
    unsigned* amax_act;
    int inter;
};

// ------------------------------------------------------------------------------ shared pieces

template <bool KCONTIG>
__device__ __forceinline__ void store_tile(float* lds, const f32x4 (&reg)[4], int tid) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        int idx = tid + THREADS * i;
        if (KCONTIG)
            *reinterpret_cast<f32x4*>(lds + (idx >> 3) * KPAD + ((idx & 7) << 2)) = reg[i];
        else
            *reinterpret_cast<f32x4*>(lds + (idx >> 5) * MNPAD + ((idx & 31) << 2)) = reg[i];
    }
}

// XCD-aware order: workgroups are dealt round-robin to the 8 XCDs, so give each XCD a contiguous run
// of logical tiles (n fastest); tiles sharing an A row-panel then share one XCD's L2.
__device__ __forceinline__ int xcd_logical_block() {
    const int nblocks = gridDim.x, bid = blockIdx.x;
    const int xcd = bid & 7, local = bid >> 3, per = nblocks >> 3, rem = nblocks & 7;
    return (xcd < rem ? xcd * (per + 1) : rem * (per + 1) + (xcd - rem) * per) + local;
}

// Where one logical block works: its output tile and its K range.
struct TileCoord {
    int split, t, m0, n0, kb, ke;
};

__device__ __forceinline__ TileCoord tile_coord(const GemmParams& p, int logical) {
    TileCoord c;
    const int tiles = p.tiles_m * p.tiles_n;
    c.split = logical / tiles;
    c.t = logical - c.split * tiles;
    const int tile_m = c.t / p.tiles_n;
    c.m0 = tile_m * BM;
    c.n0 = (c.t - tile_m * p.tiles_n) * BN;
    c.kb = c.split * p.k_per_split;
    c.ke = min(p.K, c.kb + p.k_per_split);
    return c;
}

typedef float f32x2 __attribute__((ext_vector_type(2)));

// 64 MFMAs of one wave over one LDS stage (K = 32), in steps of 8 k. Within a step lane half h holds
// k = 8s + 4h + c for c = 0..3 and MFMA c pairs the two halves, so a k-contiguous operand gives each
// lane one b128 read per 32-row tile. An mn-contiguous operand is read as b64 pairs (mn = 2·lane,
// 2·lane + 1) of one k row, one read per c: its two MFMA tiles are the even and the odd rows (or
// columns) of the wave's 64, which halves the LDS reads of the per-element b32 form.
template <bool AK, bool BKC>
__device__ __forceinline__ void mma_stage(const float* As, const float* Bs, f32x16 (&acc)[2][2], int wm, int wn,
                                          int lr, int kh) {
#pragma unroll
    for (int kk = 0; kk < BK; kk += 8) {
        const int k = kk + kh;
        float a[4][2], b[4][2];  // [c][tile]
        if (AK) {
            const f32x4 a0 = *reinterpret_cast<const f32x4*>(As + (wm * 64 + lr) * KPAD + k);
            const f32x4 a1 = *reinterpret_cast<const f32x4*>(As + (wm * 64 + 32 + lr) * KPAD + k);
#pragma unroll
            for (int cc = 0; cc < 4; ++cc) {
                a[cc][0] = a0[cc];
                a[cc][1] = a1[cc];
            }
        } else {
#pragma unroll
            for (int cc = 0; cc < 4; ++cc) {
                const f32x2 v = *reinterpret_cast<const f32x2*>(As + (k + cc) * MNPAD + wm * 64 + 2 * lr);
                a[cc][0] = v[0];
                a[cc][1] = v[1];
            }
        }
        if (BKC) {
            const f32x4 b0 = *reinterpret_cast<const f32x4*>(Bs + (wn * 64 + lr) * KPAD + k);
            const f32x4 b1 = *reinterpret_cast<const f32x4*>(Bs + (wn * 64 + 32 + lr) * KPAD + k);
#pragma unroll
            for (int cc = 0; cc < 4; ++cc) {
                b[cc][0] = b0[cc];
                b[cc][1] = b1[cc];
            }
        } else {
#pragma unroll
            for (int cc = 0; cc < 4; ++cc) {
                const f32x2 v = *reinterpret_cast<const f32x2*>(Bs + (k + cc) * MNPAD + wn * 64 + 2 * lr);
                b[cc][0] = v[0];
                b[cc][1] = v[1];
            }
        }
#pragma unroll
        for (int cc = 0; cc < 4; ++cc)
#pragma unroll
            for (int i = 0; i < 2; ++i)
#pragma unroll
                for (int j = 0; j < 2; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(a[cc][i], b[cc][j], acc[i][j], 0, 0, 0);
    }
}

// Writes the wave's 64×64 accumulators. In a 32×32 accumulator tile the lane holds column lane%32 and
// rows q = 8(r/4) + 4(lane/32) + r%4; the tile maps to the wave's rows as 32i + q (k-contiguous A) or
// 2q + i (mn-contiguous A), and to its columns as 32j + lane%32 or 2·(lane%32) + j. Every element sits
// at a fixed 32-bit offset from one base pointer. With an mn-contiguous B and VEC2, a lane's two
// column tiles are adjacent columns and go out as one float2. GUARD drops elements outside the
// matrix; RES adds the residual R (STORE only).
//
// Whatever the epilogue reads (the residual, or C itself when accumulating) is loaded for all of the
// lane's elements before the first store: the memory counter the wait instructions use also counts
// stores, so a load issued after stores waits for all of them, and interleaving load-add-store per
// element would serialise the epilogue. Each element is read and written by its own lane only, so
// this order is also right when R is C.
// AMX: also fold max|stored value| (amax_bits) into *am.
template <bool AK, bool BKC, int MODE, bool RES, bool GUARD, bool VEC2, int NI, bool AMX = false>
__device__ __forceinline__ void store_acc(const GemmParams& p, const TileCoord& c, const f32x16 (&acc)[NI][2], int wm,
                                          int wn, int lr, int kh, unsigned* am = nullptr) {
    static_assert(AK || NI == 2, "three row groups are a k-contiguous layout");
    auto rowoff = [&](int i, int r) {
        const int q = 8 * (r >> 2) + kh + (r & 3);
        return AK ? wm * 64 + 32 * i + q : wm * 64 + 2 * q + i;
    };
    auto coloff = [&](int j) { return BKC ? wn * 64 + 32 * j + lr : wn * 64 + 2 * lr + j; };
    const int ldo = MODE == PARTIAL ? p.N : (int)p.ldc;
    const int ldr = RES ? (int)p.ldr : 0;
    float* base = (MODE == PARTIAL ? p.C + (long)c.split * p.M * p.N : p.C) + (long)c.m0 * ldo + c.n0;
    const float* rbase = RES ? p.R + (long)c.m0 * p.ldr + c.n0 : nullptr;
    constexpr bool READS = RES || MODE == ACCUMULATE;
    const float* src = MODE == ACCUMULATE ? base : rbase;  // what the epilogue adds besides bias
    const int lds_ = MODE == ACCUMULATE ? ldo : ldr;
    float bj[2] = {0.0f, 0.0f};
    if ((MODE == STORE || MODE == STORE_ROPE) && p.bias) {
#pragma unroll
        for (int j = 0; j < 2; ++j)
            if (!GUARD || c.n0 + coloff(j) < p.N) bj[j] = p.bias[c.n0 + coloff(j)];
    }
    if constexpr (MODE == STORE_ROPE) {
        // Row-major NT output: the wave's 64 columns are one head, and a lane's column tiles j = 0, 1
        // are the rotation partners d = lane%32 and d + 32 of every row it holds.
        static_assert(AK && BKC, "STORE_ROPE is an NT epilogue");
        const bool rot = c.n0 + wn * 64 < p.rope_cols;  // wave-uniform
#pragma unroll
        for (int i = 0; i < NI; ++i) {
            float cs[16], sn[16];
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                cs[r] = 1.0f;
                sn[r] = 0.0f;
            }
            if (rot) {
                int pos[16];
#pragma unroll
                for (int r = 0; r < 16; ++r)
                    pos[r] = (!GUARD || c.m0 + rowoff(i, r) < p.M) ? p.rope_pos[c.m0 + rowoff(i, r)] : 0;
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    cs[r] = p.rope_cos[pos[r] * 32 + lr];
                    sn[r] = p.rope_sin[pos[r] * 32 + lr];
                }
            }
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int row = rowoff(i, r);
                if (GUARD && c.m0 + row >= p.M) continue;
                const float a = acc[i][0][r] + bj[0], b = acc[i][1][r] + bj[1];
                const float v0 = a * cs[r] - b * sn[r], v1 = b * cs[r] + a * sn[r];
                if (!GUARD || c.n0 + coloff(0) < p.N) {
                    base[row * ldo + coloff(0)] = v0;
                    if constexpr (AMX) *am = max(*am, amax_bits(v0));
                }
                if (!GUARD || c.n0 + coloff(1) < p.N) {
                    base[row * ldo + coloff(1)] = v1;
                    if constexpr (AMX) *am = max(*am, amax_bits(v1));
                }
            }
        }
        return;
    }
    if (VEC2 && !BKC) {
        const int col = coloff(0);
        auto inside = [&](int i, int r) { return !GUARD || (c.m0 + rowoff(i, r) < p.M && c.n0 + col < p.N); };
#pragma unroll
        for (int i = 0; i < NI; ++i) {  // two halves bound the registers the reads hold
            f32x2 add[16];
            if (READS) {
#pragma unroll
                for (int r = 0; r < 16; ++r)
                    add[r] = inside(i, r) ? *reinterpret_cast<const f32x2*>(src + rowoff(i, r) * lds_ + col)
                                          : f32x2{0.0f, 0.0f};
            }
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                if (!inside(i, r)) continue;
                f32x2 v = {acc[i][0][r] + bj[0], acc[i][1][r] + bj[1]};
                if (READS) v += add[r];
                *reinterpret_cast<f32x2*>(base + rowoff(i, r) * ldo + col) = v;
                if constexpr (AMX) *am = max(*am, max(amax_bits(v[0]), amax_bits(v[1])));
            }
        }
        return;
    }
    auto inside = [&](int i, int j, int r) {
        return !GUARD || (c.m0 + rowoff(i, r) < p.M && c.n0 + coloff(j) < p.N);
    };
#pragma unroll
    for (int i = 0; i < NI; ++i) {
        float add[2][16];
        if (READS) {
#pragma unroll
            for (int j = 0; j < 2; ++j)
#pragma unroll
                for (int r = 0; r < 16; ++r)
                    add[j][r] = inside(i, j, r) ? src[rowoff(i, r) * lds_ + coloff(j)] : 0.0f;
        }
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                if (!inside(i, j, r)) continue;
                float v = acc[i][j][r] + bj[j];
                if (READS) v += add[j][r];
                base[rowoff(i, r) * ldo + coloff(j)] = v;
                if constexpr (AMX) *am = max(*am, amax_bits(v));
            }
    }
}

// ------------------------------------------------------------------------------ main kernel

// One thread's share of a 128×32 operand tile: four float4 loads at offsets fixed for the whole K loop
// except for the K position. Rows (k-contiguous) or columns (mn-contiguous) past the edge are clamped.
template <bool KCONTIG>
struct Loader {
    const float* src;
    unsigned off[4];  // k-contiguous: row offsets + kq; mn-contiguous: column offset
    unsigned ld;
    int kq;           // k-contiguous: this thread's k within the tile; mn-contiguous: its first k row

    __device__ __forceinline__ Loader(const float* s, long ldl, int mn0, int MN, int tid) : src(s), ld((unsigned)ldl) {
        if (KCONTIG) {
            kq = (tid & 7) << 2;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int row = min(mn0 + (tid >> 3) + 32 * i, MN - 1);
                off[i] = (unsigned)row * ld + kq;
            }
        } else {
            kq = tid >> 5;
            const int col = min(mn0 + ((tid & 31) << 2), MN - 4);
#pragma unroll
            for (int i = 0; i < 4; ++i) off[i] = (unsigned)col;
        }
    }

    // A K tile that lies entirely inside [kb, ke).
    __device__ __forceinline__ void full(int k0, f32x4 (&reg)[4]) const {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const unsigned o = KCONTIG ? off[i] + (unsigned)k0 : off[i] + (unsigned)(k0 + kq + 8 * i) * ld;
            reg[i] = *reinterpret_cast<const f32x4*>(src + o);
        }
    }

    // The ragged last K tile: positions at or past `kend` read an in-bounds neighbour and become 0.
    __device__ __forceinline__ void tail(int k0, int kend, f32x4 (&reg)[4]) const {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            if (KCONTIG) {
                const int k = k0 + kq;  // kend is a multiple of 4, so k < kend covers k..k+3
                const f32x4 v = *reinterpret_cast<const f32x4*>(src + off[i] - kq + (unsigned)min(k, kend - 4));
                reg[i] = k < kend ? v : f32x4{0, 0, 0, 0};
            } else {
                const int k = k0 + kq + 8 * i;
                const f32x4 v = *reinterpret_cast<const f32x4*>(src + off[i] + (unsigned)min(k, kend - 1) * ld);
                reg[i] = k < kend ? v : f32x4{0, 0, 0, 0};
            }
        }
    }
};

// The thread index passed through an empty asm statement. Addresses derived from it then cannot be
// hoisted out of a loop over tiles (the persistent kernels), which would keep dozens of per-lane
// values live for the whole kernel and push it into spills.
__device__ __forceinline__ int opaque_tid() {
    int t = threadIdx.x;
    asm volatile("" : "+v"(t));
    return t;
}

// The 128×128 accumulators of one output tile over the K range [c.kb, c.ke) of C = op(A)·op(B).
//
// Each tile walks its full K tiles starting at its own offset (rotation by the tile index), then the
// ragged tail if any. Operand rows are often a multiple of 1 KiB apart (768 or 2304 floats), so blocks
// that all fetched the same K columns at once would hit the same few memory channels; staggered
// starts spread them. The sum order is fixed per tile, so results stay deterministic. Ends with a
// barrier, so the caller may start another tile on the same LDS.
template <bool AK, bool BKC, int NSTAGE = 2>
__device__ __forceinline__ void tile_mma(const GemmParams& p, const TileCoord& c, float (*smem)[2][STAGE],
                                         f32x16 (&acc)[2][2]) {
    const int len = max(0, c.ke - c.kb);
    const int nfull = len / BK, ntiles = nfull + (len % BK != 0 ? 1 : 0);
    const int rot = nfull > 0 ? c.t % nfull : 0;

    const int tid = opaque_tid(), lane = tid & 63, wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    const int lr = lane & 31, kh = (lane >> 5) << 2;

    const Loader<AK> la(p.A, p.lda, c.m0, p.M, tid);
    const Loader<BKC> lb(p.B, p.ldb, c.n0, p.N, tid);
    f32x4 ra[4], rb[4];
    auto fetch = [&](int j) {  // block-uniform branch
        if (j < nfull) {
            int q = j + rot;
            if (q >= nfull) q -= nfull;
            la.full(c.kb + q * BK, ra);
            lb.full(c.kb + q * BK, rb);
        } else {
            la.tail(c.kb + nfull * BK, c.ke, ra);
            lb.tail(c.kb + nfull * BK, c.ke, rb);
        }
    };

#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) acc[i][j] = f32x16{};

    if constexpr (NSTAGE == 1) {
        // One LDS stage (half the LDS, so three workgroups fit on a CU): the next K tile waits in registers
        // while this one is multiplied, and is stored once every wave has finished reading the stage.
        if (ntiles > 0) fetch(0);
        for (int j = 0; j < ntiles; ++j) {
            __syncthreads();
            store_tile<AK>(smem[0][0], ra, tid);
            store_tile<BKC>(smem[0][1], rb, tid);
            __syncthreads();
            if (j + 1 < ntiles) fetch(j + 1);
            mma_stage<AK, BKC>(smem[0][0], smem[0][1], acc, wm, wn, lr, kh);
        }
        __syncthreads();
        return;
    }
    if (ntiles > 0) {
        fetch(0);
        store_tile<AK>(smem[0][0], ra, tid);
        store_tile<BKC>(smem[0][1], rb, tid);
    }
    __syncthreads();
    for (int j = 0; j < ntiles; ++j) {
        const int cur = j & 1;
        if (j + 1 < ntiles) fetch(j + 1);
        mma_stage<AK, BKC>(smem[cur][0], smem[cur][1], acc, wm, wn, lr, kh);
        if (j + 1 < ntiles) {
            store_tile<AK>(smem[cur ^ 1][0], ra, tid);
            store_tile<BKC>(smem[cur ^ 1][1], rb, tid);
        }
        __syncthreads();
    }
}

// ------------------------------------------------------------------------------ bf16 main loop
//
// The same tiles with bf16 operands on v_mfma_f32_32x32x16_bf16 and fp32 accumulation. Operands are read
// as fp32 (activations, and the fp32 master weights), rounded to bf16 (nearest even, the hardware
// convert) on their way into LDS, and laid out there as [mn][k] rows of 32 k with an 80-byte stride
// whatever their global orientation: every MFMA fragment (8 consecutive k of one row) is then one b128
// read, and 16 consecutive rows fall on distinct bank groups for both the fragment reads and the row
// writes. The accumulators come out in the fp32 loop's layout for k-contiguous operands, so the same
// epilogues store them.
constexpr int KPADH = BK + 8;        // bf16 row stride of an [mn][k] tile
constexpr int STAGE_H = BM * KPADH;  // bf16 elements per operand tile

// One thread's share of a 128×32 bf16 operand tile, read as fp32, in one of three forms:
//  KVEC     k-contiguous with float4 access: the fp32 loader's four float4 (rows (tid >> 3) + 32i,
//           k = 4(tid & 7)), coalesced along k;
//  KSCALAR  k-contiguous, any extent or alignment: one tile row per thread (tid & 127) and 16
//           consecutive k (16·(tid >> 7) …), one element at a time;
//  MNSCALAR mn-contiguous: the same row/k split, one element at a time, coalesced along mn across the
//           wave.
// Rows past the edge are clamped; positions at or past a ragged K end read an in-bounds neighbour and
// become 0.
enum : int { KVEC = 0, KSCALAR = 1, MNSCALAR = 2 };

template <int KIND>
struct OperandH;

template <>
struct OperandH<KVEC> {
    Loader<true> ld;
    f32x4 reg[4];
    __device__ __forceinline__ OperandH(const float* s, long ldl, int mn0, int MN, int tid) : ld(s, ldl, mn0, MN, tid) {}
    __device__ __forceinline__ void full(int k0) { ld.full(k0, reg); }
    __device__ __forceinline__ void tail(int k0, int kend) { ld.tail(k0, kend, reg); }
    __device__ __forceinline__ void store(__bf16* lds, int tid) const {
#pragma unroll
        for (int i = 0; i < 4; ++i)
            *reinterpret_cast<bf16x4*>(lds + ((tid >> 3) + 32 * i) * KPADH + ((tid & 7) << 2)) =
                __builtin_convertvector(reg[i], bf16x4);
    }
};

// The two one-element-at-a-time forms: element k of this thread's row at src[base + k·kstride].
template <int KIND>
struct OperandH {
    static_assert(KIND == KSCALAR || KIND == MNSCALAR, "operand form");
    const float* src;
    unsigned base, kstride;
    int kq;
    float v[16];
    __device__ __forceinline__ OperandH(const float* s, long ldl, int mn0, int MN, int tid) : src(s), kq((tid >> 7) << 4) {
        const unsigned row = (unsigned)min(mn0 + (tid & 127), MN - 1);
        base = KIND == KSCALAR ? row * (unsigned)ldl : row;
        kstride = KIND == KSCALAR ? 1u : (unsigned)ldl;
    }
    __device__ __forceinline__ void full(int k0) {
#pragma unroll
        for (int e = 0; e < 16; ++e) v[e] = src[base + (unsigned)(k0 + kq + e) * kstride];
    }
    __device__ __forceinline__ void tail(int k0, int kend) {
#pragma unroll
        for (int e = 0; e < 16; ++e) {
            const int k = k0 + kq + e;
            const float x = src[base + (unsigned)min(k, kend - 1) * kstride];
            v[e] = k < kend ? x : 0.0f;
        }
    }
    __device__ __forceinline__ void store(__bf16* lds, int tid) const {
        bf16x8 h0, h1;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            h0[e] = (__bf16)v[e];
            h1[e] = (__bf16)v[8 + e];
        }
        __bf16* row = lds + (tid & 127) * KPADH + kq;
        *reinterpret_cast<bf16x8*>(row) = h0;
        *reinterpret_cast<bf16x8*>(row + 8) = h1;
    }
};

// 8 MFMAs of one wave over one LDS stage (K = 32): two steps of 16 k; lane half h holds k = 16s + 8h … + 7
// of row lane % 32 for both operands.
__device__ __forceinline__ void mma_stage_h(const __bf16* As, const __bf16* Bs, f32x16 (&acc)[2][2], int wm, int wn,
                                            int lr, int half) {
#pragma unroll
    for (int ks = 0; ks < BK; ks += 16) {
        const int k = ks + 8 * half;
        bf16x8 a[2], b[2];
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            a[i] = *reinterpret_cast<const bf16x8*>(As + (wm * 64 + 32 * i + lr) * KPADH + k);
            b[i] = *reinterpret_cast<const bf16x8*>(Bs + (wn * 64 + 32 * i + lr) * KPADH + k);
        }
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
            for (int j = 0; j < 2; ++j) acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[i], b[j], acc[i][j], 0, 0, 0);
    }
}

// tile_mma with bf16 operands: the same K order (rotation, peeled tail), so the result is deterministic.
template <int AOP, int BOP>
__device__ __forceinline__ void tile_mma_h(const GemmParams& p, const TileCoord& c, __bf16 (*smem)[2][STAGE_H],
                                           f32x16 (&acc)[2][2]) {
    const int len = max(0, c.ke - c.kb);
    const int nfull = len / BK, ntiles = nfull + (len % BK != 0 ? 1 : 0);
    const int rot = nfull > 0 ? c.t % nfull : 0;

    const int tid = opaque_tid(), lane = tid & 63, wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    const int lr = lane & 31, half = lane >> 5;

    OperandH<AOP> a(p.A, p.lda, c.m0, p.M, tid);
    OperandH<BOP> b(p.B, p.ldb, c.n0, p.N, tid);
    auto fetch = [&](int j) {  // block-uniform branch
        if (j < nfull) {
            int q = j + rot;
            if (q >= nfull) q -= nfull;
            a.full(c.kb + q * BK);
            b.full(c.kb + q * BK);
        } else {
            a.tail(c.kb + nfull * BK, c.ke);
            b.tail(c.kb + nfull * BK, c.ke);
        }
    };

#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) acc[i][j] = f32x16{};

    if (ntiles > 0) {
        fetch(0);
        a.store(smem[0][0], tid);
        b.store(smem[0][1], tid);
    }
    __syncthreads();
    for (int j = 0; j < ntiles; ++j) {
        const int cur = j & 1;
        if (j + 1 < ntiles) fetch(j + 1);
        mma_stage_h(smem[cur][0], smem[cur][1], acc, wm, wn, lr, half);
        if (j + 1 < ntiles) {
            a.store(smem[cur ^ 1][0], tid);
            b.store(smem[cur ^ 1][1], tid);
        }
        __syncthreads();
    }
}

// The epilogue of one tile: unguarded when the tile lies inside C.
template <bool AK, bool BKC, int MODE, bool RES>
__device__ __forceinline__ void tile_store(const GemmParams& p, const TileCoord& c, const f32x16 (&acc)[2][2]) {
    const int tid = opaque_tid(), lane = tid & 63, wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1, lr = lane & 31, kh = (lane >> 5) << 2;
    if (c.m0 + BM <= p.M && c.n0 + BN <= p.N)
        store_acc<AK, BKC, MODE, RES, false, true>(p, c, acc, wm, wn, lr, kh);
    else
        store_acc<AK, BKC, MODE, RES, true, true>(p, c, acc, wm, wn, lr, kh);
}

template <bool AK, bool BKC, int MODE, bool RES>
__global__ __launch_bounds__(THREADS, 2) void gemm_kernel(GemmParams p) {
    __shared__ __attribute__((aligned(16))) float smem[2][2][STAGE];
    const TileCoord c = tile_coord(p, xcd_logical_block());
    f32x16 acc[2][2];
    tile_mma<AK, BKC>(p, c, smem, acc);
    tile_store<AK, BKC, MODE, RES>(p, c, acc);
}

// The same product with one LDS stage, three workgroups per CU: for tile counts that would leave the
// last round of two-per-CU workgroups mostly empty (e.g. 654 tiles on 512 slots: one round instead of two).
template <bool AK, bool BKC, int MODE, bool RES>
__global__ __launch_bounds__(THREADS, 3) void gemm3_kernel(GemmParams p) {
    __shared__ __attribute__((aligned(16))) float smem[1][2][STAGE];
    const TileCoord c = tile_coord(p, xcd_logical_block());
    f32x16 acc[2][2];
    tile_mma<AK, BKC, 1>(p, c, smem, acc);
    tile_store<AK, BKC, MODE, RES>(p, c, acc);
}

// ------------------------------------------------------------------------------ fp32 from bf16 pieces
//
// fp32 products on the bf16 matrix cores. Every fp32 operand x is split exactly into three bf16 pieces,
// x = x1 + x2 + x3 (x1 = bf16(x) to nearest, x2 = bf16(x − x1), x3 = x − x1 − x2: 8 + 8 + 8 significand
// bits, each remainder exact in fp32), and a·b is accumulated in fp32 from the six piece products whose
// combined order is at most 2⁻¹⁶ of the product — a1b1, a1b2, a2b1, a1b3, a3b1, a2b2 (the three dropped
// ones are below 2⁻²⁴, under fp32 rounding). Each piece product is exact in the fp32 accumulator, so the
// result carries fp32 rounding only, like an fp32 product; the smallest terms are added first. Six
// v_mfma_f32_32x32x16_bf16 do the work of 32 fp32 v_mfma_f32_32x32x2_f32 in 192 against 512 cycles.
// The pieces are staged in LDS as three bf16 planes ([mn][k], the bf16 loop's layout) in one stage.
template <int KIND>
__device__ __forceinline__ void store_x3(const OperandH<KIND>& op, __bf16* lds0, __bf16* lds1, __bf16* lds2, int tid) {
    if constexpr (KIND == KVEC) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            bf16x4 h1, h2, h3;
            split3_4(op.reg[i], h1, h2, h3);
            const int o = ((tid >> 3) + 32 * i) * KPADH + ((tid & 7) << 2);
            *reinterpret_cast<bf16x4*>(lds0 + o) = h1;
            *reinterpret_cast<bf16x4*>(lds1 + o) = h2;
            *reinterpret_cast<bf16x4*>(lds2 + o) = h3;
        }
    } else {
        const int o = (tid & 127) * KPADH + op.kq;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            bf16x4 h1, h2, h3;
            split3_4(f32x4{op.v[4 * q], op.v[4 * q + 1], op.v[4 * q + 2], op.v[4 * q + 3]}, h1, h2, h3);
            *reinterpret_cast<bf16x4*>(lds0 + o + 4 * q) = h1;
            *reinterpret_cast<bf16x4*>(lds1 + o + 4 * q) = h2;
            *reinterpret_cast<bf16x4*>(lds2 + o + 4 * q) = h3;
        }
    }
}

// The two-piece form of store_x3: the two fp16 planes of sc·x (ONE: the hi plane only, for bf16-valued
// operands), in the same layout for every operand form.
template <bool ONE = false, int KIND>
__device__ __forceinline__ void store_x2(const OperandH<KIND>& op, __bf16* lds0, __bf16* lds1, int tid, float sc) {
    auto put = [&](int o, f32x4 x) {
        if constexpr (ONE) {
            *reinterpret_cast<f16x4*>(lds0 + o) = split1h_4(x, sc);
        } else {
            f16x4 hi, lo;
            split2h_4(x, sc, hi, lo);
            *reinterpret_cast<f16x4*>(lds0 + o) = hi;
            *reinterpret_cast<f16x4*>(lds1 + o) = lo;
        }
    };
    if constexpr (KIND == KVEC) {
#pragma unroll
        for (int i = 0; i < 4; ++i) put(((tid >> 3) + 32 * i) * KPADH + ((tid & 7) << 2), op.reg[i]);
    } else {
        const int o = (tid & 127) * KPADH + op.kq;
#pragma unroll
        for (int q = 0; q < 4; ++q)
            put(o + 4 * q, f32x4{op.v[4 * q], op.v[4 * q + 1], op.v[4 * q + 2], op.v[4 * q + 3]});
    }
}

// The two-piece form of mma_stage_x6: two fp16 planes, three products per block, the smallest first (B1: B
// in one piece, two products).
template <bool B1 = false>
__device__ __forceinline__ void mma_stage_x2(const __bf16* A, const __bf16* B, f32x16 (&acc)[2][2], int wm, int wn,
                                             int lr, int half) {
    constexpr int BP = B1 ? 1 : 2;
#pragma unroll
    for (int ks = 0; ks < BK; ks += 16) {
        const int k = ks + 8 * half;
        f16x8 a[2][2], b[2][2];
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
            for (int pl = 0; pl < 2; ++pl) {
                a[i][pl] = *reinterpret_cast<const f16x8*>(A + pl * STAGE_H + (wm * 64 + 32 * i + lr) * KPADH + k);
                if (pl < BP)
                    b[i][pl] = *reinterpret_cast<const f16x8*>(B + pl * STAGE_H + (wn * 64 + 32 * i + lr) * KPADH + k);
            }
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                f32x16 c = acc[i][j];
                c = __builtin_amdgcn_mfma_f32_32x32x16_f16(a[i][1], b[j][0], c, 0, 0, 0);
                if constexpr (!B1) c = __builtin_amdgcn_mfma_f32_32x32x16_f16(a[i][0], b[j][1], c, 0, 0, 0);
                c = __builtin_amdgcn_mfma_f32_32x32x16_f16(a[i][0], b[j][0], c, 0, 0, 0);
                acc[i][j] = c;
            }
    }
}

__device__ __forceinline__ void mma_stage_x6(const __bf16* A, const __bf16* B, f32x16 (&acc)[2][2], int wm, int wn,
                                             int lr, int half) {
#pragma unroll
    for (int ks = 0; ks < BK; ks += 16) {
        const int k = ks + 8 * half;
        bf16x8 a[2][3], b[2][3];
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
            for (int pl = 0; pl < 3; ++pl) {
                a[i][pl] = *reinterpret_cast<const bf16x8*>(A + pl * STAGE_H + (wm * 64 + 32 * i + lr) * KPADH + k);
                b[i][pl] = *reinterpret_cast<const bf16x8*>(B + pl * STAGE_H + (wn * 64 + 32 * i + lr) * KPADH + k);
            }
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                f32x16 c = acc[i][j];
                c = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[i][2], b[j][0], c, 0, 0, 0);
                c = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[i][0], b[j][2], c, 0, 0, 0);
                c = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[i][1], b[j][1], c, 0, 0, 0);
                c = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[i][1], b[j][0], c, 0, 0, 0);
                c = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[i][0], b[j][1], c, 0, 0, 0);
                c = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[i][0], b[j][0], c, 0, 0, 0);
                acc[i][j] = c;
            }
    }
}

// NP = 2 (float4 operands only): two-piece products with the operands' scales sa, sb (B1: B in one piece).
template <int AOP, int BOP, int NP = 3, bool B1 = false>
__device__ __forceinline__ void tile_mma_x6(const GemmParams& p, const TileCoord& c, __bf16 (*smem)[3 * STAGE_H],
                                            f32x16 (&acc)[2][2], float sa = 1.0f, float sb = 1.0f) {
    const int len = max(0, c.ke - c.kb);
    const int nfull = len / BK, ntiles = nfull + (len % BK != 0 ? 1 : 0);
    const int rot = nfull > 0 ? c.t % nfull : 0;
    const int tid = opaque_tid(), lane = tid & 63, wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    const int lr = lane & 31, half = lane >> 5;
    OperandH<AOP> a(p.A, p.lda, c.m0, p.M, tid);
    OperandH<BOP> b(p.B, p.ldb, c.n0, p.N, tid);
    auto fetch = [&](int j) {
        if (j < nfull) {
            int q = j + rot;
            if (q >= nfull) q -= nfull;
            a.full(c.kb + q * BK);
            b.full(c.kb + q * BK);
        } else {
            a.tail(c.kb + nfull * BK, c.ke);
            b.tail(c.kb + nfull * BK, c.ke);
        }
    };
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) acc[i][j] = f32x16{};
    if (ntiles > 0) fetch(0);
    for (int j = 0; j < ntiles; ++j) {
        __syncthreads();
        if constexpr (NP == 2) {
            store_x2(a, smem[0], smem[0] + STAGE_H, tid, sa);
            store_x2<B1>(b, smem[1], smem[1] + STAGE_H, tid, sb);
        } else {
            store_x3<AOP>(a, smem[0], smem[0] + STAGE_H, smem[0] + 2 * STAGE_H, tid);
            store_x3<BOP>(b, smem[1], smem[1] + STAGE_H, smem[1] + 2 * STAGE_H, tid);
        }
        __syncthreads();
        if (j + 1 < ntiles) fetch(j + 1);
        if constexpr (NP == 2)
            mma_stage_x2<B1>(smem[0], smem[1], acc, wm, wn, lr, half);
        else
            mma_stage_x6(smem[0], smem[1], acc, wm, wn, lr, half);
    }
    __syncthreads();
}

// The power-of-two operand scales 2^ea, 2^eb of a two-piece fp16 product; the accumulators are scaled
// back by 2^-(ea+eb) with one exact ldexp each.
struct PairScales {
    float sa = 1.0f, sb = 1.0f;
    int ex = 0;
    __device__ __forceinline__ PairScales() = default;
    __device__ __forceinline__ PairScales(const unsigned* amax_a, const unsigned* amax_b) {
        const int ea = pair_scale_exp(amax_group_max(amax_a)), eb = pair_scale_exp(amax_group_max(amax_b));
        sa = exp2_int(ea);
        sb = exp2_int(eb);
        ex = -(ea + eb);
    }
    __device__ __forceinline__ void unscale(f32x16& a) const {
#pragma unroll
        for (int i = 0; i < 16; ++i) a[i] = __builtin_amdgcn_ldexpf(a[i], ex);
    }
    template <int A, int B>
    __device__ __forceinline__ void unscale(f32x16 (&acc)[A][B]) const {
#pragma unroll
        for (int i = 0; i < A; ++i)
#pragma unroll
            for (int j = 0; j < B; ++j) unscale(acc[i][j]);
    }
    template <int A, int B, int C>
    __device__ __forceinline__ void unscale(f32x16 (&acc)[A][B][C]) const {
#pragma unroll
        for (int i = 0; i < A; ++i) unscale(acc[i]);
    }
};

// Split products with 16-deep K stages, three workgroups per CU: half the LDS (36 KB) and half the staging
// registers of the 32-deep form, for grids that fill the chip in one round at three per CU but not at two
// (e.g. 654 tiles: one round on 768 slots instead of two on 512). k-contiguous float4 operands only.
constexpr int BKQ = 16;
constexpr int KPADQ = BKQ + 8;       // 48-byte rows: b128 fragment reads of 16 consecutive rows hit distinct banks
constexpr int STAGE_Q = BM * KPADQ;  // bf16 elements per operand plane

struct OperandQ {
    const float* src;
    unsigned off[2];
    int kq;
    f32x4 reg[2];
    __device__ __forceinline__ OperandQ(const float* s, long ldl, int mn0, int MN, int tid) : src(s) {
        kq = (tid & 3) << 2;
#pragma unroll
        for (int i = 0; i < 2; ++i) off[i] = (unsigned)min(mn0 + (tid >> 2) + 64 * i, MN - 1) * (unsigned)ldl + kq;
    }
    __device__ __forceinline__ void full(int k0) {
#pragma unroll
        for (int i = 0; i < 2; ++i) reg[i] = *reinterpret_cast<const f32x4*>(src + off[i] + (unsigned)k0);
    }
    // The ragged last K stage: positions at or past kend (a multiple of 4) become 0.
    __device__ __forceinline__ void tail(int k0, int kend) {
        const int k = k0 + kq;
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const f32x4 v = *reinterpret_cast<const f32x4*>(src + off[i] - kq + (unsigned)min(k, kend - 4));
            reg[i] = k < kend ? v : f32x4{0, 0, 0, 0};
        }
    }
    // NP = 3: the three split planes; NP = 2: the two fp16 planes of sc·x.
    template <int NP = 3>
    __device__ __forceinline__ void store(__bf16* lds, int tid, float sc = 1.0f) const {
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const int o = ((tid >> 2) + 64 * i) * KPADQ + ((tid & 3) << 2);
            if constexpr (NP == 2) {
                f16x4 hi, lo;
                split2h_4(reg[i], sc, hi, lo);
                *reinterpret_cast<f16x4*>(lds + o) = hi;
                *reinterpret_cast<f16x4*>(lds + STAGE_Q + o) = lo;
            } else {
                bf16x4 h1, h2, h3;
                split3_4(reg[i], h1, h2, h3);
                *reinterpret_cast<bf16x4*>(lds + o) = h1;
                *reinterpret_cast<bf16x4*>(lds + STAGE_Q + o) = h2;
                *reinterpret_cast<bf16x4*>(lds + 2 * STAGE_Q + o) = h3;
            }
        }
    }
};

// The two-piece form of mma_stage_q: two fp16 planes, three products per block, the smallest first.
__device__ __forceinline__ void mma_stage_q2(const __bf16* A, const __bf16* B, f32x16 (&acc)[2][2], int wm, int wn,
                                             int lr, int half) {
    f16x8 a[2][2], b[2][2];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int pl = 0; pl < 2; ++pl) {
            a[i][pl] = *reinterpret_cast<const f16x8*>(A + pl * STAGE_Q + (wm * 64 + 32 * i + lr) * KPADQ + 8 * half);
            b[i][pl] = *reinterpret_cast<const f16x8*>(B + pl * STAGE_Q + (wn * 64 + 32 * i + lr) * KPADQ + 8 * half);
        }
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            f32x16 c = acc[i][j];
            c = __builtin_amdgcn_mfma_f32_32x32x16_f16(a[i][1], b[j][0], c, 0, 0, 0);
            c = __builtin_amdgcn_mfma_f32_32x32x16_f16(a[i][0], b[j][1], c, 0, 0, 0);
            c = __builtin_amdgcn_mfma_f32_32x32x16_f16(a[i][0], b[j][0], c, 0, 0, 0);
            acc[i][j] = c;
        }
}

__device__ __forceinline__ void mma_stage_q(const __bf16* A, const __bf16* B, f32x16 (&acc)[2][2], int wm, int wn,
                                            int lr, int half) {
    bf16x8 a[2][3], b[2][3];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int pl = 0; pl < 3; ++pl) {
            a[i][pl] = *reinterpret_cast<const bf16x8*>(A + pl * STAGE_Q + (wm * 64 + 32 * i + lr) * KPADQ + 8 * half);
            b[i][pl] = *reinterpret_cast<const bf16x8*>(B + pl * STAGE_Q + (wn * 64 + 32 * i + lr) * KPADQ + 8 * half);
        }
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            f32x16 c = acc[i][j];
            c = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[i][2], b[j][0], c, 0, 0, 0);
            c = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[i][0], b[j][2], c, 0, 0, 0);
            c = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[i][1], b[j][1], c, 0, 0, 0);
            c = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[i][1], b[j][0], c, 0, 0, 0);
            c = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[i][0], b[j][1], c, 0, 0, 0);
            c = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[i][0], b[j][0], c, 0, 0, 0);
            acc[i][j] = c;
        }
}

// NP = 3: split products; NP = 2: two-piece fp16 products (p.amax_a, p.amax_b set).
template <int MODE, bool RES, int NP = 3>
__global__ __launch_bounds__(THREADS, 3) void gemm_x6q_kernel(GemmParams p) {
    __shared__ __attribute__((aligned(16))) __bf16 smem[2][NP * STAGE_Q];
    PairScales ps;
    if constexpr (NP == 2) ps = PairScales(p.amax_a, p.amax_b);
    const TileCoord c = tile_coord(p, xcd_logical_block());
    const int len = max(0, c.ke - c.kb);
    const int nfull = len / BKQ, ntiles = nfull + (len % BKQ != 0 ? 1 : 0);
    const int rot = nfull > 0 ? c.t % nfull : 0;
    const int tid = opaque_tid(), lane = tid & 63, wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    const int lr = lane & 31, half = lane >> 5;
    OperandQ a(p.A, p.lda, c.m0, p.M, tid);
    OperandQ b(p.B, p.ldb, c.n0, p.N, tid);
    auto fetch = [&](int j) {
        if (j < nfull) {
            int q = j + rot;
            if (q >= nfull) q -= nfull;
            a.full(c.kb + q * BKQ);
            b.full(c.kb + q * BKQ);
        } else {
            a.tail(c.kb + nfull * BKQ, c.ke);
            b.tail(c.kb + nfull * BKQ, c.ke);
        }
    };
    f32x16 acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) acc[i][j] = f32x16{};
    if (ntiles > 0) fetch(0);
    for (int j = 0; j < ntiles; ++j) {
        __syncthreads();
        a.template store<NP>(smem[0], tid, ps.sa);
        b.template store<NP>(smem[1], tid, ps.sb);
        __syncthreads();
        if (j + 1 < ntiles) fetch(j + 1);
        if constexpr (NP == 2)
            mma_stage_q2(smem[0], smem[1], acc, wm, wn, lr, half);
        else
            mma_stage_q(smem[0], smem[1], acc, wm, wn, lr, half);
    }
    if constexpr (NP == 2) ps.unscale(acc);
    tile_store<true, true, MODE, RES>(p, c, acc);
}

// Split products on 256 x 256 tiles: eight waves (2 x 4), each owning two 64 x 64 subtiles 128 rows apart,
// one workgroup per CU, two 16-deep LDS stages (147 KB). The operand split is VALU work that the SIMD does
// not overlap with its matrix-core work, and a tile splits its A and B rows once per stage: 256 x 256
// splits half as many elements per MFMA as 128 x 128, and reads 25 % fewer LDS fragment bytes per MFMA.
// The stage being filled (split and stored by every thread) and the stage being multiplied alternate
// with one barrier per stage, and the barrier orders LDS only, so the next stage's global loads stay in
// flight across it. NT (both operands k-contiguous float4), whole K range, K a multiple of 16.
constexpr int WT = 256, WT_THREADS = 512, STAGE_W = WT * KPADQ;

// A barrier that orders this workgroup's LDS accesses only (global loads in flight are not waited for).
__device__ __forceinline__ void lds_barrier() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// Raw buffer descriptor over `bytes` bytes of p (offsets are 32-bit; the host keeps operands under 2³¹ B).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buffer_of(const void* p, unsigned bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), 0, (int)bytes, 0x00020000);
}

// GeGLU's product y = x·Wᵀ, W = [first half; second half] ([2·inter, K]), with the GeGLU applied in the epilogue
// (STORE_GEGLU): a 256-wide tile covers 128 output columns a0 … a0 + 127 of both halves. Tile row ρ of B
// (wave column wn = ρ / 64, block j = ρ / 32 mod 2, lane l = ρ mod 32) is W's row a (j = 0) or inter + a (j = 1),
// a = a0 + 32·wn + l, so a wave's two column blocks hold the two halves of the same 32 columns, lane by lane.
__device__ __forceinline__ int geglu_b_row(int rho, int a0, int inter) {
    const int a = min(a0 + 32 * (rho >> 6) + (rho & 31), inter - 1);
    return ((rho >> 5) & 1) ? inter + a : a;
}

// The STORE_GEGLU epilogue of one wave's rows (the accumulator layout store_acc takes for AK, BKC): both halves
// into C at their own columns, and act = gelu(first)·second (geglu_fwd's arithmetic) with its bf16 copy; am
// collects max|act|. c.n0 is the tile's first output column a0.
template <bool GUARD, int NI>
__device__ __forceinline__ void store_geglu(const GemmParams& p, const TileCoord& c, const f32x16 (&acc)[NI][2], int wm,
                                            int wn, int lr, int kh, unsigned* am) {
    const int a = c.n0 + 32 * wn + lr;
    if (GUARD && a >= p.inter) return;
    const float bg = p.bias ? p.bias[a] : 0.0f, bu = p.bias ? p.bias[p.inter + a] : 0.0f;
#pragma unroll
    for (int i = 0; i < NI; ++i)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const int row = c.m0 + wm * 64 + 32 * i + 8 * (r >> 2) + kh + (r & 3);
            if (GUARD && row >= p.M) continue;
            const float g = acc[i][0][r] + bg, u = acc[i][1][r] + bu;
            float* w = p.C + (long)row * p.ldc;
            w[a] = g;
            w[p.inter + a] = u;
            const float v = gelu_f(g) * u;
            p.act[(long)row * p.inter + a] = v;
            if (p.act16) p.act16[(long)row * p.inter + a] = (__bf16)v;
            *am = max(*am, amax_bits(v));
        }
}

// A 256-row k-contiguous operand's 16-deep stage: thread t holds 4 consecutive k of rows t/4 and t/4 + 128.
// Buffer loads: the per-thread row offset in a VGPR, the stage's k offset in the wave-uniform SGPR offset.
struct OperandW {
    __amdgpu_buffer_rsrc_t rsrc;
    unsigned off[2];
    f32x4 reg[2];
    __device__ __forceinline__ OperandW(const float* s, long ldl, int mn0, int MN, int tid, unsigned bytes)
        : rsrc(buffer_of(s, bytes)) {
#pragma unroll
        for (int i = 0; i < 2; ++i)
            off[i] = ((unsigned)min(mn0 + (tid >> 2) + 128 * i, MN - 1) * (unsigned)ldl + ((tid & 3) << 2)) * 4u;
    }
    // The GeGLU form (STORE_GEGLU): tile row ρ is B's row geglu_b_row(ρ, a0, inter).
    __device__ __forceinline__ OperandW(const float* s, long ldl, int a0, int inter, int tid, unsigned bytes, bool)
        : rsrc(buffer_of(s, bytes)) {
#pragma unroll
        for (int i = 0; i < 2; ++i)
            off[i] = ((unsigned)geglu_b_row((tid >> 2) + 128 * i, a0, inter) * (unsigned)ldl + ((tid & 3) << 2)) * 4u;
    }
    __device__ __forceinline__ void full(int k0) {
#pragma unroll
        for (int i = 0; i < 2; ++i)
            reg[i] = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(rsrc, off[i], k0 * 4, 0));
    }
    // NP = 3: the three split planes; NP = 2: the two fp16 planes of s·x (ONE: the hi plane only, for
    // bf16-valued operands); NP = 1: one plane of the values rounded to bf16.
    template <int NP = 3, bool ONE = false>
    __device__ __forceinline__ void store(__bf16* lds, int tid, float sc = 1.0f) const {
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const int o = ((tid >> 2) + 128 * i) * KPADQ + ((tid & 3) << 2);
            if constexpr (NP == 2 && ONE) {
                *reinterpret_cast<f16x4*>(lds + o) = split1h_4(reg[i], sc);
            } else if constexpr (NP == 2) {
                f16x4 hi, lo;
                split2h_4(reg[i], sc, hi, lo);
                *reinterpret_cast<f16x4*>(lds + o) = hi;
                *reinterpret_cast<f16x4*>(lds + STAGE_W + o) = lo;
            } else if constexpr (NP == 3) {
                bf16x4 h1, h2, h3;
                split3_4(reg[i], h1, h2, h3);
                *reinterpret_cast<bf16x4*>(lds + o) = h1;
                *reinterpret_cast<bf16x4*>(lds + STAGE_W + o) = h2;
                *reinterpret_cast<bf16x4*>(lds + 2 * STAGE_W + o) = h3;
            } else {
                *reinterpret_cast<bf16x4*>(lds + o) = __builtin_convertvector(reg[i], bf16x4);
            }
        }
    }
};

// OperandW over a bf16 copy (one plane, the bf16 products): thread t loads its 4 k of each row as 8 bytes
// and stores them as loaded.
struct OperandW16 {
    typedef unsigned u32x2 __attribute__((ext_vector_type(2)));
    __amdgpu_buffer_rsrc_t rsrc;
    unsigned off[2];
    u32x2 reg[2];
    __device__ __forceinline__ OperandW16(const __bf16* s, long ldl, int mn0, int MN, int tid, unsigned bytes)
        : rsrc(buffer_of(s, bytes)) {
#pragma unroll
        for (int i = 0; i < 2; ++i)
            off[i] = ((unsigned)min(mn0 + (tid >> 2) + 128 * i, MN - 1) * (unsigned)ldl + ((tid & 3) << 2)) * 2u;
    }
    __device__ __forceinline__ void full(int k0) {
#pragma unroll
        for (int i = 0; i < 2; ++i) reg[i] = __builtin_amdgcn_raw_buffer_load_b64(rsrc, off[i], k0 * 2, 0);
    }
    __device__ __forceinline__ void tail(int k0, int) { full(k0); }
    template <int NP = 1, bool = false>
    __device__ __forceinline__ void store(__bf16* lds, int tid, float = 1.0f) const {
        static_assert(NP == 1, "a bf16 copy feeds bf16 products");
#pragma unroll
        for (int i = 0; i < 2; ++i)
            *reinterpret_cast<u32x2*>(lds + ((tid >> 2) + 128 * i) * KPADQ + ((tid & 3) << 2)) = reg[i];
    }
};

__device__ __forceinline__ void mma6(const bf16x8 (&a)[3], const bf16x8 (&b)[3], f32x16& acc) {
    f32x16 c = acc;
    c = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[2], b[0], c, 0, 0, 0);
    c = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[0], b[2], c, 0, 0, 0);
    c = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[1], b[1], c, 0, 0, 0);
    c = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[1], b[0], c, 0, 0, 0);
    c = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[0], b[1], c, 0, 0, 0);
    c = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[0], b[0], c, 0, 0, 0);
    acc = c;
}

// The three fp16 piece products of a two-piece product block, smallest first.
__device__ __forceinline__ void mma3h(const f16x8 (&a)[2], const f16x8 (&b)[2], f32x16& acc) {
    f32x16 c = acc;
    c = __builtin_amdgcn_mfma_f32_32x32x16_f16(a[1], b[0], c, 0, 0, 0);
    c = __builtin_amdgcn_mfma_f32_32x32x16_f16(a[0], b[1], c, 0, 0, 0);
    c = __builtin_amdgcn_mfma_f32_32x32x16_f16(a[0], b[0], c, 0, 0, 0);
    acc = c;
}

// The two products of a two-piece block whose B is one piece (bf16-valued), smallest first.
__device__ __forceinline__ void mma2h(const f16x8 (&a)[2], const f16x8 (&b)[2], f32x16& acc) {
    f32x16 c = acc;
    c = __builtin_amdgcn_mfma_f32_32x32x16_f16(a[1], b[0], c, 0, 0, 0);
    c = __builtin_amdgcn_mfma_f32_32x32x16_f16(a[0], b[0], c, 0, 0, 0);
    acc = c;
}

// Two-piece fp16 stage: the same fragment walk as mma_stage_w over two fp16 planes, three products each
// (B1: B's one plane, two products each).
template <bool B1 = false>
__device__ __forceinline__ void mma_stage_w2(const __bf16* A, const __bf16* B, f32x16 (&acc)[2][2][2], int wm, int wn,
                                             int lr, int half) {
    constexpr int BP = B1 ? 1 : 2;
    const _Float16* Ah = reinterpret_cast<const _Float16*>(A);
    const _Float16* Bh = reinterpret_cast<const _Float16*>(B);
    f16x8 b[2][2], a[2][2];
    auto rd_a = [&](int g, f16x8 (&dst)[2]) {
        const int row = 128 * (g >> 1) + wm * 64 + 32 * (g & 1) + lr;
#pragma unroll
        for (int pl = 0; pl < 2; ++pl)
            dst[pl] = *reinterpret_cast<const f16x8*>(Ah + pl * STAGE_W + row * KPADQ + 8 * half);
    };
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int pl = 0; pl < BP; ++pl)
            b[j][pl] = *reinterpret_cast<const f16x8*>(Bh + pl * STAGE_W + (wn * 64 + 32 * j + lr) * KPADQ + 8 * half);
    rd_a(0, a[0]);
#pragma unroll
    for (int g = 0; g < 4; ++g) {
        if (g + 1 < 4) rd_a(g + 1, a[(g + 1) & 1]);
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            if constexpr (B1)
                mma2h(a[g & 1], b[j], acc[g >> 1][g & 1][j]);
            else
                mma3h(a[g & 1], b[j], acc[g >> 1][g & 1][j]);
        }
    }
}

// One 16-deep stage of a wave's two subtiles: B fragments once, A fragments one 32-row group ahead.
// NP = 3: six piece products per block (split products); NP = 2: three fp16 piece products (two-piece
// products; B1: B in one piece, two); NP = 1: one bf16 product.
template <int NP = 3, bool B1 = false>
__device__ __forceinline__ void mma_stage_w(const __bf16* A, const __bf16* B, f32x16 (&acc)[2][2][2], int wm, int wn,
                                            int lr, int half) {
    if constexpr (NP == 2) {
        mma_stage_w2<B1>(A, B, acc, wm, wn, lr, half);
        return;
    }
    bf16x8 b[2][3], a[2][3];
    auto rd_a = [&](int g, bf16x8 (&dst)[3]) {
        const int row = 128 * (g >> 1) + wm * 64 + 32 * (g & 1) + lr;
#pragma unroll
        for (int pl = 0; pl < NP; ++pl)
            dst[pl] = *reinterpret_cast<const bf16x8*>(A + pl * STAGE_W + row * KPADQ + 8 * half);
    };
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int pl = 0; pl < NP; ++pl)
            b[j][pl] = *reinterpret_cast<const bf16x8*>(B + pl * STAGE_W + (wn * 64 + 32 * j + lr) * KPADQ + 8 * half);
    rd_a(0, a[0]);
#pragma unroll
    for (int g = 0; g < 4; ++g) {
        if (g + 1 < 4) rd_a(g + 1, a[(g + 1) & 1]);
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            if constexpr (NP == 3)
                mma6(a[g & 1], b[j], acc[g >> 1][g & 1][j]);
            else
                acc[g >> 1][g & 1][j] =
                    __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[g & 1][0], b[j][0], acc[g >> 1][g & 1][j], 0, 0, 0);
        }
    }
}

// The k-contiguous operand of the wide NT kernel: fp32 (split or rounded as it is staged) or its bf16 copy.
template <bool H>
struct WideK {
    typedef OperandW T;
    static __device__ __forceinline__ T make(const float* s, const __bf16*, long ld, int mn0, int MN, int tid) {
        return T(s, ld, mn0, MN, tid, (unsigned)(MN * ld * 4));
    }
};
template <>
struct WideK<true> {
    typedef OperandW16 T;
    static __device__ __forceinline__ T make(const float*, const __bf16* h, long ld, int mn0, int MN, int tid) {
        return T(h, ld, mn0, MN, tid, (unsigned)(MN * ld * 2));
    }
};


// NP = 3: the split (fp32) product; NP = 2: the two-piece fp16 product (fp32-accurate, scaled operands; B1:
// B bf16-valued, in one piece); NP = 1: the bf16 product, with AH / BH reading A / B from their bf16 copies.
template <int MODE, int NP = 3, bool AH = false, bool BH = false, bool B1 = false>
__global__ __launch_bounds__(WT_THREADS, 1) void gemm_x6w_kernel(GemmParams p) {
    static_assert(MODE == STORE || MODE == STORE_ROPE || MODE == STORE_GEGLU, "whole-K NT epilogues");
    static_assert(MODE != STORE_GEGLU || (NP == 2 && !BH), "the GeGLU epilogue is a two-piece product's");
    static_assert(NP == 1 || !(AH || BH), "bf16 copies feed bf16 products");
    static_assert(NP == 2 || !B1, "one-piece B is a two-piece product's");
    PairScales ps;
    if constexpr (NP == 2) ps = PairScales(p.amax_a, p.amax_b);
    __shared__ __attribute__((aligned(16))) __bf16 smem[2][2][3 * STAGE_W];  // [stage][operand]
    const int t = xcd_logical_block();
    const int tm = t / p.tiles_n;
    TileCoord c;
    c.split = 0;
    c.t = t;
    c.m0 = tm * WT;
    c.n0 = (t - tm * p.tiles_n) * (MODE == STORE_GEGLU ? WT / 2 : WT);  // GeGLU: output columns of act
    c.kb = 0;
    c.ke = p.K;
    const int nt = p.K / BKQ;
    const int rot = t % nt;
    const int tid = opaque_tid(), lane = tid & 63, wave = tid >> 6;
    const int wm = wave >> 2, wn = wave & 3;
    const int lr = lane & 31, half = lane >> 5;
    typename WideK<AH>::T a = WideK<AH>::make(p.A, p.A16, p.lda, c.m0, p.M, tid);
    typename WideK<BH>::T b = [&] {
        if constexpr (MODE == STORE_GEGLU)
            return OperandW(p.B, p.ldb, c.n0, p.inter, tid, (unsigned)(p.N * p.ldb * 4), true);
        else
            return WideK<BH>::make(p.B, p.B16, p.ldb, c.n0, p.N, tid);
    }();
    auto kof = [&](int j) {
        const int q = j + rot;
        return (q >= nt ? q - nt : q) * BKQ;
    };
    f32x16 acc[2][2][2];
#pragma unroll
    for (int s = 0; s < 2; ++s)
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
            for (int j = 0; j < 2; ++j) acc[s][i][j] = f32x16{};
    a.full(kof(0));
    b.full(kof(0));
    a.template store<NP>(smem[0][0], tid, ps.sa);
    b.template store<NP, B1>(smem[0][1], tid, ps.sb);
    a.full(kof(min(1, nt - 1)));
    b.full(kof(min(1, nt - 1)));
    lds_barrier();
    // Branch-free body: the last two iterations reload the last stage and fill a stage no one reads.
    for (int j = 0; j < nt; ++j) {
        const int cur = j & 1;
        const int kn = kof(min(j + 2, nt - 1));
        mma_stage_w<NP, B1>(smem[cur][0], smem[cur][1], acc, wm, wn, lr, half);
        a.template store<NP>(smem[cur ^ 1][0], tid, ps.sa);
        b.template store<NP, B1>(smem[cur ^ 1][1], tid, ps.sb);
        a.full(kn);
        b.full(kn);
        lds_barrier();
    }
    if constexpr (NP == 2) ps.unscale(acc);
    unsigned am = 0;  // max|C| of the lane's stores, when the product keeps C's magnitude word
    if constexpr (NP == 2 && MODE == STORE_ROPE) {
        // The RoPE epilogue has no registers to spare for the stores' maximum: without a bias, C's word takes
        // twice the largest product instead, a bound on the rotated values (a rotated pair is at most
        // √2 × the larger of the two, plus rounding). The word only sets the power-of-two scale of the
        // attention operands, which a bound within a factor 4 of the maximum keeps in fp16 range.
        if (p.amax_c && !p.bias) {
            // One max per value (NaNs drop out of fmaxf); an infinity among the products takes the exact
            // finite maximum instead, so that the scale still fits the finite values.
            float m4[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int s = 0; s < 2; ++s)
#pragma unroll
                for (int i = 0; i < 2; ++i)
#pragma unroll
                    for (int j = 0; j < 2; ++j)
#pragma unroll
                        for (int r = 0; r < 16; ++r) m4[r & 3] = fmaxf(m4[r & 3], fabsf(acc[s][i][j][r]));
            am = __builtin_bit_cast(unsigned, fmaxf(fmaxf(m4[0], m4[1]), fmaxf(m4[2], m4[3])));
            if (am >= 0x7f800000u) {
                am = 0;
#pragma unroll
                for (int s = 0; s < 2; ++s)
#pragma unroll
                    for (int i = 0; i < 2; ++i)
#pragma unroll
                        for (int j = 0; j < 2; ++j)
#pragma unroll
                            for (int r = 0; r < 16; ++r) am = max(am, amax_bits(acc[s][i][j][r]));
            }
            am = am == 0 ? 0u : am < 0x7f000000u ? am + 0x00800000u : 0x7f7fffffu;  // 2·max, finite
        }
        // Folded here, so that no register holds it through the epilogue.
        block_amax_fold(am, p.bias ? nullptr : p.amax_c);
    }
    // The epilogue's lane coordinates are taken again after the K loop, so its store offsets are computed
    // here rather than held across the loop (the RoPE epilogue measured fewer spills the other way).
    const int te = MODE == STORE_ROPE ? tid : opaque_tid(), le = te & 63, we = te >> 6;
    // The stages are done (the loop ended on a barrier): park the second subtile's accumulators in LDS,
    // each thread in its own slots, so the first subtile's epilogue has their registers.
    f32x16* park = reinterpret_cast<f32x16*>(&smem[0][0][0]);
#pragma unroll
    for (int q = 0; q < 4; ++q) park[q * WT_THREADS + te] = acc[1][q >> 1][q & 1];
#pragma unroll
    for (int s = 0; s < 2; ++s) {
        TileCoord cs = c;
        cs.m0 = c.m0 + 128 * s;
        if (cs.m0 >= p.M) break;
        if (s == 1) {
#pragma unroll
            for (int q = 0; q < 4; ++q) acc[1][q >> 1][q & 1] = park[q * WT_THREADS + te];
        }
        if constexpr (MODE == STORE_GEGLU) {
            if (cs.m0 + 128 <= p.M && c.n0 + WT / 2 <= p.inter)
                store_geglu<false, 2>(p, cs, acc[s], we >> 2, we & 3, le & 31, (le >> 5) << 2, &am);
            else
                store_geglu<true, 2>(p, cs, acc[s], we >> 2, we & 3, le & 31, (le >> 5) << 2, &am);
            continue;
        } else {
        const bool full = cs.m0 + 128 <= p.M && c.n0 + WT <= p.N;
        // (Not with the RoPE epilogue, whose registers it would spill: the bound above, or launch_wide
        // measures C afterwards when there is a bias.)
        if (NP == 2 && MODE != STORE_ROPE && p.amax_c) {
            if (full)
                store_acc<true, true, MODE, false, false, true, 2, true>(p, cs, acc[s], we >> 2, we & 3, le & 31,
                                                                         (le >> 5) << 2, &am);
            else
                store_acc<true, true, MODE, false, true, true, 2, true>(p, cs, acc[s], we >> 2, we & 3, le & 31,
                                                                        (le >> 5) << 2, &am);
        } else if (full) {
            store_acc<true, true, MODE, false, false, true>(p, cs, acc[s], we >> 2, we & 3, le & 31, (le >> 5) << 2);
        } else {
            store_acc<true, true, MODE, false, true, true>(p, cs, acc[s], we >> 2, we & 3, le & 31, (le >> 5) << 2);
        }
        }
    }
    if constexpr (MODE == STORE_GEGLU)
        block_amax_fold(am, p.amax_act);
    else if constexpr (NP == 2 && MODE != STORE_ROPE)
        block_amax_fold(am, p.amax_c);
}

// ------------------------------------------------------------- operand magnitudes for two-piece products
//
// max|x| over the finite elements of a rows x cols operand (row stride ld) as an fp32 bit pattern,
// folded into *out (which holds 0 or a smaller pattern beforehand) by one atomicMax per block: the
// maximum is the same whatever the order, and the product that reads it is a later launch. Infinities
// and NaNs are left out, so the scale fits the finite values and the non-finite ones still reach the
// products (an infinity's low piece is a NaN: outputs that an infinity reaches are non-finite, as in
// fp32, though possibly NaN where fp32 gives an infinity).
constexpr int AMAX_BLOCKS = 1024, AMAX_SLOTS = 6;

__global__ __launch_bounds__(256) void absmax_kernel(const float* __restrict__ x, int rows, int cols, long ld,
                                                     int vec, unsigned* out) {
    unsigned m = 0;
    const int tid = threadIdx.x;
    if (vec && ld == cols) {
        const long n4 = (long)rows * cols / 4;
        const f32x4* x4 = reinterpret_cast<const f32x4*>(x);
        const long stride = (long)gridDim.x * 256;
        long i = (long)blockIdx.x * 256 + tid;
        for (; i + 3 * stride < n4; i += 4 * stride) {
            f32x4 v[4];
#pragma unroll
            for (int u = 0; u < 4; ++u) v[u] = __builtin_nontemporal_load(x4 + i + u * stride);
#pragma unroll
            for (int u = 0; u < 4; ++u) m = max(m, amax_bits4(v[u]));
        }
        for (; i < n4; i += stride) m = max(m, amax_bits4(x4[i]));
    } else if (vec) {
        for (int r = blockIdx.x; r < rows; r += gridDim.x) {
            const f32x4* row = reinterpret_cast<const f32x4*>(x + (long)r * ld);
            for (int c = tid; c < cols / 4; c += 256) m = max(m, amax_bits4(row[c]));
        }
    } else {
        for (int r = blockIdx.x; r < rows; r += gridDim.x)
            for (int c = tid; c < cols; c += 256) m = max(m, amax_bits(x[(long)r * ld + c]));
    }
    block_amax_fold(m, out);
}

// ------------------------------------------------------------- split products on 192 x 256 tiles
//
// The wide kernel's loop on 192-row tiles, for outputs 256-wide products leave under-filled: an output
// 768 columns wide and ≈ 14 k rows is 165 tiles of 256 x 256 (65 % of 256 CUs) but 219 of 192 x 256
// (one round at 86 %), the same work per CU as three 128 x 128 tiles with the wide tile's operand reuse.
// Eight waves (2 x 4), each owning 96 x 64 (three 32-row groups by two 32-column groups). NT, whole K,
// K a multiple of 16; STORE with optional residual, or STORE_ROPE.
constexpr int TM = 192, STAGE_T = TM * KPADQ;
constexpr double TALL_GAIN = 1.25;  // 192 x 256 over three 128 x 128 per CU, per unit of work

// The 192-row k-contiguous operand's 16-deep stage: thread t holds 4 consecutive k of row t/4 and, for
// t < 256 (waves 0-3, wave-uniform), of row 128 + t/4.
struct OperandT {
    __amdgpu_buffer_rsrc_t rsrc;
    unsigned off[2];
    f32x4 reg[2];
    bool two;
    __device__ __forceinline__ OperandT(const float* s, long ldl, int mn0, int MN, int tid, unsigned bytes)
        : rsrc(buffer_of(s, bytes)), two(tid < 256) {
#pragma unroll
        for (int i = 0; i < 2; ++i)
            off[i] = ((unsigned)min(mn0 + (tid >> 2) + 128 * i, MN - 1) * (unsigned)ldl + ((tid & 3) << 2)) * 4u;
    }
    __device__ __forceinline__ void full(int k0) {
        reg[0] = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(rsrc, off[0], k0 * 4, 0));
        if (two) reg[1] = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(rsrc, off[1], k0 * 4, 0));
    }
    template <int NP = 3>
    __device__ __forceinline__ void store(__bf16* lds, int tid, float sc = 1.0f) const {
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            if (i == 1 && !two) break;
            const int o = ((tid >> 2) + 128 * i) * KPADQ + ((tid & 3) << 2);
            if constexpr (NP == 2) {
                f16x4 hi, lo;
                split2h_4(reg[i], sc, hi, lo);
                *reinterpret_cast<f16x4*>(lds + o) = hi;
                *reinterpret_cast<f16x4*>(lds + STAGE_T + o) = lo;
                continue;
            }
            bf16x4 h1, h2, h3;
            split3_4(reg[i], h1, h2, h3);
            *reinterpret_cast<bf16x4*>(lds + o) = h1;
            *reinterpret_cast<bf16x4*>(lds + STAGE_T + o) = h2;
            *reinterpret_cast<bf16x4*>(lds + 2 * STAGE_T + o) = h3;
        }
    }
};

// The two-piece fp16 form of mma_stage_t: two fp16 planes, three products per block (B1: B's one plane, two).
template <bool B1 = false>
__device__ __forceinline__ void mma_stage_t2(const __bf16* A, const __bf16* B, f32x16 (&acc)[3][2], int wm, int wn,
                                             int lr, int half) {
    constexpr int BP = B1 ? 1 : 2;
    const _Float16* Ah = reinterpret_cast<const _Float16*>(A);
    const _Float16* Bh = reinterpret_cast<const _Float16*>(B);
    f16x8 b[2][2], a[2][2];
    auto rd_a = [&](int g, f16x8 (&dst)[2]) {
        const int row = 96 * wm + 32 * g + lr;
#pragma unroll
        for (int pl = 0; pl < 2; ++pl)
            dst[pl] = *reinterpret_cast<const f16x8*>(Ah + pl * STAGE_T + row * KPADQ + 8 * half);
    };
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int pl = 0; pl < BP; ++pl)
            b[j][pl] = *reinterpret_cast<const f16x8*>(Bh + pl * STAGE_W + (wn * 64 + 32 * j + lr) * KPADQ + 8 * half);
    rd_a(0, a[0]);
#pragma unroll
    for (int g = 0; g < 3; ++g) {
        if (g + 1 < 3) rd_a(g + 1, a[(g + 1) & 1]);
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            if constexpr (B1)
                mma2h(a[g & 1], b[j], acc[g][j]);
            else
                mma3h(a[g & 1], b[j], acc[g][j]);
        }
    }
}

// One 16-deep stage of a wave's 96 x 64: B fragments once, A fragments one 32-row group ahead.
template <int NP = 3, bool B1 = false>
__device__ __forceinline__ void mma_stage_t(const __bf16* A, const __bf16* B, f32x16 (&acc)[3][2], int wm, int wn,
                                            int lr, int half) {
    if constexpr (NP == 2) {
        mma_stage_t2<B1>(A, B, acc, wm, wn, lr, half);
        return;
    }
    bf16x8 b[2][3], a[2][3];
    auto rd_a = [&](int g, bf16x8 (&dst)[3]) {
        const int row = 96 * wm + 32 * g + lr;
#pragma unroll
        for (int pl = 0; pl < 3; ++pl)
            dst[pl] = *reinterpret_cast<const bf16x8*>(A + pl * STAGE_T + row * KPADQ + 8 * half);
    };
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int pl = 0; pl < 3; ++pl)
            b[j][pl] = *reinterpret_cast<const bf16x8*>(B + pl * STAGE_W + (wn * 64 + 32 * j + lr) * KPADQ + 8 * half);
    rd_a(0, a[0]);
#pragma unroll
    for (int g = 0; g < 3; ++g) {
        if (g + 1 < 3) rd_a(g + 1, a[(g + 1) & 1]);
#pragma unroll
        for (int j = 0; j < 2; ++j) mma6(a[g & 1], b[j], acc[g][j]);
    }
}

// NP = 3: split products; NP = 2: two-piece fp16 products (B1: B bf16-valued, in one piece).
template <int MODE, bool RES, int NP = 3, bool B1 = false>
__global__ __launch_bounds__(WT_THREADS, 1) void gemm_x6t_kernel(GemmParams p) {
    static_assert(MODE == STORE || ((MODE == STORE_ROPE || MODE == STORE_GEGLU) && !RES), "whole-K NT epilogues");
    static_assert(MODE != STORE_GEGLU || NP == 2, "the GeGLU epilogue is a two-piece product's");
    static_assert(NP == 2 || !B1, "one-piece B is a two-piece product's");
    PairScales ps;
    if constexpr (NP == 2) ps = PairScales(p.amax_a, p.amax_b);
    __shared__ __attribute__((aligned(16))) __bf16 smem[2][3 * (STAGE_T + STAGE_W)];  // [stage][A planes, B planes]
    const int t = xcd_logical_block();
    const int tm = t / p.tiles_n;
    TileCoord c;
    c.split = 0;
    c.t = t;
    c.m0 = tm * TM;
    c.n0 = (t - tm * p.tiles_n) * (MODE == STORE_GEGLU ? WT / 2 : WT);  // GeGLU: output columns of act
    c.kb = 0;
    c.ke = p.K;
    const int nt = p.K / BKQ;
    const int rot = t % nt;
    const int tid = opaque_tid(), lane = tid & 63, wave = tid >> 6;
    const int wm = wave >> 2, wn = wave & 3;
    const int lr = lane & 31, half = lane >> 5;
    OperandT a(p.A, p.lda, c.m0, p.M, tid, (unsigned)(p.M * p.lda * 4));
    OperandW b = MODE == STORE_GEGLU ? OperandW(p.B, p.ldb, c.n0, p.inter, tid, (unsigned)(p.N * p.ldb * 4), true)
                                     : OperandW(p.B, p.ldb, c.n0, p.N, tid, (unsigned)(p.N * p.ldb * 4));
    auto kof = [&](int j) {
        const int q = j + rot;
        return (q >= nt ? q - nt : q) * BKQ;
    };
    f32x16 acc[3][2];
#pragma unroll
    for (int i = 0; i < 3; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) acc[i][j] = f32x16{};
    a.full(kof(0));
    b.full(kof(0));
    a.template store<NP>(smem[0], tid, ps.sa);
    b.template store<NP, B1>(smem[0] + 3 * STAGE_T, tid, ps.sb);
    a.full(kof(min(1, nt - 1)));
    b.full(kof(min(1, nt - 1)));
    lds_barrier();
    // Branch-free body: the last two iterations reload the last stage and fill a stage no one reads. The
    // next stage is committed and the one after it requested before this stage's products, so the loads have
    // the whole stage of products to arrive (the other buffer was last read before the barrier): measured
    // faster on these tiles, slower on the 256 × 256 ones, whose split the compiler interleaves with the
    // products.
    for (int j = 0; j < nt; ++j) {
        const int cur = j & 1;
        const int kn = kof(min(j + 2, nt - 1));
        a.template store<NP>(smem[cur ^ 1], tid, ps.sa);
        b.template store<NP, B1>(smem[cur ^ 1] + 3 * STAGE_T, tid, ps.sb);
        a.full(kn);
        b.full(kn);
        __builtin_amdgcn_sched_barrier(0);  // the loads are issued before the products
        mma_stage_t<NP, B1>(smem[cur], smem[cur] + 3 * STAGE_T, acc, wm, wn, lr, half);
        lds_barrier();
    }
    if constexpr (NP == 2) ps.unscale(acc);
    const int te = opaque_tid(), le = te & 63, we = te >> 6, wme = we >> 2;
    // store_acc places row group i of wave row wm at 64·wm + 32·i: a base 32·wm further down puts the
    // wave's three groups at 96·wm + 32·i.
    TileCoord cs = c;
    cs.m0 = c.m0 + 32 * wme;
    unsigned am = 0;  // max|C| (GeGLU: max|act|) of the lane's stores, when the product keeps that word
    if constexpr (MODE == STORE_GEGLU) {
        if (c.m0 + TM <= p.M && c.n0 + WT / 2 <= p.inter)
            store_geglu<false, 3>(p, cs, acc, wme, we & 3, le & 31, (le >> 5) << 2, &am);
        else
            store_geglu<true, 3>(p, cs, acc, wme, we & 3, le & 31, (le >> 5) << 2, &am);
        block_amax_fold(am, p.amax_act);
        return;
    } else {
    const bool full = c.m0 + TM <= p.M && c.n0 + WT <= p.N;
    if (NP == 2 && p.amax_c) {
        if (full)
            store_acc<true, true, MODE, RES, false, true, 3, true>(p, cs, acc, wme, we & 3, le & 31, (le >> 5) << 2,
                                                                   &am);
        else
            store_acc<true, true, MODE, RES, true, true, 3, true>(p, cs, acc, wme, we & 3, le & 31, (le >> 5) << 2,
                                                                  &am);
    } else if (full) {
        store_acc<true, true, MODE, RES, false, true>(p, cs, acc, wme, we & 3, le & 31, (le >> 5) << 2);
    } else {
        store_acc<true, true, MODE, RES, true, true>(p, cs, acc, wme, we & 3, le & 31, (le >> 5) << 2);
    }
    if constexpr (NP == 2) block_amax_fold(am, p.amax_c);
    }
}

// The fp32 product from bf16 pieces (NP = 3) or, for float4 operands, two-piece fp16 products (NP = 2);
// accumulators in the k-contiguous layout whatever the operands' form.
// B1 (NP = 2): B bf16-valued, in one piece.
template <int AOP, int BOP, int MODE, bool RES, int NP = 3, bool B1 = false>
__global__ __launch_bounds__(THREADS, 2) void gemm_x6_kernel(GemmParams p) {
    static_assert(NP == 2 || !B1, "one-piece B is a two-piece product's");
    __shared__ __attribute__((aligned(16))) __bf16 smem[2][3 * STAGE_H];
    PairScales ps;
    if constexpr (NP == 2) ps = PairScales(p.amax_a, p.amax_b);
    const TileCoord c = tile_coord(p, xcd_logical_block());
    f32x16 acc[2][2];
    tile_mma_x6<AOP, BOP, NP, B1>(p, c, smem, acc, ps.sa, ps.sb);
    if constexpr (NP == 2) ps.unscale(acc);
    tile_store<true, true, MODE, RES>(p, c, acc);
}

// The bf16 product: the tile's accumulators are in the k-contiguous layout whatever the operands' form.
template <int AOP, int BOP, int MODE, bool RES>
__global__ __launch_bounds__(THREADS, 2) void gemm_bf16_kernel(GemmParams p) {
    __shared__ __attribute__((aligned(16))) __bf16 smem[2][2][STAGE_H];
    const TileCoord c = tile_coord(p, xcd_logical_block());
    f32x16 acc[2][2];
    tile_mma_h<AOP, BOP>(p, c, smem, acc);
    tile_store<true, true, MODE, RES>(p, c, acc);
}

// dX = dY·W (NN, + residual when RES) and dW += dYᵀ·X (TN, accumulated in place or as split-K
// partials) in one grid: the first `blocks0` logical blocks are dX tiles, the rest dW slices. The two
// products are independent, and one grid lets their tiles fill the CUs together instead of each
// leaving a partial last wave.
template <int TN_MODE, bool RES>
__global__ __launch_bounds__(THREADS, 2) void gemm_pair_kernel(GemmParams nn, GemmParams tn, int blocks0) {
    __shared__ __attribute__((aligned(16))) float smem[2][2][STAGE];
    const int logical = xcd_logical_block();
    const bool is_nn = logical < blocks0;
    const GemmParams& p = is_nn ? nn : tn;
    const TileCoord c = tile_coord(p, is_nn ? logical : logical - blocks0);
    f32x16 acc[2][2];
    if (is_nn) {
        tile_mma<true, false>(nn, c, smem, acc);
        tile_store<true, false, STORE, RES>(nn, c, acc);
    } else {
        tile_mma<false, false>(tn, c, smem, acc);
        tile_store<false, false, TN_MODE, false>(tn, c, acc);
    }
}

// ------------------------------------------------------------------------------ planned pair
//
// A static, balanced schedule for the backward pair. The grid is exactly the G = 2·CUs workgroups that
// fit at once. Work is counted in units of one 128×128×32 MFMA step. Worker g takes whole dX tiles
// g, g + G, g + 2G, … and then a contiguous run of the dW unit sequence (tile t, K step a) sized so
// every worker ends up with floor((g+1)·W/G) − floor(g·W/G) units in total. A dW tile covered by one
// worker is accumulated in place; a dW tile cut between workers gets one partial per covering worker
// (a worker holds at most two: its first and its last dW tile) and `pair_fixup_kernel` adds them in
// worker order. No workgroup ever waits on another, and the sums do not depend on timing.

constexpr int FIXUP_MAX_WORKERS = 2048;  // workers a pair plan may have (2 per CU)

struct PairPlan {
    int G;                   // workers = grid size
    int nn_tiles, nn_units;  // dX tiles and K units per dX tile
    int tn_tiles, tn_units;  // dW tiles and K units per dW tile
    int q, r;                // nn_tiles = q·G + r
    int W;                   // total units (G·W < 2³¹, checked on the host)
    float* partial;          // [G][2][BM·BN] dW partial tiles, lane order
};

// First dW unit of worker g (the end of worker g is the start of worker g + 1).
__device__ __forceinline__ int plan_tn_lo(const PairPlan& s, int g) {
    return g * s.W / s.G - s.nn_units * (g * s.q + min(g, s.r));
}

__device__ __forceinline__ TileCoord unit_coord(const GemmParams& p, int t, int a, int b) {
    TileCoord c;
    c.split = 0;
    c.t = t;
    const int tile_m = t / p.tiles_n;
    c.m0 = tile_m * BM;
    c.n0 = (t - tile_m * p.tiles_n) * BN;
    c.kb = a * BK;
    c.ke = min(p.K, b * BK);
    return c;
}

// Accumulators in lane order: thread tid's 64 values as 16 float4 at (q·256 + tid)·4, q = (2i + j)·4 + r/4.
__device__ __forceinline__ void write_partial(float* slot, const f32x16 (&acc)[2][2]) {
#pragma unroll
    for (int q = 0; q < 16; ++q) {
        const int i = q >> 3, j = (q >> 2) & 1, r = (q & 3) * 4;
        *reinterpret_cast<f32x4*>(slot + (q * THREADS + threadIdx.x) * 4) =
            f32x4{acc[i][j][r], acc[i][j][r + 1], acc[i][j][r + 2], acc[i][j][r + 3]};
    }
}

template <bool RES>
__global__ __launch_bounds__(THREADS, 2) void gemm_pair_planned_kernel(GemmParams nn, GemmParams tn, PairPlan s) {
    __shared__ __attribute__((aligned(16))) float smem[2][2][STAGE];
    const int g = xcd_logical_block();
    const int count = s.q + (g < s.r ? 1 : 0);
    for (int n = 0; n < count; ++n) {
        const TileCoord c = unit_coord(nn, g + n * s.G, 0, s.nn_units);
        f32x16 acc[2][2];
        tile_mma<true, false>(nn, c, smem, acc);
        tile_store<true, false, STORE, RES>(nn, c, acc);
    }
    const int lo = plan_tn_lo(s, g), hi = plan_tn_lo(s, g + 1);
    for (int u = lo; u < hi;) {
        const int t = u / s.tn_units;
        const int a = u - t * s.tn_units;
        const int b = min(s.tn_units, a + (hi - u));
        const TileCoord c = unit_coord(tn, t, a, b);
        f32x16 acc[2][2];
        tile_mma<false, false>(tn, c, smem, acc);
        write_partial(s.partial + ((long)g * 2 + (u == lo ? 0 : 1)) * (BM * BN), acc);
        u += b - a;
    }
}

// The planned pair with split products: the same schedule and partial slots; dX tiles read dY as a
// k-contiguous operand (AOP) and W as an mn-contiguous one, dW slices read dY and x mn-contiguous.
template <int AOP, bool RES>
__global__ __launch_bounds__(THREADS, 2) void gemm_pair_planned_x6_kernel(GemmParams nn, GemmParams tn, PairPlan s) {
    __shared__ __attribute__((aligned(16))) __bf16 smem[2][3 * STAGE_H];
    const int g = xcd_logical_block();
    const int count = s.q + (g < s.r ? 1 : 0);
    for (int n = 0; n < count; ++n) {
        const TileCoord c = unit_coord(nn, g + n * s.G, 0, s.nn_units);
        f32x16 acc[2][2];
        tile_mma_x6<AOP, MNSCALAR>(nn, c, smem, acc);
        tile_store<true, true, STORE, RES>(nn, c, acc);
    }
    const int lo = plan_tn_lo(s, g), hi = plan_tn_lo(s, g + 1);
    for (int u = lo; u < hi;) {
        const int t = u / s.tn_units;
        const int a = u - t * s.tn_units;
        const int b = min(s.tn_units, a + (hi - u));
        const TileCoord c = unit_coord(tn, t, a, b);
        f32x16 acc[2][2];
        tile_mma_x6<MNSCALAR, MNSCALAR>(tn, c, smem, acc);
        write_partial(s.partial + ((long)g * 2 + (u == lo ? 0 : 1)) * (BM * BN), acc);
        u += b - a;
    }
}

// The planned pair with bf16 products (the bf16 policies for both backward product classes).
template <int AOP, bool RES>
__global__ __launch_bounds__(THREADS, 2) void gemm_pair_planned_h_kernel(GemmParams nn, GemmParams tn, PairPlan s) {
    __shared__ __attribute__((aligned(16))) __bf16 smem[2][2][STAGE_H];
    const int g = xcd_logical_block();
    const int count = s.q + (g < s.r ? 1 : 0);
    for (int n = 0; n < count; ++n) {
        const TileCoord c = unit_coord(nn, g + n * s.G, 0, s.nn_units);
        f32x16 acc[2][2];
        tile_mma_h<AOP, MNSCALAR>(nn, c, smem, acc);
        tile_store<true, true, STORE, RES>(nn, c, acc);
        __syncthreads();
    }
    const int lo = plan_tn_lo(s, g), hi = plan_tn_lo(s, g + 1);
    for (int u = lo; u < hi;) {
        const int t = u / s.tn_units;
        const int a = u - t * s.tn_units;
        const int b = min(s.tn_units, a + (hi - u));
        const TileCoord c = unit_coord(tn, t, a, b);
        f32x16 acc[2][2];
        tile_mma_h<MNSCALAR, MNSCALAR>(tn, c, smem, acc);
        write_partial(s.partial + ((long)g * 2 + (u == lo ? 0 : 1)) * (BM * BN), acc);
        __syncthreads();
        u += b - a;
    }
}

// ------------------------------------------------------------- the backward pair on 256 x 256 tiles
//
// The planned pair with the wide tiles' loop: one worker per CU (eight waves, two 16-deep LDS stages),
// whole dX tiles, then a contiguous run of 16-deep dW units whose partial tiles the wide fixup adds.

// A 256-wide mn-contiguous operand's 16-deep stage (element (mn, k) at src[k·ld + mn]): thread t holds
// mn = t mod 256 at 8 consecutive k. Full stages are buffer loads whose k row offsets are wave-uniform
// SGPR offsets; in the ragged last stage positions at or past kend read an in-bounds row and become 0.
struct OperandWS {
    __amdgpu_buffer_rsrc_t rsrc;
    unsigned base, ld4;
    int kq;
    float v[8];
    __device__ __forceinline__ OperandWS(const float* s, long ldl, int mn0, int MN, int tid, unsigned bytes)
        : rsrc(buffer_of(s, bytes)), base((unsigned)min(mn0 + (tid & 255), MN - 1) * 4u),
          ld4((unsigned)ldl * 4u), kq((tid >> 8) << 3) {}
    __device__ __forceinline__ void full(int k0) {
        const unsigned o = base + (unsigned)(k0 + kq) * ld4;
#pragma unroll
        for (int e = 0; e < 8; ++e)
            v[e] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rsrc, o, (int)(e * ld4), 0));
    }
    __device__ __forceinline__ void tail(int k0, int kend) {
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const int k = k0 + kq + e;
            const float x = __builtin_bit_cast(
                float, __builtin_amdgcn_raw_buffer_load_b32(rsrc, base + (unsigned)min(k, kend - 1) * ld4, 0, 0));
            v[e] = k < kend ? x : 0.0f;
        }
    }
    template <int NP = 3>
    __device__ __forceinline__ void store(__bf16* lds, int tid, float sc = 1.0f) const {
        const int o = (tid & 255) * KPADQ + kq;
        if constexpr (NP == 2) {
            f16x4 a1, a2, b1, b2;
            split2h_4(f32x4{v[0], v[1], v[2], v[3]}, sc, a1, a2);
            split2h_4(f32x4{v[4], v[5], v[6], v[7]}, sc, b1, b2);
            *reinterpret_cast<f16x8*>(lds + o) = __builtin_shufflevector(a1, b1, 0, 1, 2, 3, 4, 5, 6, 7);
            *reinterpret_cast<f16x8*>(lds + STAGE_W + o) = __builtin_shufflevector(a2, b2, 0, 1, 2, 3, 4, 5, 6, 7);
        } else if constexpr (NP == 3) {
            bf16x4 a1, a2, a3, b1, b2, b3;
            split3_4(f32x4{v[0], v[1], v[2], v[3]}, a1, a2, a3);
            split3_4(f32x4{v[4], v[5], v[6], v[7]}, b1, b2, b3);
            *reinterpret_cast<bf16x8*>(lds + o) = __builtin_shufflevector(a1, b1, 0, 1, 2, 3, 4, 5, 6, 7);
            *reinterpret_cast<bf16x8*>(lds + STAGE_W + o) = __builtin_shufflevector(a2, b2, 0, 1, 2, 3, 4, 5, 6, 7);
            *reinterpret_cast<bf16x8*>(lds + 2 * STAGE_W + o) = __builtin_shufflevector(a3, b3, 0, 1, 2, 3, 4, 5, 6, 7);
        } else {
            const bf16x4 lo = __builtin_convertvector((f32x4{v[0], v[1], v[2], v[3]}), bf16x4);
            const bf16x4 hi = __builtin_convertvector((f32x4{v[4], v[5], v[6], v[7]}), bf16x4);
            *reinterpret_cast<bf16x8*>(lds + o) = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
        }
    }
};

// The k-contiguous operand of the wide loop with the ragged-stage form the pair's loop calls (never
// taken: the plan requires the dX product's K to be a multiple of 16).
struct OperandWK : OperandW {
    using OperandW::OperandW;
    __device__ __forceinline__ void tail(int k0, int) { full(k0); }
};

// OperandWS over a bf16 copy (element (mn, k) at src[k·ld + mn]): the same 8 k per thread as 2-byte loads,
// stored as loaded (one plane, the bf16 products).
struct OperandWS16 {
    __amdgpu_buffer_rsrc_t rsrc;
    unsigned base, ld2;
    int kq;
    unsigned short v[8];
    __device__ __forceinline__ OperandWS16(const __bf16* s, long ldl, int mn0, int MN, int tid, unsigned bytes)
        : rsrc(buffer_of(s, bytes)), base((unsigned)min(mn0 + (tid & 255), MN - 1) * 2u),
          ld2((unsigned)ldl * 2u), kq((tid >> 8) << 3) {}
    __device__ __forceinline__ void full(int k0) {
        const unsigned o = base + (unsigned)(k0 + kq) * ld2;
#pragma unroll
        for (int e = 0; e < 8; ++e) v[e] = __builtin_amdgcn_raw_buffer_load_b16(rsrc, o, (int)(e * ld2), 0);
    }
    __device__ __forceinline__ void tail(int k0, int kend) {
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const int k = k0 + kq + e;
            const unsigned short x =
                __builtin_amdgcn_raw_buffer_load_b16(rsrc, base + (unsigned)min(k, kend - 1) * ld2, 0, 0);
            v[e] = k < kend ? x : (unsigned short)0;
        }
    }
    template <int NP = 1>
    __device__ __forceinline__ void store(__bf16* lds, int tid, float = 1.0f) const {
        static_assert(NP == 1, "a bf16 copy feeds bf16 products");
        typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
        u32x4 w;
#pragma unroll
        for (int i = 0; i < 4; ++i) w[i] = (unsigned)v[2 * i] | ((unsigned)v[2 * i + 1] << 16);
        *reinterpret_cast<u32x4*>(lds + (tid & 255) * KPADQ + kq) = w;
    }
};

// The mn-contiguous B operand of the wide pair: fp32 or its bf16 copy.
template <bool H>
struct WideS {
    typedef OperandWS T;
    static __device__ __forceinline__ T make(const float* s, const __bf16*, long ld, int mn0, int MN, int tid,
                                             long rows) {
        return T(s, ld, mn0, MN, tid, (unsigned)(rows * ld * 4));
    }
};
template <>
struct WideS<true> {
    typedef OperandWS16 T;
    static __device__ __forceinline__ T make(const float*, const __bf16* h, long ld, int mn0, int MN, int tid,
                                             long rows) {
        return T(h, ld, mn0, MN, tid, (unsigned)(rows * ld * 2));
    }
};

// acc += A·Bᵀ over K positions [kb, ke) in 16-deep stages: the full stages in rotated order starting at
// `rot`, then the ragged last one (when ke − kb is not a multiple of 16) on its own, so the loop body
// carries no per-element selects.
// sa, sb: the operands' scales (two-piece fp16 products; 1 otherwise).
template <int NP, class OA, class OB>
__device__ __forceinline__ void wide_mma(OA& a, OB& b, int kb, int ke, int rot, __bf16 (*smem)[2][3 * STAGE_W],
                                         f32x16 (&acc)[2][2][2], int tid, int wm, int wn, int lr, int half,
                                         float sa = 1.0f, float sb = 1.0f) {
    const int len = ke - kb, nfull = len / BKQ;
    rot = nfull > 0 ? rot % nfull : 0;
    auto fetch = [&](int j) {
        const int q = j + rot;
        const int k0 = kb + (q >= nfull ? q - nfull : q) * BKQ;
        a.full(k0);
        b.full(k0);
    };
#pragma unroll
    for (int s = 0; s < 2; ++s)
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
            for (int j = 0; j < 2; ++j) acc[s][i][j] = f32x16{};
    if (NP == 1 && nfull > 1) {
        // bf16 products: one MFMA per block leaves a 16-deep stage short, so each LDS buffer holds two stages
        // (the second in the plane the single-plane form leaves free) and a barrier serves both; (a, b) and
        // (a1, b1) are the two register stages, each requested an iteration before its commit. (Three stages
        // per buffer, in the third free plane, measured slower.)
        OA a1 = a;
        OB b1 = b;
        auto fetch_to = [&](OA& x, OB& y, int j) {
            const int q = j + rot;
            const int k0 = kb + (q >= nfull ? q - nfull : q) * BKQ;
            x.full(k0);
            y.full(k0);
        };
        fetch_to(a, b, 0);
        fetch_to(a1, b1, 1);
        a.template store<NP>(smem[0][0], tid, sa);
        b.template store<NP>(smem[0][1], tid, sb);
        a1.template store<NP>(smem[0][0] + STAGE_W, tid, sa);
        b1.template store<NP>(smem[0][1] + STAGE_W, tid, sb);
        fetch_to(a, b, min(2, nfull - 1));
        fetch_to(a1, b1, min(3, nfull - 1));
        lds_barrier();
        for (int j = 0; j < nfull; j += 2) {
            const int cur = (j >> 1) & 1;
            mma_stage_w<NP>(smem[cur][0], smem[cur][1], acc, wm, wn, lr, half);
            a.template store<NP>(smem[cur ^ 1][0], tid, sa);
            b.template store<NP>(smem[cur ^ 1][1], tid, sb);
            fetch_to(a, b, min(j + 4, nfull - 1));
            if (j + 1 < nfull)  // block-uniform
                mma_stage_w<NP>(smem[cur][0] + STAGE_W, smem[cur][1] + STAGE_W, acc, wm, wn, lr, half);
            a1.template store<NP>(smem[cur ^ 1][0] + STAGE_W, tid, sa);
            b1.template store<NP>(smem[cur ^ 1][1] + STAGE_W, tid, sb);
            fetch_to(a1, b1, min(j + 5, nfull - 1));
            lds_barrier();
        }
    } else if (nfull > 0) {
        fetch(0);
        a.template store<NP>(smem[0][0], tid, sa);
        b.template store<NP>(smem[0][1], tid, sb);
        fetch(min(1, nfull - 1));
        lds_barrier();
        for (int j = 0; j < nfull; ++j) {
            const int cur = j & 1;
            mma_stage_w<NP>(smem[cur][0], smem[cur][1], acc, wm, wn, lr, half);
            a.template store<NP>(smem[cur ^ 1][0], tid, sa);
            b.template store<NP>(smem[cur ^ 1][1], tid, sb);
            fetch(min(j + 2, nfull - 1));
            lds_barrier();
        }
    }
    if (len % BKQ != 0) {
        a.tail(kb + nfull * BKQ, ke);
        b.tail(kb + nfull * BKQ, ke);
        a.template store<NP>(smem[0][0], tid, sa);
        b.template store<NP>(smem[0][1], tid, sb);
        lds_barrier();
        mma_stage_w<NP>(smem[0][0], smem[0][1], acc, wm, wn, lr, half);
        lds_barrier();
    }
}

// A wide partial tile in lane order: group q = 16s + 8i + 4j + r4 holds elements 4·r4 … 4·r4 + 3 of
// acc[s][i][j], [q][thread][4].
__device__ __forceinline__ void write_partial_w(float* slot, const f32x16 (&acc)[2][2][2]) {
#pragma unroll
    for (int q = 0; q < 32; ++q) {
        const int s = q >> 4, i = (q >> 3) & 1, j = (q >> 2) & 1, r = (q & 3) * 4;
        *reinterpret_cast<f32x4*>(slot + (q * WT_THREADS + threadIdx.x) * 4) =
            f32x4{acc[s][i][j][r], acc[s][i][j][r + 1], acc[s][i][j][r + 2], acc[s][i][j][r + 3]};
    }
}

// nn and tn carry wide tile counts (tiles_m, tiles_n of 256 x 256 tiles); s counts 16-deep units.
// NP = 3: split products (fp32); NP = 2: two-piece fp16 products (fp32-accurate; nn.amax_a = max|dY|,
// nn.amax_b = max|W|, tn.amax_b = max|x|); NP = 1: bf16 products (the bf16 policies of both backward
// classes).
// RES: dX = dY·W + nn.R (the residual may be dX itself: each element is read and written by one lane).
// BH (NP = 1): W and x are read from their bf16 copies (nn.B16, tn.B16).
template <int NP, bool RES, bool BH = false>
__global__ __launch_bounds__(WT_THREADS, 1) void gemm_pair_wide_kernel(GemmParams nn, GemmParams tn, PairPlan s) {
    static_assert(NP == 1 || !BH, "bf16 copies feed bf16 products");
    PairScales px, pw;  // dX = dY·W, dW = dYᵀ·x
    if constexpr (NP == 2) {
        px = PairScales(nn.amax_a, nn.amax_b);
        pw = PairScales(nn.amax_a, tn.amax_b);
    }
    unsigned am = 0;  // max|dX| of the lane's stores, when the product keeps dX's magnitude word
    __shared__ __attribute__((aligned(16))) __bf16 smem[2][2][3 * STAGE_W];
    const int g = xcd_logical_block();
    const int count = s.q + (g < s.r ? 1 : 0);
    for (int n = 0; n < count; ++n) {
        // The lane's coordinates are taken afresh for each tile: derived from a value the compiler cannot
        // see through, the epilogue's per-lane store offsets are not hoisted out of the loop and spilled.
        const int tid = opaque_tid(), lane = tid & 63, wave = tid >> 6;
        const int wm = wave >> 2, wn = wave & 3, lr = lane & 31, half = lane >> 5;
        const int t = g + n * s.G, tm = t / nn.tiles_n;
        TileCoord c;
        c.split = 0;
        c.t = t;
        c.m0 = tm * WT;
        c.n0 = (t - tm * nn.tiles_n) * WT;
        c.kb = 0;
        c.ke = nn.K;
        OperandWK a(nn.A, nn.lda, c.m0, nn.M, tid, (unsigned)(nn.M * nn.lda * 4));
        typename WideS<BH>::T b = WideS<BH>::make(nn.B, nn.B16, nn.ldb, c.n0, nn.N, tid, nn.K);
        f32x16 acc[2][2][2];
        wide_mma<NP>(a, b, 0, nn.K, t, smem, acc, tid, wm, wn, lr, half, px.sa, px.sb);
        if constexpr (NP == 2) px.unscale(acc);
        // The epilogue's lane coordinates are taken again after the K loop, so its store offsets are
        // computed here rather than before the loop (where they would be held, spilled, across it).
        const int te = opaque_tid(), le = te & 63, we = te >> 6;
        // With a residual to read, the second subtile's accumulators wait in LDS (the stages are done:
        // wide_mma ends on a barrier), each thread in its own slots, during the first subtile's epilogue.
        f32x16* park = reinterpret_cast<f32x16*>(&smem[0][0][0]);
        if constexpr (RES) {
#pragma unroll
            for (int q = 0; q < 4; ++q) park[q * WT_THREADS + te] = acc[1][q >> 1][q & 1];
        }
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            TileCoord cs = c;
            cs.m0 = c.m0 + 128 * h;
            if (cs.m0 >= nn.M) break;
            if (RES && h == 1) {
#pragma unroll
                for (int q = 0; q < 4; ++q) acc[1][q >> 1][q & 1] = park[q * WT_THREADS + te];
            }
            const bool full = cs.m0 + 128 <= nn.M && c.n0 + WT <= nn.N;
            if (NP == 2 && !RES && nn.amax_c) {  // (with a residual the host measures dX afterwards)
                if (full)
                    store_acc<true, true, STORE, RES, false, true, 2, true>(nn, cs, acc[h], we >> 2, we & 3, le & 31,
                                                                           (le >> 5) << 2, &am);
                else
                    store_acc<true, true, STORE, RES, true, true, 2, true>(nn, cs, acc[h], we >> 2, we & 3, le & 31,
                                                                          (le >> 5) << 2, &am);
            } else if (full) {
                store_acc<true, true, STORE, RES, false, true>(nn, cs, acc[h], we >> 2, we & 3, le & 31,
                                                               (le >> 5) << 2);
            } else {
                store_acc<true, true, STORE, RES, true, true>(nn, cs, acc[h], we >> 2, we & 3, le & 31,
                                                              (le >> 5) << 2);
            }
        }
        if constexpr (RES) lds_barrier();  // every park slot is read before the next stages overwrite them
    }
    const int lo = plan_tn_lo(s, g), hi = plan_tn_lo(s, g + 1);
    for (int u = lo; u < hi;) {
        const int tid = opaque_tid(), lane = tid & 63, wave = tid >> 6;
        const int wm = wave >> 2, wn = wave & 3, lr = lane & 31, half = lane >> 5;
        const int t = u / s.tn_units;
        const int a0 = u - t * s.tn_units;
        const int b0 = min(s.tn_units, a0 + (hi - u));
        const int tm = t / tn.tiles_n;
        const int m0 = tm * WT, n0 = (t - tm * tn.tiles_n) * WT;
        OperandWS a(tn.A, tn.lda, m0, tn.M, tid, (unsigned)(tn.K * tn.lda * 4));
        typename WideS<BH>::T b = WideS<BH>::make(tn.B, tn.B16, tn.ldb, n0, tn.N, tid, tn.K);
        f32x16 acc[2][2][2];
        wide_mma<NP>(a, b, a0 * BKQ, min(tn.K, b0 * BKQ), g, smem, acc, tid, wm, wn, lr, half, pw.sa, pw.sb);
        if constexpr (NP == 2) pw.unscale(acc);
        write_partial_w(s.partial + ((long)g * 2 + (u == lo ? 0 : 1)) * (WT * WT), acc);
        u += b0 - a0;
    }
    if constexpr (NP == 2) block_amax_fold(am, nn.amax_c);
}

// dW += the partials of the workers that shared each wide dW tile, summed in worker order. Block (t, q)
// takes group q of tile t. The block first lists the covering workers' slots in worker order (one thread
// per worker, an ordered compaction by wave ballots), then each thread sums its float4 of that group over
// the list, sixteen loads in flight at a time.
__global__ __launch_bounds__(WT_THREADS) void pair_fixup_w_kernel(GemmParams tn, PairPlan s) {
    const int t = blockIdx.x, q = blockIdx.y;
    const int a = t * s.tn_units, b = a + s.tn_units;
    __shared__ int run_lo[FIXUP_MAX_WORKERS + 1];
    __shared__ int slots[FIXUP_MAX_WORKERS];
    __shared__ int wave_count[WT_THREADS / 64];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave >> 2, wn = wave & 3, lr = lane & 31, kh = (lane >> 5) << 2;
    const int sq = q >> 4, i = (q >> 3) & 1, j = (q >> 2) & 1, r4 = q & 3;
    const int tm = t / tn.tiles_n;
    const int row0 = tm * WT + 128 * sq + wm * 64 + 32 * i + 8 * r4 + kh;
    const int col = (t - tm * tn.tiles_n) * WT + wn * 64 + 32 * j + lr;
    // dW's current values are requested first, so their latency overlaps the slot list's set-up and the
    // partials' loads.
    float cur[4];
#pragma unroll
    for (int e = 0; e < 4; ++e)
        cur[e] = col < tn.N && row0 + e < tn.M ? tn.C[(long)(row0 + e) * tn.ldc + col] : 0.0f;
    for (int g = tid; g <= s.G; g += WT_THREADS) run_lo[g] = plan_tn_lo(s, g);
    __syncthreads();
    int base = 0;
    for (int g0 = 0; g0 < s.G; g0 += WT_THREADS) {
        const int g = g0 + tid;
        bool covers = false;
        int slot = 0;
        if (g < s.G) {
            const int glo = run_lo[g], ghi = run_lo[g + 1];
            covers = ghi > glo && glo < b && ghi > a;
            slot = g * 2 + (glo / s.tn_units == t ? 0 : 1);
        }
        const unsigned long long mask = __ballot(covers);
        const int before = __popcll(mask & ((1ull << lane) - 1ull));
        if (lane == 0) wave_count[wave] = __popcll(mask);
        __syncthreads();
        int offset = base;
        for (int w = 0; w < wave; ++w) offset += wave_count[w];
        if (covers) slots[offset + before] = slot;
        for (int w = 0; w < WT_THREADS / 64; ++w) base += wave_count[w];
        __syncthreads();
    }
    const int n = base;
    if (col >= tn.N) return;  // no barrier follows
    const long off = (long)q * WT_THREADS + tid;
    f32x4 sum = f32x4{0, 0, 0, 0};
    for (int k0 = 0; k0 < n; k0 += 16) {
        f32x4 v[16];
#pragma unroll
        for (int k = 0; k < 16; ++k)
            if (k0 + k < n) v[k] = reinterpret_cast<const f32x4*>(s.partial + (long)slots[k0 + k] * (WT * WT))[off];
#pragma unroll
        for (int k = 0; k < 16; ++k)
            if (k0 + k < n) sum += v[k];
    }
#pragma unroll
    for (int e = 0; e < 4; ++e)
        if (row0 + e < tn.M) tn.C[(long)(row0 + e) * tn.ldc + col] = cur[e] + sum[e];
}

// Adds the partials of the workers that shared a dW tile, in worker order, into dW. Eight workgroups
// per tile (blockIdx.y = 4i + r/4): each thread sums the two float4 groups (j = 0, 1) of its lanes'
// accumulator rows and adds them to dW as four column pairs, in the layout `store_acc` uses.
template <bool KLAYOUT>
__global__ __launch_bounds__(THREADS) void pair_fixup_kernel(GemmParams tn, PairPlan s) {
    const int t = blockIdx.x, i = blockIdx.y >> 2, r4 = blockIdx.y & 3;
    const int a = t * s.tn_units, b = a + s.tn_units;
    // Every worker's dW run start, computed once per block in parallel (G ≤ FIXUP_MAX_WORKERS).
    __shared__ int run_lo[FIXUP_MAX_WORKERS + 1];
    for (int g = threadIdx.x; g <= s.G; g += THREADS) run_lo[g] = plan_tn_lo(s, g);
    __syncthreads();
    // First worker whose dW run ends after a (runs are ordered and contiguous).
    int lo = 0, hi = s.G - 1;
    while (lo < hi) {
        const int mid = (lo + hi) >> 1;
        if (run_lo[mid + 1] > a) hi = mid; else lo = mid + 1;
    }
    int covering = 0;
    for (int g = lo; g < s.G && run_lo[g] < b; ++g)
        if (run_lo[g + 1] > run_lo[g]) ++covering;
    if (covering <= 1) return;  // one worker held the whole tile and accumulated it in place

    // The covering workers' partial slots in worker order, in batches of 8 so the loads of a batch are
    // in flight together; the sum order stays the worker order.
    const int tid = threadIdx.x;
    const long off0 = ((2 * i) * 4 + r4) * THREADS + tid, off1 = ((2 * i + 1) * 4 + r4) * THREADS + tid;
    f32x4 sum[2] = {f32x4{0, 0, 0, 0}, f32x4{0, 0, 0, 0}};
    int g = lo;
    while (g < s.G) {
        int slots[8];
        int n = 0;
        for (; g < s.G && n < 8; ++g) {
            const int glo = run_lo[g], ghi = run_lo[g + 1];
            if (glo >= b) {
                g = s.G;
                break;
            }
            if (ghi <= glo || ghi <= a) continue;
            slots[n++] = g * 2 + (glo / s.tn_units == t ? 0 : 1);
        }
        f32x4 v[8][2];
#pragma unroll
        for (int k = 0; k < 8; ++k)
            if (k < n) {
                const f32x4* slot = reinterpret_cast<const f32x4*>(s.partial + (long)slots[k] * (BM * BN));
                v[k][0] = slot[off0];
                v[k][1] = slot[off1];
            }
#pragma unroll
        for (int k = 0; k < 8; ++k)
            if (k < n) {
                sum[0] += v[k][0];
                sum[1] += v[k][1];
            }
    }
    const int lane = tid & 63, wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1, lr = lane & 31, kh = (lane >> 5) << 2;
    const TileCoord c = unit_coord(tn, t, 0, s.tn_units);
    if constexpr (KLAYOUT) {
        // Split-product accumulators: element e of group (i, j, r4) is row 32i + 8·r4 + kh + e, column
        // 32j + lr of the wave's 64×64 block.
        float cur[2][4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {  // all reads before the first write (see store_acc)
            const int row = c.m0 + wm * 64 + 32 * i + 8 * r4 + kh + e;
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                const int col = c.n0 + wn * 64 + 32 * j + lr;
                cur[j][e] = row < tn.M && col < tn.N ? tn.C[(long)row * tn.ldc + col] : 0.0f;
            }
        }
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const int row = c.m0 + wm * 64 + 32 * i + 8 * r4 + kh + e;
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                const int col = c.n0 + wn * 64 + 32 * j + lr;
                if (row < tn.M && col < tn.N) tn.C[(long)row * tn.ldc + col] = cur[j][e] + sum[j][e];
            }
        }
        return;
    }
    const int col = c.n0 + wn * 64 + 2 * lr;
    f32x2 cur[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {  // all reads before the first write (see store_acc)
        const int row = c.m0 + wm * 64 + 2 * (8 * r4 + kh + e) + i;
        cur[e] = row < tn.M && col < tn.N ? *reinterpret_cast<const f32x2*>(tn.C + (long)row * tn.ldc + col)
                                          : f32x2{0.0f, 0.0f};
    }
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        const int row = c.m0 + wm * 64 + 2 * (8 * r4 + kh + e) + i;
        if (row < tn.M && col < tn.N)
            *reinterpret_cast<f32x2*>(tn.C + (long)row * tn.ldc + col) = cur[e] + f32x2{sum[0][e], sum[1][e]};
    }
}

// ------------------------------------------------------------------------------ generic kernel

// Loads one 128×32 operand tile into 4 float4 registers per thread, testing every element.
template <bool KCONTIG>
__device__ __forceinline__ void load_tile_checked(const float* __restrict__ src, long ld, int mn0, int MN, int k0,
                                                  int kend, bool vec, f32x4 (&reg)[4], int tid) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        int idx = tid + THREADS * i;
        if (KCONTIG) {
            int mn = mn0 + (idx >> 3);
            int k = k0 + ((idx & 7) << 2);
            if (vec && mn < MN && k + 3 < kend) {
                reg[i] = *reinterpret_cast<const f32x4*>(src + (long)mn * ld + k);
            } else {
#pragma unroll
                for (int e = 0; e < 4; ++e) reg[i][e] = (mn < MN && k + e < kend) ? src[(long)mn * ld + k + e] : 0.0f;
            }
        } else {
            int k = k0 + (idx >> 5);
            int mn = mn0 + ((idx & 31) << 2);
            if (vec && k < kend && mn + 3 < MN) {
                reg[i] = *reinterpret_cast<const f32x4*>(src + (long)k * ld + mn);
            } else {
#pragma unroll
                for (int e = 0; e < 4; ++e) reg[i][e] = (k < kend && mn + e < MN) ? src[(long)k * ld + mn + e] : 0.0f;
            }
        }
    }
}

// Any shape and alignment; K tiles in natural order; runtime residual.
template <bool AK, bool BKC, int MODE>
__global__ __launch_bounds__(THREADS, 2) void gemm_generic_kernel(GemmParams p) {
    __shared__ __attribute__((aligned(16))) float smem[2][2][STAGE];
    const TileCoord c = tile_coord(p, xcd_logical_block());
    const int nk = c.ke > c.kb ? (c.ke - c.kb + BK - 1) / BK : 0;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    const int lr = lane & 31, kh = (lane >> 5) << 2;

    f32x16 acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) acc[i][j] = f32x16{};
    f32x4 ra[4], rb[4];
    if (nk > 0) {
        load_tile_checked<AK>(p.A, p.lda, c.m0, p.M, c.kb, c.ke, p.vec_a, ra, tid);
        load_tile_checked<BKC>(p.B, p.ldb, c.n0, p.N, c.kb, c.ke, p.vec_b, rb, tid);
        store_tile<AK>(smem[0][0], ra, tid);
        store_tile<BKC>(smem[0][1], rb, tid);
    }
    __syncthreads();
    for (int kt = 0; kt < nk; ++kt) {
        const int cur = kt & 1;
        if (kt + 1 < nk) {
            const int k0 = c.kb + (kt + 1) * BK;
            load_tile_checked<AK>(p.A, p.lda, c.m0, p.M, k0, c.ke, p.vec_a, ra, tid);
            load_tile_checked<BKC>(p.B, p.ldb, c.n0, p.N, k0, c.ke, p.vec_b, rb, tid);
        }
        mma_stage<AK, BKC>(smem[cur][0], smem[cur][1], acc, wm, wn, lr, kh);
        if (kt + 1 < nk) {
            store_tile<AK>(smem[cur ^ 1][0], ra, tid);
            store_tile<BKC>(smem[cur ^ 1][1], rb, tid);
        }
        __syncthreads();
    }
    if (MODE == STORE && p.R)
        store_acc<AK, BKC, MODE, true, true, false>(p, c, acc, wm, wn, lr, kh);
    else
        store_acc<AK, BKC, MODE, false, true, false>(p, c, acc, wm, wn, lr, kh);
}

// ------------------------------------------------------------------------------ reductions

// C[m, n] = (Σ_s P[s][m][n] + bias[n]) + R[m, n], s in order: the epilogue of a stored product whose K
// was split, in the order the unsplit epilogue adds (R may be C itself: one thread reads and writes each
// element).
__global__ void splitk_store_kernel(const float* __restrict__ P, int splits, int M, int N, float* C, long ldc,
                                    const float* __restrict__ bias, const float* R, long ldr) {
    const long total = (long)M * N;
    for (long i = blockIdx.x * (long)blockDim.x + threadIdx.x; i < total; i += (long)gridDim.x * blockDim.x) {
        float s = 0.0f;
        for (int k = 0; k < splits; ++k) s += P[(long)k * total + i];
        const long m = i / N, n = i - m * N;
        if (bias) s += bias[n];
        if (R) s += R[m * ldr + n];
        C[m * ldc + n] = s;
    }
}

// C[m, n] += Σ_s P[s][m][n], s in order.
__global__ void splitk_reduce_kernel(const float* __restrict__ P, int splits, int M, int N, float* C, long ldc) {
    const long total = (long)M * N;
    for (long i = blockIdx.x * (long)blockDim.x + threadIdx.x; i < total; i += (long)gridDim.x * blockDim.x) {
        float s = 0.0f;
        for (int k = 0; k < splits; ++k) s += P[(long)k * total + i];
        const long m = i / N, n = i - m * N;
        C[m * ldc + n] += s;
    }
}

// The same two sums, four consecutive columns per thread (N, ldc and ldr multiples of 4, 16-byte aligned arrays),
// the partial loads of several splits in flight at once; the per-element order of the additions is unchanged.
__device__ __forceinline__ f32x4 splitk_sum4(const float* __restrict__ P, int splits, long total, long e) {
    f32x4 s = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll 4
    for (int k = 0; k < splits; ++k) s += *reinterpret_cast<const f32x4*>(P + (long)k * total + e);
    return s;
}

// amax (optional): max|C| folded in (C's magnitude word).
__global__ void splitk_store4_kernel(const float* __restrict__ P, int splits, int M, int N, float* C, long ldc,
                                     const float* __restrict__ bias, const float* R, long ldr, unsigned* amax) {
    const long total = (long)M * N, quads = total >> 2;
    unsigned am = 0;
    for (long i = blockIdx.x * (long)blockDim.x + threadIdx.x; i < quads; i += (long)gridDim.x * blockDim.x) {
        const long e = i * 4, m = e / N, n = e - m * N;
        f32x4 s = splitk_sum4(P, splits, total, e);
        if (bias) s += *reinterpret_cast<const f32x4*>(bias + n);
        if (R) s += *reinterpret_cast<const f32x4*>(R + m * ldr + n);
        *reinterpret_cast<f32x4*>(C + m * ldc + n) = s;
        am = max(am, amax_bits4(s));
    }
    block_amax_fold(am, amax);
}

__global__ void splitk_reduce4_kernel(const float* __restrict__ P, int splits, int M, int N, float* C, long ldc) {
    const long total = (long)M * N, quads = total >> 2;
    for (long i = blockIdx.x * (long)blockDim.x + threadIdx.x; i < quads; i += (long)gridDim.x * blockDim.x) {
        const long e = i * 4, m = e / N, n = e - m * N;
        const f32x4 s = splitk_sum4(P, splits, total, e);
        f32x4* c = reinterpret_cast<f32x4*>(C + m * ldc + n);
        *c = *c + s;
    }
}

// The split-K epilogue of the QKV projection with RoPE (gemm_rope on 128 x 128 tiles): each thread takes V
// consecutive rotation pairs (columns 64h + d … and 64h + d + 32 … of row m, V = 4 with float4 access), sums
// their partials in split order and adds the bias (splitk_store_kernel's order), rotates each pair when it
// lies in the first rope_cols columns (the STORE_ROPE epilogue's arithmetic: a·cos − b·sin, b·cos + a·sin at
// the row's position) and stores them; amax (optional) receives max|C|. N a multiple of 64.
template <int V>
__global__ __launch_bounds__(256) void splitk_store_rope_kernel(const float* __restrict__ P, int splits, int M, int N,
                                                                float* __restrict__ C, const float* __restrict__ bias,
                                                                const int* __restrict__ pos,
                                                                const float* __restrict__ cos_t,
                                                                const float* __restrict__ sin_t, int rope_cols,
                                                                unsigned* amax) {
    typedef float vec __attribute__((ext_vector_type(V)));
    const long total = (long)M * N, units = total / (2 * V);
    const int per_row = N / (2 * V), per_head = 32 / V;
    unsigned am = 0;
    for (long i = blockIdx.x * (long)blockDim.x + threadIdx.x; i < units; i += (long)gridDim.x * blockDim.x) {
        const long m = i / per_row;
        const int r = (int)(i - m * per_row), d = (r % per_head) * V, c0 = (r / per_head) * 64 + d, c1 = c0 + 32;
        const long e0 = m * N + c0, e1 = m * N + c1;
        vec a = {}, b = {};
        for (int k = 0; k < splits; ++k) {
            a += *reinterpret_cast<const vec*>(P + (long)k * total + e0);
            b += *reinterpret_cast<const vec*>(P + (long)k * total + e1);
        }
        if (bias) {
            a += *reinterpret_cast<const vec*>(bias + c0);
            b += *reinterpret_cast<const vec*>(bias + c1);
        }
        vec v0 = a, v1 = b;
        if (c0 < rope_cols) {
            const int q = pos[m];
            const vec cs = *reinterpret_cast<const vec*>(cos_t + q * 32 + d);
            const vec sn = *reinterpret_cast<const vec*>(sin_t + q * 32 + d);
            v0 = a * cs - b * sn;
            v1 = b * cs + a * sn;
        }
        *reinterpret_cast<vec*>(C + e0) = v0;
        *reinterpret_cast<vec*>(C + e1) = v1;
#pragma unroll
        for (int j = 0; j < V; ++j) am = max(am, max(amax_bits(v0[j]), amax_bits(v1[j])));
    }
    block_amax_fold(am, amax);
}

__global__ void column_sum_kernel(const float* __restrict__ x, int rows, int n, float* out) {
    // One thread per column; rows summed in order (bias gradients are small: n ≤ a few thousand).
    const int c = blockIdx.x * blockDim.x + threadIdx.x;
    if (c >= n) return;
    float s = 0.0f;
    for (int r = 0; r < rows; ++r) s += x[(long)r * n + c];
    out[c] += s;
}

__global__ void column_partial_kernel(const float* __restrict__ x, int rows, int n, int rows_per, float* part) {
    const int c = blockIdx.x * blockDim.x + threadIdx.x;
    const int chunk = blockIdx.y;
    if (c >= n) return;
    const int r0 = chunk * rows_per, r1 = min(rows, r0 + rows_per);
    float s = 0.0f;
    for (int r = r0; r < r1; ++r) s += x[(long)r * n + c];
    part[(long)chunk * n + c] = s;
}

__global__ void column_reduce_kernel(const float* __restrict__ part, int chunks, int n, float* out) {
    const int c = blockIdx.x * blockDim.x + threadIdx.x;
    if (c >= n) return;
    float s = 0.0f;
    for (int k = 0; k < chunks; ++k) s += part[(long)k * n + c];
    out[c] += s;
}

// ------------------------------------------------------------------------------ host side

inline bool aligned16(const void* ptr) { return ((uintptr_t)ptr & 15u) == 0; }
inline bool aligned8(const void* ptr) { return ((uintptr_t)ptr & 7u) == 0; }

// The main kernel's requirements for operand `src` (extent `mn` × K, contiguous along K when kcontig).
bool operand_fast(const float* src, long ld, bool vec, bool kcontig, int mn, int K) {
    const long contiguous = kcontig ? K : mn;
    const long lines = kcontig ? mn : K;
    return vec && contiguous % 4 == 0 && contiguous >= 4 && lines >= 1 && ld >= contiguous &&
           (lines - 1) * ld + contiguous < (1L << 31) && src != nullptr;
}

bool gemm_fast(const GemmParams& p, bool ak, bool bkc) {
    // An mn-contiguous B makes the epilogue store column pairs (float2): C, R and bias must allow it.
    const bool pairs_ok = bkc || (p.ldc % 2 == 0 && aligned8(p.C) && (p.R == nullptr || (p.ldr % 2 == 0 && aligned8(p.R))) &&
                                  (p.bias == nullptr || aligned8(p.bias)));
    return operand_fast(p.A, p.lda, p.vec_a, ak, p.M, p.K) && operand_fast(p.B, p.ldb, p.vec_b, bkc, p.N, p.K) &&
           (long)p.M * p.ldc < (1L << 31) && (p.R == nullptr || (long)p.M * p.ldr < (1L << 31)) && pairs_ok;
}

// The bf16 kernel reads an mn-contiguous operand, or a k-contiguous one without float4 access, one
// element at a time: it takes every shape whose offsets fit in 32 bits.
bool gemm_fits_h(const GemmParams& p, bool ak, bool bkc) {
    auto fits = [](const float* src, long ld, bool kcontig, int mn, int K) {
        const long last = kcontig ? (long)(mn - 1) * ld + K : (long)(K - 1) * ld + mn;
        return src != nullptr && K >= 1 && mn >= 1 && ld >= (kcontig ? K : mn) && last < (1L << 31);
    };
    return fits(p.A, p.lda, ak, p.M, p.K) && fits(p.B, p.ldb, bkc, p.N, p.K) && (long)p.M * p.ldc < (1L << 31) &&
           (p.R == nullptr || (long)p.M * p.ldr < (1L << 31));
}

template <int AOP, int BOP> void launch_h(laya_ctx* ctx, const GemmParams& p, int blocks) {
    const dim3 g(blocks), b(THREADS);
    switch (p.mode) {
        case STORE:
            if (p.R)
                LAYA_LAUNCH((gemm_bf16_kernel<AOP, BOP, STORE, true>), g, b, 0, ctx->stream, p);
            else
                LAYA_LAUNCH((gemm_bf16_kernel<AOP, BOP, STORE, false>), g, b, 0, ctx->stream, p);
            break;
        case ACCUMULATE:
            LAYA_LAUNCH((gemm_bf16_kernel<AOP, BOP, ACCUMULATE, false>), g, b, 0, ctx->stream, p);
            break;
        default: LAYA_LAUNCH((gemm_bf16_kernel<AOP, BOP, PARTIAL, false>), g, b, 0, ctx->stream, p);
    }
    check_launch("gemm_bf16_kernel");
}

// Picks the operand forms of a bf16 product (float4 access for a k-contiguous operand where it is allowed).
bool wide_tiles_pay(const laya_ctx* ctx, const GemmParams& p, bool three);
void launch_wide_h(laya_ctx* ctx, GemmParams p);

template <bool AK, bool BKC> void launch_bf16(laya_ctx* ctx, const GemmParams& p, int blocks) {
    const bool va = AK && operand_fast(p.A, p.lda, p.vec_a, true, p.M, p.K);
    const bool vb = BKC && operand_fast(p.B, p.ldb, p.vec_b, true, p.N, p.K);
    if constexpr (AK && BKC) {
        if (va && vb && wide_tiles_pay(ctx, p, false)) launch_wide_h(ctx, p);
        else if (va && vb) launch_h<KVEC, KVEC>(ctx, p, blocks);
        else if (va) launch_h<KVEC, KSCALAR>(ctx, p, blocks);
        else if (vb) launch_h<KSCALAR, KVEC>(ctx, p, blocks);
        else launch_h<KSCALAR, KSCALAR>(ctx, p, blocks);
    } else if constexpr (AK) {
        if (va) launch_h<KVEC, MNSCALAR>(ctx, p, blocks);
        else launch_h<KSCALAR, MNSCALAR>(ctx, p, blocks);
    } else {
        static_assert(!BKC, "no TN-with-k-contiguous-B layout");
        launch_h<MNSCALAR, MNSCALAR>(ctx, p, blocks);
    }
}

// The precision class of a layout: NT forward (bit 0), NN input gradient (bit 1), TN weight gradient (bit 2).
constexpr int layout_bit(bool ak, bool bkc) { return ak && bkc ? 1 : ak ? 2 : 4; }

// Three single-stage workgroups per CU when the tile count makes that fewer rounds of work: a round of
// three shares each CU's matrix cores three ways, so it is worth 1.5 rounds of two.
bool three_per_cu(const laya_ctx* ctx, int blocks) {
    const long two = (blocks + 2L * ctx->cu_count - 1) / (2L * ctx->cu_count);
    const long three = (blocks + 3L * ctx->cu_count - 1) / (3L * ctx->cu_count);
    return 3 * three < 2 * two;
}

// 256 x 256 tiles when their rounds take less time than the 128 x 128 grid's (two or three per CU): one
// wide tile per CU is four 128 x 128 tiles of work done ≈ 13 % faster (measured on 13871 x 2304 x 768).
// A whole-K NT product without residual, K a multiple of 16; `three` when the three-per-CU kernel would
// take the 128 x 128 grid.
bool wide_tiles_pay(const laya_ctx* ctx, const GemmParams& p, bool three) {
    if (p.mode != STORE && p.mode != STORE_ROPE) return false;
    if (p.R || p.K <= 0 || p.K % BKQ != 0 || p.splits != 1) return false;
    if ((long)p.M * p.lda * 4 >= (1L << 31) || (long)p.N * p.ldb * 4 >= (1L << 31)) return false;  // buffer offsets
    const long cu = ctx->cu_count;
    const long wide = (long)((p.M + WT - 1) / WT) * ((p.N + WT - 1) / WT);
    const long tiles = (long)p.tiles_m * p.tiles_n;
    const double t_wide = (double)((wide + cu - 1) / cu) * 4.0 / 1.13;
    const double t_two = (double)((tiles + 2 * cu - 1) / (2 * cu)) * 2.0;
    const double t_three = (double)((tiles + 3 * cu - 1) / (3 * cu)) * 3.0 / 1.08;
    return t_wide < (three ? std::min(t_two, t_three) : t_two);
}

// 192 x 256 tiles when their rounds take less time than the 128 x 128 grid's at two or (STORE only)
// three per CU (the same work per CU per round, done faster by the larger tile: the factor is measured
// on 13871 x 768 x 768). A whole-K NT STORE (residual allowed) or STORE_ROPE, K a multiple of 16.
bool tall_tiles_pay(const laya_ctx* ctx, const GemmParams& p) {
    if ((p.mode != STORE && p.mode != STORE_ROPE) || p.K <= 0 || p.K % BKQ != 0 || p.splits != 1) return false;
    if (p.mode == STORE_ROPE && p.R) return false;
    if ((long)p.M * p.lda * 4 >= (1L << 31) || (long)p.N * p.ldb * 4 >= (1L << 31)) return false;  // buffer offsets
    const long cu = ctx->cu_count;
    const long tall = (long)((p.M + TM - 1) / TM) * ((p.N + WT - 1) / WT);
    const long tiles = (long)p.tiles_m * p.tiles_n;
    const double t_tall = (double)((tall + cu - 1) / cu) * 3.0 / TALL_GAIN;
    const double t_two = (double)((tiles + 2 * cu - 1) / (2 * cu)) * 2.0;
    const double t_three = p.mode == STORE ? (double)((tiles + 3 * cu - 1) / (3 * cu)) * 3.0 / 1.08 : 1e30;
    return t_tall < std::min(t_two, t_three);
}

// Several tensors' magnitudes in one launch: block b covers elements [off[b], off[b] + len[b]) of the
// arena (16-byte aligned, len a multiple of 4 but for a tensor's last block) and folds them into word group
// word[b] of `words`.
__global__ __launch_bounds__(256) void absmax_multi_kernel(const float* __restrict__ arena, const long* __restrict__ off,
                                                           const int* __restrict__ len, const int* __restrict__ word,
                                                           unsigned* words) {
    const long o = off[blockIdx.x];
    const int n = len[blockIdx.x];
    const f32x4* x4 = reinterpret_cast<const f32x4*>(arena + o);
    unsigned m = 0;
    for (int i = threadIdx.x; i < n / 4; i += 256) m = max(m, amax_bits4(x4[i]));
    for (int i = (n / 4) * 4 + threadIdx.x; i < n; i += 256) m = max(m, amax_bits(arena[o + i]));
    block_amax_fold(m, words + (long)word[blockIdx.x] * AMAX_GROUP);
}

}  // namespace

void absmax_multi(laya_ctx* ctx, const float* arena, const long* off, const int* len, const int* word, int blocks,
                  unsigned* words, double bytes) {
    if (blocks <= 0) return;
    ProfileScope scope(ctx, "absmax", 0.0, bytes);
    LAYA_LAUNCH(absmax_multi_kernel, dim3(blocks), dim3(256), 0, ctx->stream, arena, off, len, word, words);
    check_launch("absmax_multi_kernel");
}

// max|x| of a rows x cols operand folded into *out (0 beforehand for the operand's own maximum).
void absmax_into(laya_ctx* ctx, const float* x, int rows, int cols, long ld, unsigned* out) {
    const long n = (long)rows * cols;
    if (n <= 0) return;
    ProfileScope scope(ctx, "absmax", 0.0, 4.0 * n);
    const int vec = cols % 4 == 0 && ld % 4 == 0 && aligned16(x);
    const long per_block = 256L * 4 * 8;  // eight float4 per thread
    const int blocks = (int)std::max(1L, std::min<long>(AMAX_BLOCKS, (n + per_block - 1) / per_block));
    LAYA_LAUNCH(absmax_kernel, dim3(vec && ld == cols ? blocks : std::min(blocks, std::max(rows, 1))),
                       dim3(256), 0, ctx->stream, x, rows, cols, ld, vec, out);
    check_launch("absmax_kernel");
}

namespace {

// max|x| of a rows x cols operand into the context's next word group; returns it. `slot` names the operand's
// role for the callers' bookkeeping only.
const unsigned* operand_absmax(laya_ctx* ctx, int slot, const float* x, int rows, int cols, long ld) {
    (void)slot;
    unsigned* out = operand_ring_word(ctx);
    absmax_into(ctx, x, rows, cols, ld, out);
    return out;
}

// The magnitude word of an operand: the caller's (measured now if it is not known yet: an unknown word
// holds zero) or the context's slot `slot`, measured now.
const unsigned* operand_amax(laya_ctx* ctx, AmaxRef r, int slot, const float* x, int rows, int cols, long ld) {
    if (!r.word) return operand_absmax(ctx, slot, x, rows, cols, ld);
    if (!*r.known) {
        absmax_into(ctx, x, rows, cols, ld, r.word);
        *r.known = 1;
    }
    return r.word;
}

// An NT product on 256-wide tiles (wide or tall) as two-piece fp16 products: both operands' magnitudes
// are taken first (outside the product's profile scope) and the launchers below see amax_a set.
void prepare_pair_nt(laya_ctx* ctx, GemmParams& p, AmaxRef ra, AmaxRef rb) {
    p.amax_a = operand_amax(ctx, ra, 0, p.A, p.M, p.K, p.lda);
    p.amax_b = operand_amax(ctx, rb, 1, p.B, p.N, p.K, p.ldb);
    p.b_one = rb.bf16 ? 1 : 0;
}

void launch_tall(laya_ctx* ctx, GemmParams p) {
    p.tiles_m = (p.M + TM - 1) / TM;
    p.tiles_n = (p.N + WT - 1) / WT;
    const dim3 g(p.tiles_m * p.tiles_n), b(WT_THREADS);
    if (p.amax_a && p.b_one) {
        profile_rename("gemm_nt_h2b1t");
        if (p.mode == STORE_ROPE)
            LAYA_LAUNCH((gemm_x6t_kernel<STORE_ROPE, false, 2, true>), g, b, 0, ctx->stream, p);
        else if (p.R)
            LAYA_LAUNCH((gemm_x6t_kernel<STORE, true, 2, true>), g, b, 0, ctx->stream, p);
        else
            LAYA_LAUNCH((gemm_x6t_kernel<STORE, false, 2, true>), g, b, 0, ctx->stream, p);
        check_launch("gemm_x6t_kernel");
        return;
    }
    if (p.amax_a) {
        profile_rename("gemm_nt_h2t");
        if (p.mode == STORE_ROPE)
            LAYA_LAUNCH((gemm_x6t_kernel<STORE_ROPE, false, 2>), g, b, 0, ctx->stream, p);
        else if (p.R)
            LAYA_LAUNCH((gemm_x6t_kernel<STORE, true, 2>), g, b, 0, ctx->stream, p);
        else
            LAYA_LAUNCH((gemm_x6t_kernel<STORE, false, 2>), g, b, 0, ctx->stream, p);
        check_launch("gemm_x6t_kernel");
        return;
    }
    profile_rename("gemm_nt_x6t");
    if (p.mode == STORE_ROPE)
        LAYA_LAUNCH((gemm_x6t_kernel<STORE_ROPE, false>), g, b, 0, ctx->stream, p);
    else if (p.R)
        LAYA_LAUNCH((gemm_x6t_kernel<STORE, true>), g, b, 0, ctx->stream, p);
    else
        LAYA_LAUNCH((gemm_x6t_kernel<STORE, false>), g, b, 0, ctx->stream, p);
    check_launch("gemm_x6t_kernel");
}

void launch_wide(laya_ctx* ctx, GemmParams p) {
    p.tiles_n = (p.N + WT - 1) / WT;
    const dim3 g(((p.M + WT - 1) / WT) * p.tiles_n), b(WT_THREADS);
    if (p.amax_a) {
        profile_rename(p.b_one ? "gemm_nt_h2b1w" : "gemm_nt_h2w");
        if (p.mode == STORE_ROPE && p.b_one)
            LAYA_LAUNCH((gemm_x6w_kernel<STORE_ROPE, 2, false, false, true>), g, b, 0, ctx->stream, p);
        else if (p.mode == STORE_ROPE)
            LAYA_LAUNCH((gemm_x6w_kernel<STORE_ROPE, 2>), g, b, 0, ctx->stream, p);
        else if (p.b_one)
            LAYA_LAUNCH((gemm_x6w_kernel<STORE, 2, false, false, true>), g, b, 0, ctx->stream, p);
        else
            LAYA_LAUNCH((gemm_x6w_kernel<STORE, 2>), g, b, 0, ctx->stream, p);
        check_launch("gemm_x6w_kernel");
        // With a bias the RoPE epilogue does not fold C's magnitude (or a bound on it) in: measure it here.
        if (p.mode == STORE_ROPE && p.amax_c && p.bias) absmax_into(ctx, p.C, p.M, p.N, p.ldc, p.amax_c);
        return;
    }
    profile_rename("gemm_nt_x6w");
    if (p.mode == STORE_ROPE)
        LAYA_LAUNCH((gemm_x6w_kernel<STORE_ROPE>), g, b, 0, ctx->stream, p);
    else
        LAYA_LAUNCH((gemm_x6w_kernel<STORE>), g, b, 0, ctx->stream, p);
    check_launch("gemm_x6w_kernel");
}

// The bf16 NT product on 256 x 256 tiles, reading whichever operands have bf16 copies.
void launch_wide_h(laya_ctx* ctx, GemmParams p) {
    profile_rename("gemm_nt_bf16w");
    p.tiles_n = (p.N + WT - 1) / WT;
    const dim3 g(((p.M + WT - 1) / WT) * p.tiles_n), b(WT_THREADS);
    const bool ah = p.A16 != nullptr, bh = p.B16 != nullptr;
#define WIDE_H(MODE)                                                                                         \
    if (ah && bh)                                                                                            \
        LAYA_LAUNCH((gemm_x6w_kernel<MODE, 1, true, true>), g, b, 0, ctx->stream, p);                 \
    else if (ah)                                                                                             \
        LAYA_LAUNCH((gemm_x6w_kernel<MODE, 1, true, false>), g, b, 0, ctx->stream, p);                \
    else if (bh)                                                                                             \
        LAYA_LAUNCH((gemm_x6w_kernel<MODE, 1, false, true>), g, b, 0, ctx->stream, p);                \
    else                                                                                                     \
        LAYA_LAUNCH((gemm_x6w_kernel<MODE, 1, false, false>), g, b, 0, ctx->stream, p);
    if (p.mode == STORE_ROPE) {
        WIDE_H(STORE_ROPE)
    } else {
        WIDE_H(STORE)
    }
#undef WIDE_H
    check_launch("gemm_x6w_kernel");
}

template <int AOP, int BOP> void launch_x(laya_ctx* ctx, const GemmParams& p, int blocks) {
    const dim3 g(blocks), b(THREADS);
    // Two-piece NN (dX = dY·W) and TN (dW += dYᵀ·X) products on 128 x 128 tiles: the backward of a linear
    // whose rows are too few for the 256-wide pair.
    if constexpr (AOP == KVEC && BOP == MNSCALAR) {
        if (p.amax_a) {
            profile_rename("gemm_nn_h2");
            if (p.mode == STORE && p.R)
                LAYA_LAUNCH((gemm_x6_kernel<KVEC, MNSCALAR, STORE, true, 2>), g, b, 0, ctx->stream, p);
            else if (p.mode == STORE)
                LAYA_LAUNCH((gemm_x6_kernel<KVEC, MNSCALAR, STORE, false, 2>), g, b, 0, ctx->stream, p);
            else if (p.mode == PARTIAL)
                LAYA_LAUNCH((gemm_x6_kernel<KVEC, MNSCALAR, PARTIAL, false, 2>), g, b, 0, ctx->stream, p);
            else
                LAYA_LAUNCH((gemm_x6_kernel<KVEC, MNSCALAR, ACCUMULATE, false, 2>), g, b, 0, ctx->stream, p);
            check_launch("gemm_x6_kernel");
            return;
        }
    }
    if constexpr (AOP == MNSCALAR && BOP == MNSCALAR) {
        if (p.amax_a && !p.R && p.mode != STORE) {
            profile_rename("gemm_tn_h2");
            if (p.mode == PARTIAL)
                LAYA_LAUNCH((gemm_x6_kernel<MNSCALAR, MNSCALAR, PARTIAL, false, 2>), g, b, 0, ctx->stream, p);
            else
                LAYA_LAUNCH((gemm_x6_kernel<MNSCALAR, MNSCALAR, ACCUMULATE, false, 2>), g, b, 0, ctx->stream, p);
            check_launch("gemm_x6_kernel");
            return;
        }
    }
    if constexpr (AOP == KVEC && BOP == KVEC) {
        if (p.amax_a) {  // two-piece products (NT, float4 operands)
            profile_rename(p.mode == STORE && p.b_one ? "gemm_nt_h2b1" : "gemm_nt_h2");
            switch (p.mode) {
                case STORE:
                    if (p.R && p.b_one)
                        LAYA_LAUNCH((gemm_x6_kernel<KVEC, KVEC, STORE, true, 2, true>), g, b, 0, ctx->stream, p);
                    else if (p.R)
                        LAYA_LAUNCH((gemm_x6_kernel<KVEC, KVEC, STORE, true, 2>), g, b, 0, ctx->stream, p);
                    else if (p.b_one)
                        LAYA_LAUNCH((gemm_x6_kernel<KVEC, KVEC, STORE, false, 2, true>), g, b, 0, ctx->stream, p);
                    else
                        LAYA_LAUNCH((gemm_x6_kernel<KVEC, KVEC, STORE, false, 2>), g, b, 0, ctx->stream, p);
                    break;
                case ACCUMULATE:
                    LAYA_LAUNCH((gemm_x6_kernel<KVEC, KVEC, ACCUMULATE, false, 2>), g, b, 0, ctx->stream, p);
                    break;
                default: LAYA_LAUNCH((gemm_x6_kernel<KVEC, KVEC, PARTIAL, false, 2>), g, b, 0, ctx->stream, p);
            }
            check_launch("gemm_x6_kernel");
            return;
        }
    }
    switch (p.mode) {
        case STORE:
            if (p.R)
                LAYA_LAUNCH((gemm_x6_kernel<AOP, BOP, STORE, true>), g, b, 0, ctx->stream, p);
            else
                LAYA_LAUNCH((gemm_x6_kernel<AOP, BOP, STORE, false>), g, b, 0, ctx->stream, p);
            break;
        case ACCUMULATE:
            LAYA_LAUNCH((gemm_x6_kernel<AOP, BOP, ACCUMULATE, false>), g, b, 0, ctx->stream, p);
            break;
        default: LAYA_LAUNCH((gemm_x6_kernel<AOP, BOP, PARTIAL, false>), g, b, 0, ctx->stream, p);
    }
    check_launch("gemm_x6_kernel");
}

// The operand forms of a split product, as for a bf16 one.
template <bool AK, bool BKC> void launch_x6(laya_ctx* ctx, const GemmParams& p, int blocks) {
    const bool va = AK && operand_fast(p.A, p.lda, p.vec_a, true, p.M, p.K);
    const bool vb = BKC && operand_fast(p.B, p.ldb, p.vec_b, true, p.N, p.K);
    if constexpr (AK && BKC) {
        if (va && vb && wide_tiles_pay(ctx, p, p.mode == STORE && three_per_cu(ctx, blocks))) {
            launch_wide(ctx, p);
        } else if (va && vb && tall_tiles_pay(ctx, p)) {
            launch_tall(ctx, p);
        } else if (va && vb && p.mode == STORE && three_per_cu(ctx, blocks)) {
            const dim3 g(blocks), b(THREADS);
            if (p.amax_a) {
                profile_rename("gemm_nt_h2q");
                if (p.R)
                    LAYA_LAUNCH((gemm_x6q_kernel<STORE, true, 2>), g, b, 0, ctx->stream, p);
                else
                    LAYA_LAUNCH((gemm_x6q_kernel<STORE, false, 2>), g, b, 0, ctx->stream, p);
            } else if (p.R) {
                LAYA_LAUNCH((gemm_x6q_kernel<STORE, true>), g, b, 0, ctx->stream, p);
            } else {
                LAYA_LAUNCH((gemm_x6q_kernel<STORE, false>), g, b, 0, ctx->stream, p);
            }
            check_launch("gemm_x6q_kernel");
        } else if (va && vb) launch_x<KVEC, KVEC>(ctx, p, blocks);
        else if (va) launch_x<KVEC, KSCALAR>(ctx, p, blocks);
        else if (vb) launch_x<KSCALAR, KVEC>(ctx, p, blocks);
        else launch_x<KSCALAR, KSCALAR>(ctx, p, blocks);
    } else if constexpr (AK) {
        if (va) launch_x<KVEC, MNSCALAR>(ctx, p, blocks);
        else launch_x<KSCALAR, MNSCALAR>(ctx, p, blocks);
    } else {
        launch_x<MNSCALAR, MNSCALAR>(ctx, p, blocks);
    }
}

template <bool AK, bool BKC> void launch(laya_ctx* ctx, const GemmParams& p, int blocks) {
    const dim3 g(blocks), b(THREADS);
    if (ctx->matmul_bf16 & layout_bit(AK, BKC)) {
        LAYA_REQUIRE(gemm_fits_h(p, AK, BKC), "gemm: bf16 operands need offsets below 2^31");
        launch_bf16<AK, BKC>(ctx, p, blocks);
        return;
    }
    if ((ctx->matmul_split & layout_bit(AK, BKC)) && gemm_fits_h(p, AK, BKC)) {
        launch_x6<AK, BKC>(ctx, p, blocks);
        return;
    }
    if (!gemm_fast(p, AK, BKC)) {
        switch (p.mode) {
            case STORE: LAYA_LAUNCH((gemm_generic_kernel<AK, BKC, STORE>), g, b, 0, ctx->stream, p); break;
            case ACCUMULATE:
                LAYA_LAUNCH((gemm_generic_kernel<AK, BKC, ACCUMULATE>), g, b, 0, ctx->stream, p);
                break;
            default: LAYA_LAUNCH((gemm_generic_kernel<AK, BKC, PARTIAL>), g, b, 0, ctx->stream, p);
        }
        check_launch("gemm_generic_kernel");
        return;
    }
    switch (p.mode) {
        case STORE:
            if (AK && BKC && three_per_cu(ctx, blocks)) {
                if (p.R)
                    LAYA_LAUNCH((gemm3_kernel<AK, BKC, STORE, true>), g, b, 0, ctx->stream, p);
                else
                    LAYA_LAUNCH((gemm3_kernel<AK, BKC, STORE, false>), g, b, 0, ctx->stream, p);
                break;
            }
            if (p.R)
                LAYA_LAUNCH((gemm_kernel<AK, BKC, STORE, true>), g, b, 0, ctx->stream, p);
            else
                LAYA_LAUNCH((gemm_kernel<AK, BKC, STORE, false>), g, b, 0, ctx->stream, p);
            break;
        case ACCUMULATE: LAYA_LAUNCH((gemm_kernel<AK, BKC, ACCUMULATE, false>), g, b, 0, ctx->stream, p); break;
        default: LAYA_LAUNCH((gemm_kernel<AK, BKC, PARTIAL, false>), g, b, 0, ctx->stream, p);
    }
    check_launch("gemm_kernel");
}

GemmParams make_params(int M, int N, int K, const float* A, long lda, const float* B, long ldb, float* C, long ldc,
                       const float* bias, const float* R, long ldr) {
    LAYA_REQUIRE(M >= 0 && N >= 0 && K >= 0, "gemm: negative size");
    GemmParams p{};
    p.A = A;
    p.B = B;
    p.C = C;
    p.bias = bias;
    p.R = R;
    p.lda = lda;
    p.ldb = ldb;
    p.ldc = ldc;
    p.ldr = ldr;
    p.M = M;
    p.N = N;
    p.K = K;
    p.tiles_m = (M + BM - 1) / BM;
    p.tiles_n = (N + BN - 1) / BN;
    p.vec_a = (lda % 4 == 0) && aligned16(A);
    p.vec_b = (ldb % 4 == 0) && aligned16(B);
    p.splits = 1;
    p.k_per_split = std::max(BK, (K + BK - 1) / BK * BK);
    return p;
}

// Splits K into `splits` slices of a multiple of BK; returns the realised split count.
int set_splits(GemmParams& p, int splits) {
    int kps = (p.K + splits - 1) / splits;
    kps = std::max(BK, (kps + BK - 1) / BK * BK);
    p.k_per_split = kps;
    p.splits = std::max(1, (p.K + kps - 1) / kps);
    return p.splits;
}

// An accumulating product: one writer per element (ACCUMULATE), or split-K partials into workspace
// slot 0 (PARTIAL) to be reduced by finish_accumulate.
float* prepare_accumulate(laya_ctx* ctx, GemmParams& p) {
    if (p.splits == 1) {
        p.mode = ACCUMULATE;
        return nullptr;
    }
    p.mode = PARTIAL;
    float* partial = static_cast<float*>(ctx->workspace(0, sizeof(float) * (size_t)p.splits * p.M * p.N));
    float* out = p.C;
    p.C = partial;
    return out;
}

void finish_accumulate(laya_ctx* ctx, const GemmParams& p, float* out, long ldc) {
    if (p.mode != PARTIAL) return;
    const long total = (long)p.M * p.N;
    ProfileScope scope(ctx, "gemm_splitk_reduce", 0.0, 4.0 * total * (p.splits + 2));
    if (p.N % 4 == 0 && ldc % 4 == 0 && aligned16(p.C) && aligned16(out)) {
        LAYA_LAUNCH(splitk_reduce4_kernel, dim3(blocks_for(total / 4, 256, 4096)), dim3(256), 0, ctx->stream, p.C,
                    p.splits, p.M, p.N, out, ldc);
        check_launch("splitk_reduce4_kernel");
        return;
    }
    LAYA_LAUNCH(splitk_reduce_kernel, dim3(blocks_for(total, 256, 4096)), dim3(256), 0, ctx->stream, p.C,
                       p.splits, p.M, p.N, out, ldc);
    check_launch("splitk_reduce_kernel");
}

// K splits for a grid of `tiles` that would not fill one round of two workgroups per CU: as many as fit in
// that round, keeping at least min_k of K per split. A lone workgroup's K loop is latency-bound (about a
// microsecond per 32-deep stage), so splitting K across idle CUs is what shortens such products.
int fill_splits(const laya_ctx* ctx, int tiles, int K, int min_k) {
    const int slots = 2 * ctx->cu_count;
    if (tiles <= 0 || tiles * 2 > slots) return 1;
    return std::max(1, std::min({slots / tiles, K / min_k, 32}));
}

}  // namespace

// Each half of the ring is cleared, in one launch, as the measurements enter it.
unsigned* operand_ring_word(laya_ctx* ctx) {
    static_assert(AMAX_RING % 2 == 0 && AMAX_RING >= 4, "the ring is cleared a half at a time");
    if (!ctx->amax) {
        ctx->amax = static_cast<unsigned*>(ctx->alloc(sizeof(unsigned) * AMAX_RING * AMAX_GROUP));
        ctx->amax_next = 0;
    }
    if (ctx->amax_next % (AMAX_RING / 2) == 0)  // +0.0f is the all-zero word
        fill(ctx, reinterpret_cast<float*>(ctx->amax + (size_t)ctx->amax_next * AMAX_GROUP), 0.0f,
             (size_t)(AMAX_RING / 2) * AMAX_GROUP);
    unsigned* out = ctx->amax + (size_t)ctx->amax_next * AMAX_GROUP;
    ctx->amax_next = (ctx->amax_next + 1) % AMAX_RING;
    return out;
}

const unsigned* operand_amax_ref(laya_ctx* ctx, AmaxRef r, int slot, const float* x, int rows, int cols, long ld) {
    LAYA_REQUIRE(slot >= 0 && slot < AMAX_SLOTS, "operand_amax_ref: no such slot");
    return operand_amax(ctx, r, slot, x, rows, cols, ld);
}

void gemm(laya_ctx* ctx, GemmLayout layout, GemmEpilogue ep, int M, int N, int K, const float* A, long lda,
          const float* B, long ldb, float* C, long ldc, const float* bias, const float* R, long ldr,
          const __bf16* A16, const __bf16* B16, AmaxRef amax_a, AmaxRef amax_b, unsigned* amax_c) {
    if (M == 0 || N == 0) return;
    GemmParams p = make_params(M, N, K, A, lda, B, ldb, C, ldc, bias, R, ldr);
    p.A16 = A16;
    p.B16 = B16;
    const int tiles = p.tiles_m * p.tiles_n;
    float* out = C;
    bool split_store = false;
    if (ep == GemmEpilogue::Accumulate) {
        set_splits(p, fill_splits(ctx, tiles, K, 128));
        out = prepare_accumulate(ctx, p);
    } else {
        p.mode = STORE;
        if (set_splits(p, fill_splits(ctx, tiles, K, 128)) > 1) {
            p.mode = PARTIAL;
            p.C = static_cast<float*>(ctx->workspace(0, sizeof(float) * (size_t)p.splits * M * N));
            split_store = true;
        }
    }
    const int blocks = tiles * p.splits;
    // Every NT product with float4 operands (wide, tall, three-per-CU and generic tiles) takes two-piece
    // products under the pair policy.
    if (layout == GemmLayout::NT && (ctx->matmul_pair & 1) && !(ctx->matmul_bf16 & 1) && (ctx->matmul_split & 1) &&
        gemm_fits_h(p, true, true) && operand_fast(p.A, p.lda, p.vec_a, true, p.M, p.K) &&
        operand_fast(p.B, p.ldb, p.vec_b, true, p.N, p.K)) {
        prepare_pair_nt(ctx, p, amax_a, amax_b);
        // The 128 x 128 kernels do not fold C's magnitude in: it is measured after the product.
        p.amax_c = (wide_tiles_pay(ctx, p, p.mode == STORE && three_per_cu(ctx, blocks)) || tall_tiles_pay(ctx, p))
                       ? amax_c
                       : nullptr;
    }
    // So do NN products with a float4 A (dX = dY·W: launch_x's KVEC x MNSCALAR form) and TN products into an
    // accumulated C (dW += dYᵀ·X) under the input- and weight-gradient pair policies; each operand's
    // magnitude over the array as stored (NN: B is K x N; TN: A is K x M, B is K x N).
    const int cls = layout == GemmLayout::NN ? 2 : 4;
    if (layout != GemmLayout::NT && (ctx->matmul_pair & cls) && !(ctx->matmul_bf16 & cls) &&
        (ctx->matmul_split & cls) && gemm_fits_h(p, layout == GemmLayout::NN, false) &&
        (layout == GemmLayout::TN ? ep == GemmEpilogue::Accumulate
                                  : operand_fast(p.A, p.lda, p.vec_a, true, p.M, p.K))) {
        if (layout == GemmLayout::NN)
            p.amax_a = operand_amax(ctx, amax_a, 0, p.A, p.M, p.K, p.lda);
        else
            p.amax_a = operand_amax(ctx, amax_a, 0, p.A, p.K, p.M, p.lda);
        p.amax_b = operand_amax(ctx, amax_b, 1, p.B, p.K, p.N, p.ldb);
    }
    // C's magnitude: folded in by a two-piece kernel's epilogue, else measured after the product.
    bool measure = amax_c && !p.amax_c;
    {
        static const char* names[3][3] = {{"gemm_nt", "gemm_nn", "gemm_tn"},
                                          {"gemm_nt_bf16", "gemm_nn_bf16", "gemm_tn_bf16"},
                                          {"gemm_nt_x6", "gemm_nn_x6", "gemm_tn_x6"}};
        const int bit = layout == GemmLayout::NT ? 1 : layout == GemmLayout::NN ? 2 : 4;
        const int kind = (ctx->matmul_bf16 & bit) ? 1 : (ctx->matmul_split & bit) ? 2 : 0;
        ProfileScope scope(ctx, names[kind][(int)layout], 2.0 * M * N * (double)K, 0.0);
        switch (layout) {
            case GemmLayout::NT: launch<true, true>(ctx, p, blocks); break;
            case GemmLayout::NN: launch<true, false>(ctx, p, blocks); break;
            case GemmLayout::TN: launch<false, false>(ctx, p, blocks); break;
        }
    }
    if (split_store) {
        const long total = (long)M * N;
        ProfileScope scope(ctx, "gemm_splitk_store", 0.0, 4.0 * total * (p.splits + 1 + (R ? 1 : 0)));
        if (N % 4 == 0 && ldc % 4 == 0 && aligned16(p.C) && aligned16(C) && (!bias || aligned16(bias)) &&
            (!R || (ldr % 4 == 0 && aligned16(R)))) {
            LAYA_LAUNCH(splitk_store4_kernel, dim3(blocks_for(total / 4, 256, 4096)), dim3(256), 0, ctx->stream,
                        p.C, p.splits, M, N, C, ldc, bias, R, ldr, measure ? amax_c : nullptr);
            check_launch("splitk_store4_kernel");
            measure = false;  // folded by the store pass
        } else {
            LAYA_LAUNCH(splitk_store_kernel, dim3(blocks_for(total, 256, 4096)), dim3(256), 0, ctx->stream, p.C,
                        p.splits, M, N, C, ldc, bias, R, ldr);
            check_launch("splitk_store_kernel");
        }
    } else {
        finish_accumulate(ctx, p, out, ldc);
    }
    if (measure) absmax_into(ctx, C, M, N, ldc, amax_c);
}

void gemm_rope(laya_ctx* ctx, int M, int N, int K, const float* A, const float* B, float* C, const float* bias,
               const int* pos, const float* cos_t, const float* sin_t, int rope_cols, const __bf16* A16,
               const __bf16* B16, AmaxRef amax_a, AmaxRef amax_b, unsigned* amax_c) {
    if (M == 0 || N == 0) return;
    GemmParams p = make_params(M, N, K, A, K, B, K, C, N, bias, nullptr, 0);
    [&] {
        p.A16 = A16;
        p.B16 = B16;
        LAYA_REQUIRE(gemm_fast(p, true, true), "gemm_rope: operands must allow the vectorised kernel");
        LAYA_REQUIRE(rope_cols % 64 == 0 && rope_cols <= N && pos && cos_t && sin_t, "gemm_rope: bad rotary layout");
        p.mode = STORE_ROPE;
        p.rope_pos = pos;
        p.rope_cos = cos_t;
        p.rope_sin = sin_t;
        p.rope_cols = rope_cols;
        if (ctx->matmul_bf16 & 1) {
            ProfileScope scope(ctx, "gemm_nt_bf16", 2.0 * M * N * (double)K, 0.0);
            if (wide_tiles_pay(ctx, p, false)) {
                launch_wide_h(ctx, p);
                return;
            }
            LAYA_LAUNCH((gemm_bf16_kernel<KVEC, KVEC, STORE_ROPE, false>), dim3(p.tiles_m * p.tiles_n),
                               dim3(THREADS), 0, ctx->stream, p);
            check_launch("gemm_bf16_kernel");
            return;
        }
        if (ctx->matmul_split & 1) {
            const bool big = wide_tiles_pay(ctx, p, false) || tall_tiles_pay(ctx, p);
            if (ctx->matmul_pair & 1) {
                prepare_pair_nt(ctx, p, amax_a, amax_b);
                p.amax_c = big ? amax_c : nullptr;  // the 128 x 128 epilogue does not fold C's magnitude in
            }
            // Two-piece products on 128 x 128 tiles that would not fill the chip (few rows) split K: partials,
            // then one pass that sums them, adds the bias, rotates and measures C.
            const int tiles = p.tiles_m * p.tiles_n;
            if (!big && p.amax_a && N % 64 == 0 && set_splits(p, fill_splits(ctx, tiles, K, 128)) > 1) {
                float* part = static_cast<float*>(ctx->workspace(0, sizeof(float) * (size_t)p.splits * M * N));
                p.mode = PARTIAL;
                p.C = part;
                {
                    ProfileScope scope(ctx, "gemm_nt_h2", 2.0 * M * N * (double)K, 0.0);
                    LAYA_LAUNCH((gemm_x6_kernel<KVEC, KVEC, PARTIAL, false, 2>), dim3(tiles * p.splits),
                                dim3(THREADS), 0, ctx->stream, p);
                    check_launch("gemm_x6_kernel");
                }
                ProfileScope scope(ctx, "gemm_splitk_store", 0.0, 4.0 * (double)M * N * (p.splits + 1));
                if (aligned16(C) && (!bias || aligned16(bias)) && aligned16(cos_t) && aligned16(sin_t))
                    LAYA_LAUNCH(splitk_store_rope_kernel<4>, dim3(blocks_for((size_t)M * N / 8, 256, 4096)), dim3(256),
                                0, ctx->stream, part, p.splits, M, N, C, bias, pos, cos_t, sin_t, rope_cols, amax_c);
                else
                    LAYA_LAUNCH(splitk_store_rope_kernel<1>, dim3(blocks_for((size_t)M * N / 2, 256, 4096)), dim3(256),
                                0, ctx->stream, part, p.splits, M, N, C, bias, pos, cos_t, sin_t, rope_cols, amax_c);
                check_launch("splitk_store_rope_kernel");
                p.amax_c = amax_c;  // folded by the store pass
                return;
            }
            p.splits = 1;
            p.k_per_split = std::max(BK, (K + BK - 1) / BK * BK);
            ProfileScope scope(ctx, "gemm_nt_x6", 2.0 * M * N * (double)K, 0.0);
            if (wide_tiles_pay(ctx, p, false)) {
                launch_wide(ctx, p);
                return;
            }
            if (tall_tiles_pay(ctx, p)) {
                launch_tall(ctx, p);
                return;
            }
            const dim3 g(p.tiles_m * p.tiles_n), b(THREADS);
            if (p.amax_a && p.b_one) {
                profile_rename("gemm_nt_h2b1");
                LAYA_LAUNCH((gemm_x6_kernel<KVEC, KVEC, STORE_ROPE, false, 2, true>), g, b, 0, ctx->stream, p);
            } else if (p.amax_a) {
                profile_rename("gemm_nt_h2");
                LAYA_LAUNCH((gemm_x6_kernel<KVEC, KVEC, STORE_ROPE, false, 2>), g, b, 0, ctx->stream, p);
            } else {
                LAYA_LAUNCH((gemm_x6_kernel<KVEC, KVEC, STORE_ROPE, false>), g, b, 0, ctx->stream, p);
            }
            check_launch("gemm_x6_kernel");
            return;
        }
        ProfileScope scope(ctx, "gemm_nt", 2.0 * M * N * (double)K, 0.0);
        LAYA_LAUNCH((gemm_kernel<true, true, STORE_ROPE, false>), dim3(p.tiles_m * p.tiles_n), dim3(THREADS), 0,
                           ctx->stream, p);
        check_launch("gemm_kernel");
    }();
    // C's magnitude: folded in by a two-piece kernel's epilogue, else measured after the product.
    if (amax_c && !p.amax_c) absmax_into(ctx, C, M, N, N, amax_c);
}

void gemm_geglu(laya_ctx* ctx, int M, int inter, int K, const float* x, const float* W, const float* bias, float* wide,
                float* act, __bf16* act16, const __bf16* x16, const __bf16* W16, AmaxRef amax_x, AmaxRef amax_W,
                unsigned* amax_act) {
    if (M == 0) return;
    const int N = 2 * inter;
    GemmParams p = make_params(M, N, K, x, K, W, K, wide, N, bias, nullptr, 0);
    p.A16 = x16;
    p.B16 = W16;
    p.mode = STORE;
    const int blocks = p.tiles_m * p.tiles_n;
    // Where gemm() itself would run the product as two-piece products on 256-wide tiles (launch_x6's choice).
    bool fuse = (ctx->matmul_pair & 1) && !(ctx->matmul_bf16 & 1) && (ctx->matmul_split & 1) && inter % 4 == 0 &&
                set_splits(p, fill_splits(ctx, blocks, K, 128)) == 1 && gemm_fits_h(p, true, true) &&
                operand_fast(p.A, p.lda, p.vec_a, true, p.M, p.K) && operand_fast(p.B, p.ldb, p.vec_b, true, p.N, p.K);
    const bool wide_tiles = fuse && wide_tiles_pay(ctx, p, three_per_cu(ctx, blocks));
    fuse = fuse && (wide_tiles || tall_tiles_pay(ctx, p));
    if (!fuse) {
        gemm(ctx, GemmLayout::NT, GemmEpilogue::Store, M, N, K, x, K, W, K, wide, N, bias, nullptr, 0, x16, W16, amax_x,
             amax_W);
        geglu_fwd(ctx, wide, M, inter, act, act16, amax_act);
        return;
    }
    prepare_pair_nt(ctx, p, amax_x, amax_W);
    p.mode = STORE_GEGLU;
    p.act = act;
    p.act16 = act16;
    p.amax_act = amax_act;
    p.inter = inter;
    p.tiles_n = (inter + WT / 2 - 1) / (WT / 2);
    ProfileScope scope(ctx, "gemm_nt_x6", 2.0 * M * N * (double)K, 0.0);
    if (wide_tiles) {
        p.tiles_m = (M + WT - 1) / WT;
        const dim3 g(p.tiles_m * p.tiles_n), b(WT_THREADS);
        profile_rename(p.b_one ? "gemm_nt_geglu_h2b1w" : "gemm_nt_geglu_h2w");
        if (p.b_one)
            LAYA_LAUNCH((gemm_x6w_kernel<STORE_GEGLU, 2, false, false, true>), g, b, 0, ctx->stream, p);
        else
            LAYA_LAUNCH((gemm_x6w_kernel<STORE_GEGLU, 2>), g, b, 0, ctx->stream, p);
        check_launch("gemm_x6w_kernel");
    } else {
        p.tiles_m = (M + TM - 1) / TM;
        const dim3 g(p.tiles_m * p.tiles_n), b(WT_THREADS);
        profile_rename(p.b_one ? "gemm_nt_geglu_h2b1t" : "gemm_nt_geglu_h2t");
        if (p.b_one)
            LAYA_LAUNCH((gemm_x6t_kernel<STORE_GEGLU, false, 2, true>), g, b, 0, ctx->stream, p);
        else
            LAYA_LAUNCH((gemm_x6t_kernel<STORE_GEGLU, false, 2>), g, b, 0, ctx->stream, p);
        check_launch("gemm_x6t_kernel");
    }
}

// The balanced static schedule of a backward pair, when every worker's whole dX tiles fit in its share of
// the work and every worker's dW run is shorter than one dW tile (so every dW tile is shared by two or
// more workers, whose partials the fixup adds, and no worker holds more than its two partial slots).
bool make_pair_plan(const laya_ctx* ctx, int n0, int out, int n1, int rows, PairPlan& s) {
    s = PairPlan{};
    s.G = 2 * ctx->cu_count;
    s.nn_tiles = n0;
    s.nn_units = (out + BK - 1) / BK;
    s.tn_tiles = n1;
    s.tn_units = (rows + BK - 1) / BK;
    s.q = n0 / s.G;
    s.r = n0 % s.G;
    const long W = (long)n0 * s.nn_units + (long)n1 * s.tn_units;
    s.W = (int)std::min<long>(W, 1L << 30);
    const long need_min = W / s.G - (long)(s.q + (s.r > 0 ? 1 : 0)) * s.nn_units;
    const long max_run = (W + s.G - 1) / s.G - (long)s.q * s.nn_units;
    return need_min >= 0 && s.nn_units > 0 && W * s.G < (1L << 31) && max_run < s.tn_units &&
           s.G <= FIXUP_MAX_WORKERS;
}

// The same schedule over one worker per CU, 256 x 256 tiles and 16-deep units (the wide pair).
bool make_pair_plan_wide(const laya_ctx* ctx, int n0, int out, int n1, int rows, PairPlan& s) {
    s = PairPlan{};
    s.G = ctx->cu_count;
    s.nn_tiles = n0;
    s.nn_units = (out + BKQ - 1) / BKQ;
    s.tn_tiles = n1;
    s.tn_units = (rows + BKQ - 1) / BKQ;
    s.q = n0 / s.G;
    s.r = n0 % s.G;
    const long W = (long)n0 * s.nn_units + (long)n1 * s.tn_units;
    s.W = (int)std::min<long>(W, 1L << 30);
    const long need_min = W / s.G - (long)(s.q + (s.r > 0 ? 1 : 0)) * s.nn_units;
    const long max_run = (W + s.G - 1) / s.G - (long)s.q * s.nn_units;
    return need_min >= 0 && s.nn_units > 0 && W * s.G < (1L << 31) && max_run < s.tn_units &&
           s.G <= FIXUP_MAX_WORKERS;
}

// The wide pair for split products: dX without residual, dX's K a multiple of 16, dY k-contiguous in
// float4s. Returns false (nothing launched) when the wide plan does not apply.
// amax_dx (optional): dX's magnitude word group, folded in by the two-piece kernel (*folded set), else
// left to the caller.
bool backward_pair_wide(laya_ctx* ctx, GemmParams nn, GemmParams tn, int rows, int in, int out, bool half,
                        AmaxRef amax_dy, AmaxRef amax_W, AmaxRef amax_x, unsigned* amax_dx, bool* folded) {
    const bool bh = half && nn.B16 && tn.B16;  // W and x from their bf16 copies
    if (out % BKQ != 0 || !operand_fast(nn.A, nn.lda, nn.vec_a, true, nn.M, nn.K)) return false;
    const long lim = 1L << 31;  // buffer offsets of dY, W and x
    if ((long)rows * out * 4 >= lim || (long)out * in * 4 >= lim || (long)rows * in * 4 >= lim) return false;
    nn.tiles_m = (rows + WT - 1) / WT;
    nn.tiles_n = (in + WT - 1) / WT;
    tn.tiles_m = (out + WT - 1) / WT;
    tn.tiles_n = (in + WT - 1) / WT;
    const int n0 = nn.tiles_m * nn.tiles_n, n1 = tn.tiles_m * tn.tiles_n;
    PairPlan s{};
    if (!make_pair_plan_wide(ctx, n0, out, n1, rows, s)) return false;
    s.partial = static_cast<float*>(ctx->workspace(0, sizeof(float) * (size_t)s.G * 2 * WT * WT));
    const bool pair = !half && (ctx->matmul_pair & 6) == 6;
    if (pair) {
        nn.amax_a = tn.amax_a = operand_amax(ctx, amax_dy, 0, nn.A, rows, out, nn.lda);
        nn.amax_b = operand_amax(ctx, amax_W, 1, nn.B, out, in, nn.ldb);
        tn.amax_b = operand_amax(ctx, amax_x, 2, tn.B, rows, in, tn.ldb);
        nn.amax_c = nn.R ? nullptr : amax_dx;
        *folded = nn.amax_c != nullptr;
    }
    {
        ProfileScope scope(ctx, half ? "gemm_bwd_pair_bf16w" : pair ? "gemm_bwd_pair_h2w" : "gemm_bwd_pair_x6w",
                           2.0 * 2.0 * rows * (double)in * out, 0.0);
        const dim3 g(s.G), b(WT_THREADS);
        if (pair && nn.R)
            LAYA_LAUNCH((gemm_pair_wide_kernel<2, true>), g, b, 0, ctx->stream, nn, tn, s);
        else if (pair)
            LAYA_LAUNCH((gemm_pair_wide_kernel<2, false>), g, b, 0, ctx->stream, nn, tn, s);
        else if (bh && nn.R)
            LAYA_LAUNCH((gemm_pair_wide_kernel<1, true, true>), g, b, 0, ctx->stream, nn, tn, s);
        else if (bh)
            LAYA_LAUNCH((gemm_pair_wide_kernel<1, false, true>), g, b, 0, ctx->stream, nn, tn, s);
        else if (half && nn.R)
            LAYA_LAUNCH((gemm_pair_wide_kernel<1, true>), g, b, 0, ctx->stream, nn, tn, s);
        else if (half)
            LAYA_LAUNCH((gemm_pair_wide_kernel<1, false>), g, b, 0, ctx->stream, nn, tn, s);
        else if (nn.R)
            LAYA_LAUNCH((gemm_pair_wide_kernel<3, true>), g, b, 0, ctx->stream, nn, tn, s);
        else
            LAYA_LAUNCH((gemm_pair_wide_kernel<3, false>), g, b, 0, ctx->stream, nn, tn, s);
        check_launch("gemm_pair_wide_kernel");
    }
    long partials = 0, shared = 0;
    const long Wt = (long)n0 * s.nn_units + (long)n1 * s.tn_units;
    auto tn_lo = [&](long g) { return g * Wt / s.G - (long)s.nn_units * (g * s.q + std::min<long>(g, s.r)); };
    for (int g = 0; ctx->profiling && g < s.G; ++g) {
        const long lo = tn_lo(g), hi = tn_lo(g + 1);
        for (long u = lo; u < hi;) {
            const long t = u / s.tn_units, a = u - t * s.tn_units;
            const long b = std::min<long>(s.tn_units, a + (hi - u));
            ++partials;
            if (a == 0) ++shared;
            u += b - a;
        }
    }
    ProfileScope scope(ctx, "gemm_pair_fixup", 0.0, 4.0 * WT * WT * (double)(partials + 2 * shared));
    LAYA_LAUNCH(pair_fixup_w_kernel, dim3(n1, 32), dim3(WT_THREADS), 0, ctx->stream, tn, s);
    check_launch("pair_fixup_w_kernel");
    return true;
}

void gemm_backward_pair(laya_ctx* ctx, int rows, int in, int out, const float* dy, const float* W, const float* x,
                        float* dx, const float* dx_residual, float* dW, const __bf16* W16, const __bf16* x16,
                        AmaxRef amax_dy, AmaxRef amax_W, AmaxRef amax_x, unsigned* amax_dx) {
    bool folded = false;
    gemm_backward_pair_body(ctx, rows, in, out, dy, W, x, dx, dx_residual, dW, W16, x16, amax_dy, amax_W, amax_x,
                            amax_dx, &folded);
    // dX's magnitude: folded in by the two-piece pair's epilogue, else measured after the products.
    if (amax_dx && !folded && rows > 0) absmax_into(ctx, dx, rows, in, in, amax_dx);
}

void gemm_backward_pair_body(laya_ctx* ctx, int rows, int in, int out, const float* dy, const float* W,
                             const float* x, float* dx, const float* dx_residual, float* dW, const __bf16* W16,
                             const __bf16* x16, AmaxRef amax_dy, AmaxRef amax_W, AmaxRef amax_x, unsigned* amax_dx,
                             bool* folded) {
    if (rows == 0) return;
    // dx[rows, in] = dy[rows, out] · W[out, in]       (NN, K = out)
    GemmParams nn = make_params(rows, in, out, dy, out, W, in, dx, in, nullptr, dx_residual, in);
    nn.mode = STORE;
    nn.B16 = W16;
    // dW[out, in] += dy[rows, out]ᵀ · x[rows, in]     (TN, K = rows)
    GemmParams tn = make_params(out, in, rows, dy, out, x, in, dW, in, nullptr, nullptr, 0);
    tn.B16 = x16;
    const bool split = !(ctx->matmul_bf16 & 6) && (ctx->matmul_split & 6) == 6 && gemm_fits_h(nn, true, false) &&
                       gemm_fits_h(tn, false, false);
    const bool fp32 = !((ctx->matmul_bf16 | ctx->matmul_split) & 6) && gemm_fast(nn, true, false) &&
                      gemm_fast(tn, false, false);
    const bool half = (ctx->matmul_bf16 & 6) == 6 && gemm_fits_h(nn, true, false) && gemm_fits_h(tn, false, false);
    tn.mode = ACCUMULATE;
    if ((split || half) &&
        backward_pair_wide(ctx, nn, tn, rows, in, out, half, amax_dy, amax_W, amax_x, amax_dx, folded))
        return;
    tn.mode = STORE;
    const int n0 = nn.tiles_m * nn.tiles_n, n1 = tn.tiles_m * tn.tiles_n;
    PairPlan s{};
    if ((split || fp32 || half) && make_pair_plan(ctx, n0, out, n1, rows, s)) {
        s.partial = static_cast<float*>(ctx->workspace(0, sizeof(float) * (size_t)s.G * 2 * BM * BN));
        tn.mode = ACCUMULATE;
        {
            ProfileScope scope(ctx, split ? "gemm_bwd_pair_x6" : half ? "gemm_bwd_pair_bf16" : "gemm_bwd_pair",
                               2.0 * 2.0 * rows * (double)in * out, 0.0);
            const dim3 g(s.G), b(THREADS);
            if (half) {
                const bool va = operand_fast(nn.A, nn.lda, nn.vec_a, true, nn.M, nn.K);
                if (va && dx_residual)
                    LAYA_LAUNCH((gemm_pair_planned_h_kernel<KVEC, true>), g, b, 0, ctx->stream, nn, tn, s);
                else if (va)
                    LAYA_LAUNCH((gemm_pair_planned_h_kernel<KVEC, false>), g, b, 0, ctx->stream, nn, tn, s);
                else if (dx_residual)
                    LAYA_LAUNCH((gemm_pair_planned_h_kernel<KSCALAR, true>), g, b, 0, ctx->stream, nn, tn, s);
                else
                    LAYA_LAUNCH((gemm_pair_planned_h_kernel<KSCALAR, false>), g, b, 0, ctx->stream, nn, tn, s);
                check_launch("gemm_pair_planned_h_kernel");
            } else if (split) {
                if (operand_fast(nn.A, nn.lda, nn.vec_a, true, nn.M, nn.K)) {
                    if (dx_residual)
                        LAYA_LAUNCH((gemm_pair_planned_x6_kernel<KVEC, true>), g, b, 0, ctx->stream, nn, tn, s);
                    else
                        LAYA_LAUNCH((gemm_pair_planned_x6_kernel<KVEC, false>), g, b, 0, ctx->stream, nn, tn, s);
                } else {
                    if (dx_residual)
                        LAYA_LAUNCH((gemm_pair_planned_x6_kernel<KSCALAR, true>), g, b, 0, ctx->stream, nn, tn,
                                           s);
                    else
                        LAYA_LAUNCH((gemm_pair_planned_x6_kernel<KSCALAR, false>), g, b, 0, ctx->stream, nn, tn,
                                           s);
                }
                check_launch("gemm_pair_planned_x6_kernel");
            } else {
                if (dx_residual)
                    LAYA_LAUNCH((gemm_pair_planned_kernel<true>), g, b, 0, ctx->stream, nn, tn, s);
                else
                    LAYA_LAUNCH((gemm_pair_planned_kernel<false>), g, b, 0, ctx->stream, nn, tn, s);
                check_launch("gemm_pair_planned_kernel");
            }
        }
        // Compulsory bytes of the fixup: every partial tile read once, every shared dW tile read and
        // written once (the same walk over the workers' runs the kernels make).
        long partials = 0, shared = 0;
        const long Wt = (long)n0 * s.nn_units + (long)n1 * s.tn_units;
        auto tn_lo = [&](long g) { return g * Wt / s.G - (long)s.nn_units * (g * s.q + std::min<long>(g, s.r)); };
        for (int g = 0; ctx->profiling && g < s.G; ++g) {
            const long lo = tn_lo(g), hi = tn_lo(g + 1);
            for (long u = lo; u < hi;) {
                const long t = u / s.tn_units, a = u - t * s.tn_units;
                const long b = std::min<long>(s.tn_units, a + (hi - u));
                if (!(a == 0 && b == s.tn_units)) {
                    ++partials;
                    if (a == 0) ++shared;  // count each shared tile at its first piece
                }
                u += b - a;
            }
        }
        ProfileScope scope(ctx, "gemm_pair_fixup", 0.0, 4.0 * BM * BN * (double)(partials + 2 * shared));
        if (split || half)
            LAYA_LAUNCH(pair_fixup_kernel<true>, dim3(n1, 8), dim3(THREADS), 0, ctx->stream, tn, s);
        else
            LAYA_LAUNCH(pair_fixup_kernel<false>, dim3(n1, 8), dim3(THREADS), 0, ctx->stream, tn, s);
        check_launch("pair_fixup_kernel");
        return;
    }
    if (!fp32) {
        // dX's magnitude: folded by the split-K store pass, or measured after the product, inside gemm().
        gemm(ctx, GemmLayout::NN, GemmEpilogue::Store, rows, in, out, dy, out, W, in, dx, in, nullptr, dx_residual,
             in, nullptr, nullptr, amax_dy, amax_W, amax_dx);
        if (folded) *folded = amax_dx != nullptr;
        gemm(ctx, GemmLayout::TN, GemmEpilogue::Accumulate, out, in, rows, dy, out, x, in, dW, in, nullptr, nullptr,
             0, nullptr, nullptr, amax_dy, amax_x);
        return;
    }
    // Choose the dW split so its slices are as long as a dX tile's K loop, then minimise the rounds of
    // 2-blocks-per-CU the combined grid needs times the longest block.
    const long slots = 2L * ctx->cu_count;
    const long knn = std::max(BK, (out + BK - 1) / BK * BK);
    int best_s = 1;
    double best = 1e300;
    for (int s = 1; s <= 64; ++s) {
        GemmParams t = tn;
        const int real = set_splits(t, s);
        if (real != s) continue;
        const long total = n0 + (long)n1 * s;
        // Rounds × the longest block's K, plus the split-K reduce traffic in the same K units (a round
        // of two 128×128 blocks per CU costs ≈ 1.2e-7 s per unit of K; the reduce moves 4·out·in·s bytes).
        const double est = (double)((total + slots - 1) / slots) * std::max<long>(knn, t.k_per_split) +
                           6.8e-6 * s * (double)out * in;
        if (est < best) {
            best = est;
            best_s = s;
        }
    }
    set_splits(tn, best_s);
    float* dW_out = prepare_accumulate(ctx, tn);
    const int blocks = n0 + n1 * tn.splits;
    {
        ProfileScope scope(ctx, "gemm_bwd_pair", 2.0 * 2.0 * rows * (double)in * out, 0.0);
        const dim3 g(blocks), b(THREADS);
        if (tn.mode == ACCUMULATE) {
            if (dx_residual)
                LAYA_LAUNCH((gemm_pair_kernel<ACCUMULATE, true>), g, b, 0, ctx->stream, nn, tn, n0);
            else
                LAYA_LAUNCH((gemm_pair_kernel<ACCUMULATE, false>), g, b, 0, ctx->stream, nn, tn, n0);
        } else {
            if (dx_residual)
                LAYA_LAUNCH((gemm_pair_kernel<PARTIAL, true>), g, b, 0, ctx->stream, nn, tn, n0);
            else
                LAYA_LAUNCH((gemm_pair_kernel<PARTIAL, false>), g, b, 0, ctx->stream, nn, tn, n0);
        }
        check_launch("gemm_pair_kernel");
    }
    finish_accumulate(ctx, tn, dW_out, in);
}

void column_sum_add(laya_ctx* ctx, const float* x, int rows, int n, float* out, unsigned* amax) {
    if (rows <= 0 || n <= 0) return;
    if (n % 4 == 0 && aligned16(x) && aligned16(out) && rows > 256) {
        column_sums(ctx, x, rows, n, nullptr, 1, out, 1, amax);
        return;
    }
    if (amax) absmax_into(ctx, x, rows, n, n, amax);
    const int rows_per = 256;
    const int chunks = (rows + rows_per - 1) / rows_per;
    if (chunks <= 1) {
        LAYA_LAUNCH(column_sum_kernel, dim3((n + 255) / 256), dim3(256), 0, ctx->stream, x, rows, n, out);
        check_launch("column_sum_kernel");
        return;
    }
    float* part = static_cast<float*>(ctx->workspace(1, sizeof(float) * (size_t)chunks * n));
    LAYA_LAUNCH(column_partial_kernel, dim3((n + 255) / 256, chunks), dim3(256), 0, ctx->stream, x, rows, n,
                       rows_per, part);
    check_launch("column_partial_kernel");
    LAYA_LAUNCH(column_reduce_kernel, dim3((n + 255) / 256), dim3(256), 0, ctx->stream, part, chunks, n, out);
    check_launch("column_reduce_kernel");
}

}  // namespace laya
