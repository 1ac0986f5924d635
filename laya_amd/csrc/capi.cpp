// The C-ABI of liblaya_hip (include/laya_hip.h): context, memory, stream, and one entry point per
// reference op. Every entry point validates its arguments on the host before any launch, so a bad
// call returns a status code instead of reaching the device.
#include <algorithm>
#include <cmath>
#include <cstring>
#include <vector>

#include "elementwise.hpp"

namespace laya {
static thread_local std::string g_last_error;
void set_last_error(const std::string& msg) { g_last_error = msg; }
}  // namespace laya

using namespace laya;

void* laya_ctx::alloc(size_t bytes) {
    if (bytes == 0) bytes = 16;
    if (cap && in_use + bytes > cap)
        throw Error(LAYA_ERR_MEMORY, "allocation of " + std::to_string(bytes) + " bytes exceeds the context cap of " +
                                         std::to_string(cap) + " bytes (" + std::to_string(in_use) + " in use)");
    void* p = nullptr;
    hipError_t e = hipMalloc(&p, bytes);
    if (e != hipSuccess) {
        (void)hipGetLastError();
        throw Error(LAYA_ERR_MEMORY, "hipMalloc(" + std::to_string(bytes) + ") failed: " + hipGetErrorString(e));
    }
    allocations[p] = bytes;
    in_use += bytes;
    return p;
}

void laya_ctx::release(void* p) {
    if (!p) return;
    auto it = allocations.find(p);
    if (it == allocations.end()) throw Error(LAYA_ERR_ARGUMENT, "free of a pointer this context did not allocate");
    LAYA_HIP(hipStreamSynchronize(stream));
    LAYA_HIP(hipFree(p));
    in_use -= it->second;
    allocations.erase(it);
}

void* laya_ctx::workspace(int slot, size_t bytes) {
    Workspace& w = scratch[slot];
    if (w.bytes >= bytes && w.ptr) return w.ptr;
    if (w.ptr) release(w.ptr);
    w.ptr = nullptr;
    w.bytes = 0;
    size_t grow = std::max(bytes, (size_t)1 << 20);
    w.ptr = alloc(grow);
    w.bytes = grow;
    return w.ptr;
}

namespace laya {

static int take_event(laya_ctx* ctx) {
    if (ctx->next_event >= (int)ctx->event_pool.size()) {
        hipEvent_t e;
        LAYA_HIP(hipEventCreate(&e));
        ctx->event_pool.push_back(e);
    }
    return ctx->next_event++;
}

static thread_local ProfileScope* g_scope = nullptr;

void profile_rename(const char* name) {
    if (g_scope) g_scope->name = name;
}

ProfileScope::ProfileScope(laya_ctx* c, const char* n, double f, double b)
    : ctx(c), name(n), flops(f), bytes(b), outer(g_scope) {
    g_scope = this;
    if (!ctx->profiling || !name) return;
    start = take_event(ctx);
    LAYA_HIP(hipEventRecord(ctx->event_pool[start], ctx->stream));
}

ProfileScope::~ProfileScope() {
    g_scope = outer;
    if (start < 0 || !ctx->profiling) return;
    try {
        const int stop = take_event(ctx);
        if (hipEventRecord(ctx->event_pool[stop], ctx->stream) == hipSuccess)
            ctx->launches.push_back({name, start, stop, nested ? -1 : kstart, nested ? -1 : kstop, flops, bytes});
    } catch (...) {
    }
}

void profile_kernel_events(hipEvent_t* ev_start, hipEvent_t* ev_stop) {
    ProfileScope* s = g_scope;
    if (!s || s->start < 0 || !s->ctx->profiling) return;
    for (ProfileScope* o = s->outer; o; o = o->outer) o->nested = true;
    if (s->kstart < 0) {
        s->kstart = take_event(s->ctx);
        *ev_start = s->ctx->event_pool[s->kstart];
    }
    if (s->kstop < 0) s->kstop = take_event(s->ctx);
    *ev_stop = s->ctx->event_pool[s->kstop];
}

// Rotary tables (Ops.cs:462-484): angles in double, cos/sin rounded to float.
void build_rotary(laya_ctx* ctx, laya_rotary* r, int head_dim, double theta, int positions) {
    LAYA_REQUIRE(head_dim > 0 && head_dim % 2 == 0, "rotary: head_dim must be even");
    LAYA_REQUIRE(positions > 0, "rotary: positions must be positive");
    const int half = head_dim / 2;
    std::vector<float> c((size_t)positions * half), s((size_t)positions * half);
    for (int i = 0; i < half; ++i) {
        const double inv = 1.0 / std::pow(theta, 2.0 * i / head_dim);
        for (int p = 0; p < positions; ++p) {
            const double angle = p * inv;
            c[(size_t)p * half + i] = (float)std::cos(angle);
            s[(size_t)p * half + i] = (float)std::sin(angle);
        }
    }
    if (r->cos_t) ctx->release(r->cos_t);
    if (r->sin_t) ctx->release(r->sin_t);
    r->cos_t = static_cast<float*>(ctx->alloc(c.size() * sizeof(float)));
    r->sin_t = static_cast<float*>(ctx->alloc(s.size() * sizeof(float)));
    LAYA_HIP(hipMemcpyAsync(r->cos_t, c.data(), c.size() * sizeof(float), hipMemcpyHostToDevice, ctx->stream));
    LAYA_HIP(hipMemcpyAsync(r->sin_t, s.data(), s.size() * sizeof(float), hipMemcpyHostToDevice, ctx->stream));
    LAYA_HIP(hipStreamSynchronize(ctx->stream));
    r->head_dim = head_dim;
    r->theta = theta;
    r->positions = positions;
}

void free_rotary(laya_ctx* ctx, laya_rotary* r) {
    if (r->cos_t) ctx->release(r->cos_t);
    if (r->sin_t) ctx->release(r->sin_t);
    r->cos_t = r->sin_t = nullptr;
}

}  // namespace laya

static void require_ctx(laya_ctx* ctx) { LAYA_REQUIRE(ctx != nullptr, "null context"); }

extern "C" {

const char* laya_last_error(void) { return g_last_error.c_str(); }
const char* laya_version(void) { return "laya_hip 0.1 gfx950"; }

int laya_ctx_create(int device, laya_ctx** out) {
    return guarded([&] {
        LAYA_REQUIRE(out != nullptr, "null output pointer");
        int count = 0;
        LAYA_HIP(hipGetDeviceCount(&count));
        LAYA_REQUIRE(device >= 0 && device < count, "device index out of range");
        LAYA_HIP(hipSetDevice(device));
        noalloc_scratch_init(device);
        auto* c = new laya_ctx();
        c->device = device;
        LAYA_HIP(hipStreamCreateWithFlags(&c->stream, hipStreamNonBlocking));
        hipDeviceProp_t prop;
        if (hipGetDeviceProperties(&prop, device) == hipSuccess) c->cu_count = prop.multiProcessorCount;
        *out = c;
    });
}

int laya_ctx_destroy(laya_ctx* ctx) {
    return guarded([&] {
        if (!ctx) return;
        hipSetDevice(ctx->device);
        hipStreamSynchronize(ctx->stream);
        for (auto& kv : ctx->allocations) hipFree(kv.first);
        for (auto& t : ctx->timers)
            for (auto& e : t)
                if (e) hipEventDestroy(e);
        for (auto& e : ctx->event_pool) hipEventDestroy(e);
        hipStreamDestroy(ctx->stream);
        delete ctx;
    });
}

int laya_ctx_set_memory_cap(laya_ctx* ctx, size_t bytes) {
    return guarded([&] {
        require_ctx(ctx);
        ctx->cap = bytes;
    });
}

int laya_ctx_set_matmul_precision(laya_ctx* ctx, int precision) {
    return guarded([&] {
        require_ctx(ctx);
        LAYA_REQUIRE(precision >= 0 && precision <= (LAYA_MATMUL_BF16 | LAYA_MATMUL_FP32_MFMA | LAYA_MATMUL_FP32_SPLIT3),
                     "matmul precision: LAYA_MATMUL_FP32, LAYA_MATMUL_FP32_MFMA, LAYA_MATMUL_FP32_SPLIT3, or bf16 "
                     "classes");
        LAYA_REQUIRE(!((precision & LAYA_MATMUL_FP32_MFMA) && (precision & LAYA_MATMUL_FP32_SPLIT3)),
                     "matmul precision: LAYA_MATMUL_FP32_MFMA and LAYA_MATMUL_FP32_SPLIT3 exclude each other");
        ctx->matmul_bf16 = precision & LAYA_MATMUL_BF16;
        // fp32 classes use split products unless LAYA_MATMUL_FP32_MFMA asks for the fp32 matrix cores; the
        // 256-wide kernels of those take two-piece fp16 products unless LAYA_MATMUL_FP32_SPLIT3 asks for the
        // three-piece bf16 splits.
        ctx->matmul_split = (precision & LAYA_MATMUL_FP32_MFMA) ? 0 : (LAYA_MATMUL_SPLIT_ALL & ~ctx->matmul_bf16);
        ctx->matmul_pair = ctx->matmul_split & ~((precision & LAYA_MATMUL_FP32_SPLIT3) >> 4);
        ctx->attention_pair = !(precision & LAYA_MATMUL_SPLIT3_ATTENTION);
    });
}

int laya_ctx_memory_in_use(laya_ctx* ctx, size_t* bytes) {
    return guarded([&] {
        require_ctx(ctx);
        *bytes = ctx->in_use;
    });
}

int laya_alloc(laya_ctx* ctx, size_t bytes, void** out) {
    return guarded([&] {
        require_ctx(ctx);
        LAYA_REQUIRE(out != nullptr, "null output pointer");
        *out = ctx->alloc(bytes);
    });
}

int laya_free(laya_ctx* ctx, void* ptr) {
    return guarded([&] {
        require_ctx(ctx);
        ctx->release(ptr);
    });
}

int laya_upload(laya_ctx* ctx, void* dst, const void* src, size_t bytes) {
    return guarded([&] {
        require_ctx(ctx);
        if (!bytes) return;
        LAYA_REQUIRE(dst && src, "null pointer");
        LAYA_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, ctx->stream));
        LAYA_HIP(hipStreamSynchronize(ctx->stream));
    });
}

int laya_download(laya_ctx* ctx, void* dst, const void* src, size_t bytes) {
    return guarded([&] {
        require_ctx(ctx);
        if (!bytes) return;
        LAYA_REQUIRE(dst && src, "null pointer");
        LAYA_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, ctx->stream));
        LAYA_HIP(hipStreamSynchronize(ctx->stream));
    });
}

int laya_fill(laya_ctx* ctx, float* dst, float value, size_t count) {
    return guarded([&] {
        require_ctx(ctx);
        fill(ctx, dst, value, count);
    });
}

int laya_sync(laya_ctx* ctx) {
    return guarded([&] {
        require_ctx(ctx);
        LAYA_HIP(hipStreamSynchronize(ctx->stream));
    });
}

int laya_timer_begin(laya_ctx* ctx, int slot) {
    return guarded([&] {
        require_ctx(ctx);
        LAYA_REQUIRE(slot >= 0 && slot < 16, "timer slot out of range");
        for (auto& e : ctx->timers[slot])
            if (!e) LAYA_HIP(hipEventCreate(&e));
        LAYA_HIP(hipEventRecord(ctx->timers[slot][0], ctx->stream));
    });
}

int laya_timer_end(laya_ctx* ctx, int slot) {
    return guarded([&] {
        require_ctx(ctx);
        LAYA_REQUIRE(slot >= 0 && slot < 16 && ctx->timers[slot][1], "timer slot not started");
        LAYA_HIP(hipEventRecord(ctx->timers[slot][1], ctx->stream));
    });
}

int laya_timer_elapsed(laya_ctx* ctx, int slot, float* ms) {
    return guarded([&] {
        require_ctx(ctx);
        LAYA_REQUIRE(slot >= 0 && slot < 16 && ctx->timers[slot][1], "timer slot not started");
        LAYA_HIP(hipEventSynchronize(ctx->timers[slot][1]));
        LAYA_HIP(hipEventElapsedTime(ms, ctx->timers[slot][0], ctx->timers[slot][1]));
    });
}

namespace {
struct KernelSummary {
    std::string name;
    int launches = 0;
    double ms = 0, flops = 0, bytes = 0;
};
thread_local std::vector<KernelSummary> g_summary;
}  // namespace

int laya_profile_begin(laya_ctx* ctx) {
    return guarded([&] {
        require_ctx(ctx);
        LAYA_HIP(hipStreamSynchronize(ctx->stream));
        ctx->launches.clear();
        ctx->next_event = 0;
        ctx->profiling = true;
    });
}

int laya_profile_end(laya_ctx* ctx) {
    return guarded([&] {
        require_ctx(ctx);
        ctx->profiling = false;
        LAYA_HIP(hipStreamSynchronize(ctx->stream));
        g_summary.clear();
        for (const auto& r : ctx->launches) {
            float ms = 0.0f;
            const bool own = r.kstart >= 0 && r.kstop >= 0;  // the kernels' own start and end
            LAYA_HIP(hipEventElapsedTime(&ms, ctx->event_pool[own ? r.kstart : r.start],
                                         ctx->event_pool[own ? r.kstop : r.stop]));
            auto it = std::find_if(g_summary.begin(), g_summary.end(),
                                   [&](const KernelSummary& k) { return k.name == r.name; });
            if (it == g_summary.end()) {
                g_summary.push_back({r.name});
                it = g_summary.end() - 1;
            }
            it->launches++;
            it->ms += ms;
            it->flops += r.flops;
            it->bytes += r.bytes;
        }
        ctx->launches.clear();
        ctx->next_event = 0;
    });
}

int laya_profile_count(laya_ctx* ctx, int* kernels) {
    return guarded([&] {
        require_ctx(ctx);
        *kernels = (int)g_summary.size();
    });
}

int laya_profile_get(laya_ctx* ctx, int i, const char** name, int* launches, double* total_ms, double* flops,
                     double* bytes) {
    return guarded([&] {
        require_ctx(ctx);
        LAYA_REQUIRE(i >= 0 && i < (int)g_summary.size(), "profile index out of range");
        const auto& k = g_summary[i];
        if (name) *name = k.name.c_str();
        if (launches) *launches = k.launches;
        if (total_ms) *total_ms = k.ms;
        if (flops) *flops = k.flops;
        if (bytes) *bytes = k.bytes;
    });
}

// ------------------------------------------------------------------------------------- ops

int laya_linear_fwd(laya_ctx* ctx, const float* x, int rows, int in, const float* W, int out, const float* b,
                    const float* residual, float* y) {
    return guarded([&] {
        require_ctx(ctx);
        LAYA_REQUIRE(rows >= 0 && in > 0 && out > 0, "linear: bad size");
        LAYA_REQUIRE(x && W && y, "linear: null tensor");
        gemm(ctx, GemmLayout::NT, GemmEpilogue::Store, rows, out, in, x, in, W, in, y, out, b, residual, out);
    });
}

int laya_linear_bwd(laya_ctx* ctx, const float* x, const float* dy, int rows, int in, int out, const float* W,
                    float* dx, float* dW, float* db) {
    return guarded([&] {
        require_ctx(ctx);
        LAYA_REQUIRE(rows >= 0 && in > 0 && out > 0, "linear_bwd: bad size");
        LAYA_REQUIRE(dy && W, "linear_bwd: null tensor");
        LAYA_REQUIRE(!dW || x, "linear_bwd: dW needs x");
        if (dx && dW && db) {
            // The bias gradient's pass over dy takes dy's magnitude for the pair's two-piece products too.
            unsigned* w = operand_ring_word(ctx);
            column_sum_add(ctx, dy, rows, out, db, w);
            unsigned char known = 1;
            gemm_backward_pair(ctx, rows, in, out, dy, W, x, dx, nullptr, dW, nullptr, nullptr, AmaxRef{w, &known});
            return;
        }
        if (dx && dW)
            gemm_backward_pair(ctx, rows, in, out, dy, W, x, dx, nullptr, dW);
        else if (dx)
            gemm(ctx, GemmLayout::NN, GemmEpilogue::Store, rows, in, out, dy, out, W, in, dx, in);
        else if (dW)
            gemm(ctx, GemmLayout::TN, GemmEpilogue::Accumulate, out, in, rows, dy, out, x, in, dW, in);
        if (db) column_sum_add(ctx, dy, rows, out, db);
    });
}

int laya_layernorm_fwd(laya_ctx* ctx, const float* x, int rows, int n, const float* w, const float* b, float eps,
                       float* y, float* mean, float* rstd) {
    return guarded([&] {
        require_ctx(ctx);
        LAYA_REQUIRE(rows >= 0 && x && w && y, "layernorm: bad arguments");
        layernorm_fwd(ctx, x, rows, n, w, b, eps, y, mean, rstd);
    });
}

int laya_layernorm_bwd(laya_ctx* ctx, const float* x, int rows, int n, const float* w, float eps, const float* dy,
                       float* dx, float* dgamma, float* dbeta, const float* mean, const float* rstd) {
    return guarded([&] {
        require_ctx(ctx);
        LAYA_REQUIRE(rows >= 0 && x && w && dy && dx, "layernorm_bwd: bad arguments");
        LAYA_REQUIRE((mean == nullptr) == (rstd == nullptr), "layernorm_bwd: pass both mean and rstd, or neither");
        layernorm_bwd(ctx, x, rows, n, w, eps, dy, dx, dgamma, dbeta, mean, rstd);
    });
}

int laya_layernorm_bwd_noalloc(laya_ctx* ctx, const float* x, int rows, int n, const float* w, float eps,
                               const float* dy, float* dx, float* dgamma, float* dbeta, const float* mean,
                               const float* rstd) {
    return guarded([&] {
        require_ctx(ctx);
        LAYA_REQUIRE(rows >= 0 && x && w && dy && dx, "layernorm_bwd_noalloc: bad arguments");
        LAYA_REQUIRE((mean == nullptr) == (rstd == nullptr),
                     "layernorm_bwd_noalloc: pass both mean and rstd, or neither");
        layernorm_bwd_noalloc(ctx, x, rows, n, w, eps, dy, dx, dgamma, dbeta, mean, rstd);
    });
}

int laya_gelu_fwd(laya_ctx* ctx, const float* x, size_t n, float* y) {
    return guarded([&] {
        require_ctx(ctx);
        gelu_fwd(ctx, x, n, y);
    });
}

int laya_gelu_bwd(laya_ctx* ctx, const float* u, float* grad, size_t n) {
    return guarded([&] {
        require_ctx(ctx);
        gelu_bwd(ctx, u, grad, n);
    });
}

int laya_geglu_fwd(laya_ctx* ctx, const float* wide, int rows, int inter, float* act) {
    return guarded([&] {
        require_ctx(ctx);
        LAYA_REQUIRE(rows >= 0 && inter > 0, "geglu: bad size");
        geglu_fwd(ctx, wide, rows, inter, act);
    });
}

int laya_geglu_bwd(laya_ctx* ctx, const float* wide, const float* dact, int rows, int inter, float* dwide) {
    return guarded([&] {
        require_ctx(ctx);
        LAYA_REQUIRE(rows >= 0 && inter > 0, "geglu_bwd: bad size");
        geglu_bwd(ctx, wide, dact, rows, inter, dwide);
    });
}

float laya_uniform(uint64_t seed, uint64_t index) { return uniform01(seed, index); }
uint64_t laya_mix(uint64_t seed, uint64_t salt) { return mix64(seed, salt); }

int laya_dropout(laya_ctx* ctx, float* values, size_t n, float p, uint64_t seed) {
    return guarded([&] {
        require_ctx(ctx);
        LAYA_REQUIRE(p >= 0.0f && p < 1.0f, "dropout: p must be in [0, 1)");
        dropout(ctx, values, n, p, seed);
    });
}

int laya_relu_dropout_fwd(laya_ctx* ctx, const float* wide, size_t n, float p, uint64_t seed, float* dropped) {
    return guarded([&] {
        require_ctx(ctx);
        LAYA_REQUIRE(p >= 0.0f && p < 1.0f, "dropout: p must be in [0, 1)");
        relu_dropout_fwd(ctx, wide, n, p, seed, dropped);
    });
}

int laya_relu_dropout_bwd(laya_ctx* ctx, const float* wide, float* grad, size_t n, float p, uint64_t seed) {
    return guarded([&] {
        require_ctx(ctx);
        LAYA_REQUIRE(p >= 0.0f && p < 1.0f, "dropout: p must be in [0, 1)");
        relu_dropout_bwd(ctx, wide, grad, n, p, seed);
    });
}

int laya_add(laya_ctx* ctx, float* dst, const float* src, size_t n) {
    return guarded([&] {
        require_ctx(ctx);
        add(ctx, dst, src, n);
    });
}

int laya_rotary_create(laya_ctx* ctx, int head_dim, double theta, int positions, laya_rotary** out) {
    return guarded([&] {
        require_ctx(ctx);
        LAYA_REQUIRE(out != nullptr, "null output pointer");
        auto* r = new laya_rotary();
        try {
            build_rotary(ctx, r, head_dim, theta, positions);
        } catch (...) {
            delete r;
            throw;
        }
        *out = r;
    });
}

int laya_rotary_destroy(laya_ctx* ctx, laya_rotary* rot) {
    return guarded([&] {
        require_ctx(ctx);
        if (!rot) return;
        free_rotary(ctx, rot);
        delete rot;
    });
}

int laya_rotary_apply(laya_ctx* ctx, const laya_rotary* rot, float* vec, int rows, const int* pos, int inverse) {
    return guarded([&] {
        require_ctx(ctx);
        LAYA_REQUIRE(rot && vec && pos && rows >= 0, "rotary: bad arguments");
        rotary_apply(ctx, rot->cos_t, rot->sin_t, rot->head_dim, vec, rows, pos, inverse);
    });
}

int laya_segments_create(laya_ctx* ctx, const int* start, const int* length, int nseg, laya_segments** out) {
    return guarded([&] {
        require_ctx(ctx);
        LAYA_REQUIRE(out && nseg >= 0 && (nseg == 0 || (start && length)), "segments: bad arguments");
        auto* s = new laya_segments();
        try {
            s->nseg = nseg;
            s->start.assign(start, start + nseg);
            s->length.assign(length, length + nseg);
            for (int i = 0; i < nseg; ++i) {
                LAYA_REQUIRE(s->start[i] >= 0 && s->length[i] >= 0 && (long)s->start[i] + s->length[i] <= INT32_MAX,
                             "segments: a segment with a negative start or length");
                s->max_len = std::max(s->max_len, s->length[i]);
                s->rows = std::max(s->rows, s->start[i] + s->length[i]);
            }
            const size_t bytes = sizeof(int) * (size_t)std::max(nseg, 1);
            s->d_start = static_cast<int*>(ctx->alloc(bytes));
            s->d_len = static_cast<int*>(ctx->alloc(bytes));
            s->blocks = attention_block_list(s->length);
            if (!s->blocks.empty()) s->d_blocks = static_cast<int*>(ctx->alloc(sizeof(int) * s->blocks.size()));
            // The host vectors live as long as the handle, which outlives the copies (destroy synchronises).
            if (nseg) {
                LAYA_HIP(hipMemcpyAsync(s->d_start, s->start.data(), bytes, hipMemcpyHostToDevice, ctx->stream));
                LAYA_HIP(hipMemcpyAsync(s->d_len, s->length.data(), bytes, hipMemcpyHostToDevice, ctx->stream));
            }
            if (s->d_blocks)
                LAYA_HIP(hipMemcpyAsync(s->d_blocks, s->blocks.data(), sizeof(int) * s->blocks.size(),
                                        hipMemcpyHostToDevice, ctx->stream));
        } catch (...) {
            if (s->d_start) ctx->release(s->d_start);
            if (s->d_len) ctx->release(s->d_len);
            if (s->d_blocks) ctx->release(s->d_blocks);
            delete s;
            throw;
        }
        *out = s;
    });
}

int laya_segments_destroy(laya_ctx* ctx, laya_segments* segs) {
    return guarded([&] {
        require_ctx(ctx);
        if (!segs) return;
        ctx->release(segs->d_start);  // release synchronises the stream first
        ctx->release(segs->d_len);
        if (segs->d_blocks) ctx->release(segs->d_blocks);
        delete segs;
    });
}

static AttentionArgs attention_args(const float* qkv, const laya_segments* segs, int hidden, int heads, float scale,
                                    int half_window, const laya_rotary* rot, float p_drop, uint64_t seed) {
    LAYA_REQUIRE(qkv && segs, "attention: null tensor or segment list");
    LAYA_REQUIRE(heads > 0 && hidden % heads == 0, "attention: hidden must be a multiple of heads");
    AttentionArgs a{};
    a.qkv = qkv;
    a.seg_start = segs->d_start;
    a.seg_len = segs->d_len;
    a.nseg = segs->nseg;
    a.max_len = segs->max_len;
    a.rows = segs->rows;
    a.blocks = segs->d_blocks;
    a.n_blocks = (int)segs->blocks.size();
    a.hidden = hidden;
    a.heads = heads;
    a.head_dim = hidden / heads;
    a.half_window = half_window;
    a.scale = scale;
    a.p_drop = p_drop;
    a.seed = seed;
    if (rot) {
        LAYA_REQUIRE(rot->head_dim == a.head_dim, "attention: rotary head_dim mismatch");
        a.cos_table = rot->cos_t;
        a.sin_table = rot->sin_t;
        a.positions = rot->positions;
    }
    for (int L : segs->length) a.keys += window_keys(L, half_window);
    return a;
}

int laya_attention_fwd(laya_ctx* ctx, const float* qkv, const laya_segments* segs, int hidden, int heads, float scale,
                       int half_window, const laya_rotary* rot, float p_drop, uint64_t seed, float* context,
                       float* lse) {
    return guarded([&] {
        require_ctx(ctx);
        LAYA_REQUIRE(context && lse, "attention: null output");
        const AttentionArgs a =
            attention_args(qkv, segs, hidden, heads, scale, half_window, rot, p_drop, seed);
        attention_fwd(ctx, a, context, lse);
    });
}

int laya_attention_bwd(laya_ctx* ctx, const float* qkv, const laya_segments* segs, int hidden, int heads, float scale,
                       int half_window, const laya_rotary* rot, float p_drop, uint64_t seed, const float* context,
                       const float* lse, const float* dcontext, float* dqkv) {
    return guarded([&] {
        require_ctx(ctx);
        LAYA_REQUIRE(dcontext && dqkv, "attention_bwd: null tensor");
        const AttentionArgs a =
            attention_args(qkv, segs, hidden, heads, scale, half_window, rot, p_drop, seed);
        if (!context || !lse) {
            // Ops.AttentionBackward recomputes each row's softmax from q and k (Ops.cs:390-394); here the
            // forward runs once more into scratch for the context and the row log-sum-exp.
            const size_t rows = (size_t)std::max(a.rows, 1);
            float* c = static_cast<float*>(ctx->workspace(6, sizeof(float) * rows * hidden));
            float* l = static_cast<float*>(ctx->workspace(7, sizeof(float) * rows * heads));
            attention_fwd(ctx, a, c, l);
            context = c;
            lse = l;
        }
        attention_bwd(ctx, a, a.rows, context, lse, dcontext, dqkv);
    });
}

// ------------------------------------------------------------------ operand magnitude words
//
// The _w variants: the same work as the entry points above, with the binding's magnitude word groups in
// place of measuring inputs, and the outputs' magnitudes folded into groups the call clears first.

namespace {

// An input's group as the two-piece products take it (known: no measuring pass), or none.
struct Given {
    unsigned char known = 1;
    AmaxRef ref;
    explicit Given(const unsigned* w) { ref = w ? AmaxRef{const_cast<unsigned*>(w), &known} : AmaxRef{}; }
};

// An output's group, cleared before the kernels that fold into it run (stream order).
unsigned* cleared(laya_ctx* ctx, unsigned* w) {
    if (w) fill(ctx, reinterpret_cast<float*>(w), 0.0f, (size_t)AMAX_GROUP);
    return w;
}

}  // namespace

int laya_amax(laya_ctx* ctx, const float* x, size_t n, unsigned* words) {
    return guarded([&] {
        require_ctx(ctx);
        LAYA_REQUIRE(words && (x || n == 0), "amax: null tensor");
        LAYA_REQUIRE(n <= (size_t)INT32_MAX * 4, "amax: too many elements");
        cleared(ctx, words);
        // As rows of 4 when the count allows (float4 loads), else one row per element.
        if (n % 4 == 0)
            absmax_into(ctx, x, (int)(n / 4), 4, 4, words);
        else
            absmax_into(ctx, x, (int)n, 1, 1, words);
    });
}

int laya_linear_fwd_w(laya_ctx* ctx, const float* x, int rows, int in, const float* W, int out, const float* b,
                      const float* residual, float* y, const unsigned* x_words, const unsigned* W_words,
                      unsigned* y_words) {
    return guarded([&] {
        require_ctx(ctx);
        LAYA_REQUIRE(rows >= 0 && in > 0 && out > 0, "linear: bad size");
        LAYA_REQUIRE(x && W && y, "linear: null tensor");
        const Given gx(x_words), gw(W_words);
        gemm(ctx, GemmLayout::NT, GemmEpilogue::Store, rows, out, in, x, in, W, in, y, out, b, residual, out, nullptr,
             nullptr, gx.ref, gw.ref, cleared(ctx, y_words));
    });
}

int laya_linear_bwd_w(laya_ctx* ctx, const float* x, const float* dy, int rows, int in, int out, const float* W,
                      float* dx, float* dW, float* db, const unsigned* x_words, const unsigned* dy_words,
                      const unsigned* W_words, unsigned* dx_words) {
    return guarded([&] {
        require_ctx(ctx);
        LAYA_REQUIRE(rows >= 0 && in > 0 && out > 0, "linear_bwd: bad size");
        LAYA_REQUIRE(dy && W, "linear_bwd: null tensor");
        LAYA_REQUIRE(!dW || x, "linear_bwd: dW needs x");
        LAYA_REQUIRE(!dx_words || dx, "linear_bwd: dx_words without dx");
        unsigned* w_dy = const_cast<unsigned*>(dy_words);
        if (db && !w_dy && dx && dW) {  // the bias gradient's pass measures dy for the pair, as laya_linear_bwd does
            w_dy = operand_ring_word(ctx);
            column_sum_add(ctx, dy, rows, out, db, w_dy);
            db = nullptr;
        }
        const Given gdy(w_dy), gx(x_words), gw(W_words);
        unsigned* wdx = cleared(ctx, dx_words);
        if (dx && dW) {
            gemm_backward_pair(ctx, rows, in, out, dy, W, x, dx, nullptr, dW, nullptr, nullptr, gdy.ref, gw.ref, gx.ref,
                               wdx);
        } else if (dx) {
            gemm(ctx, GemmLayout::NN, GemmEpilogue::Store, rows, in, out, dy, out, W, in, dx, in, nullptr, nullptr, 0,
                 nullptr, nullptr, gdy.ref, gw.ref, wdx);
        } else if (dW) {
            gemm(ctx, GemmLayout::TN, GemmEpilogue::Accumulate, out, in, rows, dy, out, x, in, dW, in, nullptr, nullptr,
                 0, nullptr, nullptr, gdy.ref, gx.ref);
        }
        if (db) column_sum_add(ctx, dy, rows, out, db);
    });
}

int laya_layernorm_fwd_w(laya_ctx* ctx, const float* x, int rows, int n, const float* w, const float* b, float eps,
                         float* y, float* mean, float* rstd, unsigned* y_words) {
    return guarded([&] {
        require_ctx(ctx);
        LAYA_REQUIRE(rows >= 0 && x && w && y, "layernorm: bad arguments");
        layernorm_fwd(ctx, x, rows, n, w, b, eps, y, mean, rstd, nullptr, nullptr, nullptr, nullptr,
                      cleared(ctx, y_words));
    });
}

int laya_layernorm_bwd_w(laya_ctx* ctx, const float* x, int rows, int n, const float* w, float eps, const float* dy,
                         float* dx, float* dgamma, float* dbeta, const float* mean, const float* rstd,
                         unsigned* dx_words) {
    return guarded([&] {
        require_ctx(ctx);
        LAYA_REQUIRE(rows >= 0 && x && w && dy && dx, "layernorm_bwd: bad arguments");
        LAYA_REQUIRE((mean == nullptr) == (rstd == nullptr), "layernorm_bwd: pass both mean and rstd, or neither");
        layernorm_bwd(ctx, x, rows, n, w, eps, dy, dx, dgamma, dbeta, mean, rstd, nullptr, cleared(ctx, dx_words));
    });
}

int laya_geglu_fwd_w(laya_ctx* ctx, const float* wide, int rows, int inter, float* act, unsigned* act_words) {
    return guarded([&] {
        require_ctx(ctx);
        LAYA_REQUIRE(rows >= 0 && inter > 0, "geglu: bad size");
        geglu_fwd(ctx, wide, rows, inter, act, nullptr, cleared(ctx, act_words));
    });
}

int laya_geglu_bwd_w(laya_ctx* ctx, const float* wide, const float* dact, int rows, int inter, float* dwide,
                     unsigned* dwide_words) {
    return guarded([&] {
        require_ctx(ctx);
        LAYA_REQUIRE(rows >= 0 && inter > 0, "geglu_bwd: bad size");
        geglu_bwd(ctx, wide, dact, rows, inter, dwide, cleared(ctx, dwide_words));
    });
}

int laya_attention_fwd_w(laya_ctx* ctx, const float* qkv, const laya_segments* segs, int hidden, int heads,
                         float scale, int half_window, const laya_rotary* rot, float p_drop, uint64_t seed,
                         float* context, float* lse, const unsigned* qkv_words, unsigned* context_words) {
    return guarded([&] {
        require_ctx(ctx);
        LAYA_REQUIRE(context && lse, "attention: null output");
        const AttentionArgs a = attention_args(qkv, segs, hidden, heads, scale, half_window, rot, p_drop, seed);
        const Given gq(qkv_words);
        attention_fwd(ctx, a, context, lse, nullptr, cleared(ctx, context_words), gq.ref);
    });
}

int laya_attention_bwd_w(laya_ctx* ctx, const float* qkv, const laya_segments* segs, int hidden, int heads,
                         float scale, int half_window, const laya_rotary* rot, float p_drop, uint64_t seed,
                         const float* context, const float* lse, const float* dcontext, float* dqkv,
                         const unsigned* qkv_words, const unsigned* dcontext_words, unsigned* dqkv_words) {
    return guarded([&] {
        require_ctx(ctx);
        LAYA_REQUIRE(dcontext && dqkv, "attention_bwd: null tensor");
        const AttentionArgs a = attention_args(qkv, segs, hidden, heads, scale, half_window, rot, p_drop, seed);
        const Given gq(qkv_words), gdo(dcontext_words);
        if (!context || !lse) {  // as laya_attention_bwd: the forward once more into scratch
            const size_t rows = (size_t)std::max(a.rows, 1);
            float* c = static_cast<float*>(ctx->workspace(6, sizeof(float) * rows * hidden));
            float* l = static_cast<float*>(ctx->workspace(7, sizeof(float) * rows * heads));
            attention_fwd(ctx, a, c, l, nullptr, nullptr, gq.ref);
            context = c;
            lse = l;
        }
        attention_bwd(ctx, a, a.rows, context, lse, dcontext, dqkv, cleared(ctx, dqkv_words), gq.ref, gdo.ref);
    });
}

int laya_embedding_fwd(laya_ctx* ctx, const int* ids, int n, const float* E, int vocab, int hidden, float* out,
                       int* bad_count) {
    return guarded([&] {
        require_ctx(ctx);
        LAYA_REQUIRE(n >= 0 && vocab > 0 && hidden > 0, "embedding: bad size");
        embedding_fwd(ctx, ids, n, E, vocab, hidden, out, bad_count);
    });
}

int laya_embedding_plan(const int* ids, int n, int vocab, int* sorted_pos, int* unique_ids, int* offsets,
                        int* n_unique) {
    return guarded([&] {
        LAYA_REQUIRE(n >= 0 && vocab > 0, "embedding_plan: bad size");
        // Counting sort by id: stable, so each id's positions stay in token order.
        std::vector<int> count((size_t)vocab + 1, 0);
        for (int t = 0; t < n; ++t) {
            const int id = ids[t];
            if ((unsigned)id >= (unsigned)vocab)
                throw Error(LAYA_ERR_OUT_OF_RANGE, "token id " + std::to_string(id) + " is outside the vocabulary.");
            count[id + 1]++;
        }
        for (int v = 0; v < vocab; ++v) count[v + 1] += count[v];
        std::vector<int> cursor(count.begin(), count.end() - 1);
        for (int t = 0; t < n; ++t) sorted_pos[cursor[ids[t]]++] = t;
        int u = 0;
        for (int v = 0; v < vocab; ++v) {
            if (count[v + 1] > count[v]) {
                unique_ids[u] = v;
                offsets[u] = count[v];
                ++u;
            }
        }
        offsets[u] = n;
        *n_unique = u;
    });
}

int laya_embedding_bwd(laya_ctx* ctx, const int* sorted_pos, const int* unique_ids, const int* offsets, int n_unique,
                       const float* d, int hidden, float* grad) {
    return guarded([&] {
        require_ctx(ctx);
        LAYA_REQUIRE(n_unique >= 0 && hidden > 0, "embedding_bwd: bad size");
        embedding_bwd(ctx, sorted_pos, unique_ids, offsets, n_unique, d, hidden, grad);
    });
}

int laya_gather_rows(laya_ctx* ctx, const float* src, const int* rows_idx, int n, int width, float* dst) {
    return guarded([&] {
        require_ctx(ctx);
        gather_rows(ctx, src, rows_idx, n, width, dst);
    });
}

int laya_type_embedding_fwd(laya_ctx* ctx, float* states, const int* qtype_of_row, int rows, int width,
                            const float* table) {
    return guarded([&] {
        require_ctx(ctx);
        LAYA_REQUIRE(rows >= 0 && width > 0 && states && qtype_of_row && table, "type_embedding_fwd: bad arguments");
        add_indexed_rows(ctx, states, qtype_of_row, rows, width, table);
    });
}

int laya_type_embedding_bwd(laya_ctx* ctx, const float* dstates, const int* qtype_of_row, int rows, int width,
                            float* grad) {
    return guarded([&] {
        require_ctx(ctx);
        LAYA_REQUIRE(rows >= 0 && width > 0 && dstates && qtype_of_row && grad, "type_embedding_bwd: bad arguments");
        type_embedding_bwd(ctx, dstates, qtype_of_row, rows, width, grad);
    });
}

int laya_scatter_add_rows(laya_ctx* ctx, const float* src, const int* rows_idx, int n, int width, float* dst) {
    return guarded([&] {
        require_ctx(ctx);
        scatter_add_rows(ctx, src, rows_idx, n, width, dst);
    });
}

int laya_softmax_ce_bwd(laya_ctx* ctx, const float* logits, const float* targets, const int* option_offsets,
                        int n_items, float ce_weight, float scale_, float* grad, float* loss) {
    return guarded([&] {
        require_ctx(ctx);
        softmax_ce_bwd(ctx, logits, targets, option_offsets, n_items, ce_weight, scale_, grad, loss);
    });
}

int laya_rlcd_objective(laya_ctx* ctx, const float* logits, const float* targets, const int* option_offsets,
                        const int* qtypes, int n_items, int total_options, int max_options, int groups,
                        const double* draws, double sigma, double spherical_weight, double rps_weight,
                        double ce_weight, double scale, float* grad, double* losses) {
    return guarded([&] {
        require_ctx(ctx);
        LAYA_REQUIRE(n_items == 0 || (logits && targets && option_offsets && qtypes && draws && grad && losses),
                     "rlcd: null tensor");
        rlcd_objective(ctx, logits, targets, option_offsets, qtypes, n_items, total_options, max_options, groups, draws,
                       sigma, spherical_weight, rps_weight, ce_weight, scale, grad, losses);
    });
}

int laya_grad_norm(laya_ctx* ctx, const float* grads, size_t n, double max_norm, double* norm_out, float* coef_out) {
    return guarded([&] {
        require_ctx(ctx);
        LAYA_REQUIRE(n == 0 || grads, "grad_norm: null gradients");
        if (!ctx->nonfinite) ctx->nonfinite = static_cast<int*>(ctx->alloc(64));
        grad_norm(ctx, grads, n, max_norm, norm_out, coef_out, ctx->nonfinite);
    });
}

int laya_grad_norm_status(laya_ctx* ctx) {
    return guarded([&] {
        require_ctx(ctx);
        if (!ctx->nonfinite) throw Error(LAYA_ERR_STATE, "grad_norm_status: no gradient norm was computed on this context");
        int flag = 0;
        LAYA_HIP(hipMemcpyAsync(&flag, ctx->nonfinite, sizeof(int), hipMemcpyDeviceToHost, ctx->stream));
        LAYA_HIP(hipStreamSynchronize(ctx->stream));
        if (flag)
            throw Error(LAYA_ERR_NOT_FINITE, "the gradient norm is not finite (a NaN or infinite gradient): the clip "
                                             "coefficient stayed 1, as Gradients.ClipByGlobalNorm leaves such "
                                             "gradients unscaled");
    });
}

int laya_adamw(laya_ctx* ctx, float* params, float* grads, float* m, float* v, int n_groups, const size_t* begin,
               const size_t* end, const double* lr, double beta1, double beta2, double eps, double weight_decay,
               int step, const float* coef, int zero_grads) {
    return guarded([&] {
        require_ctx(ctx);
        LAYA_REQUIRE(n_groups >= 0 && n_groups <= 4, "adamw: at most 4 groups");
        LAYA_REQUIRE(step >= 1, "adamw: step counts from 1");
        const double c1 = 1.0 - std::pow(beta1, step), c2 = 1.0 - std::pow(beta2, step);
        AdamGroups g{};
        g.n = n_groups;
        size_t n = 0;
        for (int k = 0; k < n_groups; ++k) {
            g.begin[k] = begin[k];
            g.end[k] = end[k];
            g.decay[k] = (float)(1.0 - lr[k] * weight_decay);
            g.step_size[k] = (float)(lr[k] / c1);
            n = std::max(n, end[k]);
        }
        adamw_arena(ctx, params, grads, m, v, n, g, (float)beta1, (float)beta2, (float)eps, (float)std::sqrt(c2), coef,
                    zero_grads);
    });
}

}  // extern "C"
