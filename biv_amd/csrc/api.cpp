// The C ABI of include/biv_hip.h: context, uploads (with the repacking into
// the device planes of common.hpp), the MoE layer, and the forward pass that
// queues the kernels of kernels.hip on the context's stream.
#include "../../include/biv_hip.h"
#include "common.hpp"
#include "layout.hpp"

#include <algorithm>
#include <atomic>
#include <new>
#include <cstdlib>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <string>
#include <thread>
#include <type_traits>
#include <vector>

using biv::DevMat;

struct biv_hip_weight {
    DevMat m;
};

struct biv_hip_experts {
    DevMat m;
};

// A dense SwiGLU FFN layer (Ffn::Dense, model.rs:239-246)
struct biv_hip_dense {
    const biv_hip_weight *gate, *up, *down;
    int E, ff;
};

struct biv_hip_moe {
    const biv_hip_weight *router, *sg, *su, *sd, *gi;
    const biv_hip_experts *gate, *up, *down;
    int k, n_expert, E, ff;
};

namespace {

// Device buffers of a dense forward, grown to the largest shape seen.
struct DenseScratch {
    int cap_T = 0, E = 0, ff = 0;
    std::vector<void *> bufs;
    int8_t *xq = nullptr, *aq = nullptr;
    float *xd = nullptr, *xs = nullptr, *act = nullptr, *ad = nullptr, *as = nullptr;
    float *h_stage = nullptr, *o_stage = nullptr;
};

// Device buffers of one forward, grown to the largest T seen.
struct Scratch {
    int cap_T = 0;
    std::vector<void *> bufs;
    int8_t *xq = nullptr;
    float *xd = nullptr, *xs = nullptr;
    float *logits = nullptr, *glogit = nullptr;
    float *act = nullptr;
    int8_t *aq = nullptr;
    float *ad = nullptr, *as = nullptr;
    float *y = nullptr;
    float *h_stage = nullptr, *o_stage = nullptr;
    uint8_t *xh = nullptr, *xl = nullptr; // bf16 halves of the matrix-core inputs
    int *counters = nullptr;
    biv::Dispatch dp{};
};

std::string g_create_error;

} // namespace

struct biv_hip_ctx {
    int device = 0;
    hipStream_t own = nullptr;
    hipStream_t stream = nullptr;
    std::string err;
    std::vector<void *> allocs;
    std::vector<biv_hip_weight *> weights;
    std::vector<biv_hip_experts *> experts;
    std::vector<biv_hip_moe *> layers;
    size_t bytes = 0;
    Scratch sc;
    DenseScratch dsc;
    std::vector<biv_hip_dense *> denses;
    // scratch shape: the widest layer seen
    int sc_E = 0, sc_ff = 0, sc_ne = 0, sc_k = 0;
    // stage timing (biv_hip_set_timing): one event before each stage and
    // one after the last, per forward, read back by biv_hip_stage_times
    bool timing = false;
    // down and combine in one launch at decode sizes (BIV_HIP_FUSED_DC=0 turns it off)
    bool fused_dc = true;
    bool gu_route = true; // small batches: the routing inside the gate/up launch
    int gu_route_t = 3;   // up to this many tokens (BIV_HIP_GU_ROUTE_T, at most 4)
    std::vector<hipEvent_t> ev_pool;
    std::vector<std::vector<hipEvent_t>> ev_fwd;
    // this GPU's copy of the no-allocation scratch (hipGetSymbolAddress)
    uint8_t *noalloc = nullptr;
};

namespace {

int fail(biv_hip_ctx *ctx, int code, const char *fmt, ...)
{
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    if (ctx) ctx->err = buf;
    else g_create_error = buf;
    return code;
}

} // namespace

// the context's error from the GGUF loader (gguf.cpp)
int biv_hip_fail_ext(biv_hip_ctx *ctx, int code, const char *msg) { return fail(ctx, code, "%s", msg); }

namespace {

int hip_fail(biv_hip_ctx *ctx, hipError_t e, const char *what)
{
    return fail(ctx, BIV_HIP_E_DEVICE, "%s: %s", what, hipGetErrorString(e));
}

#define HIP_TRY(ctx, call, what)                                                                                \
    do {                                                                                                        \
        hipError_t e_ = (call);                                                                                 \
        if (e_ != hipSuccess) return hip_fail(ctx, e_, what);                                                   \
    } while (0)

bool block_of(int ty, size_t &be, size_t &bb)
{
    switch (ty) {
    case BIV_GGML_F32: be = 1; bb = 4; return true;
    case BIV_GGML_F16:
    case BIV_GGML_BF16: be = 1; bb = 2; return true;
    case BIV_GGML_Q8_0: be = 32; bb = 34; return true;
    case BIV_GGML_Q4_K: be = 256; bb = 144; return true;
    case BIV_GGML_Q6_K: be = 256; bb = 210; return true;
    default: return false;
    }
}

// Types the expert kernels compute with.
bool expert_type_ok(int ty)
{
    return ty == BIV_GGML_Q8_0 || ty == BIV_GGML_Q4_K || ty == BIV_GGML_Q6_K || ty == BIV_GGML_BF16;
}

int dev_alloc(biv_hip_ctx *ctx, size_t bytes, uint8_t **out)
{
    void *p = nullptr;
    hipError_t e = hipMalloc(&p, bytes ? bytes : 1);
    if (e != hipSuccess) return fail(ctx, BIV_HIP_E_NOMEM, "hipMalloc(%zu): %s", bytes, hipGetErrorString(e));
    ctx->allocs.push_back(p);
    ctx->bytes += bytes;
    *out = static_cast<uint8_t *>(p);
    return 0;
}

// Repack n matrices of rows x cols from ggml rows (matrix e at
// data + e*stride + offset) into the planes of DevMat.
int upload_mat_impl(biv_hip_ctx *ctx, int ty, size_t cols, size_t rows, size_t n, const uint8_t *data, size_t stride,
                    size_t offset, DevMat &m);

// upload_mat_impl with host allocation failures (its repacking buffers)
// turned into an error code rather than an exception through the C ABI
int upload_mat(biv_hip_ctx *ctx, int ty, size_t cols, size_t rows, size_t n, const uint8_t *data, size_t stride,
               size_t offset, DevMat &m)
{
    if (cols > INT32_MAX || rows > INT32_MAX || n > INT32_MAX)
        return fail(ctx, BIV_HIP_E_INVALID, "shape %zux%zux%zu out of range", cols, rows, n);
    try {
        return upload_mat_impl(ctx, ty, cols, rows, n, data, stride, offset, m);
    } catch (const std::bad_alloc &) {
        return fail(ctx, BIV_HIP_E_NOMEM, "host memory for repacking %zux%zux%zu", cols, rows, n);
    }
}

int upload_mat_impl(biv_hip_ctx *ctx, int ty, size_t cols, size_t rows, size_t n, const uint8_t *data, size_t stride,
                    size_t offset, DevMat &m)
{
    size_t be, bb;
    if (!block_of(ty, be, bb)) return fail(ctx, BIV_HIP_E_TYPE, "no kernel for ggml type %d", ty);
    if (cols == 0 || rows == 0 || n == 0 || cols % be)
        return fail(ctx, BIV_HIP_E_INVALID, "shape %zux%zux%zu does not fit type %d", cols, rows, n, ty);
    if (!data) return fail(ctx, BIV_HIP_E_INVALID, "null weight data");
    const size_t row_bytes = cols / be * bb;
    const size_t nr = n * rows;
    m.ty = ty;
    m.cols = (int)cols;
    m.rows = (int)rows;
    m.n = (int)n;
    auto src_row = [&](size_t e, size_t r) { return data + e * stride + offset + r * row_bytes; };
    size_t qrow = 0, srow = 0, drow = 0;
    switch (ty) {
    case BIV_GGML_Q8_0: qrow = cols; srow = cols / 32 * 2; break;
    case BIV_GGML_Q4_K: qrow = cols / 2; srow = cols / 256 * 16; break;
    case BIV_GGML_Q6_K: qrow = cols / 256 * 192; srow = cols / 256 * 16; drow = cols / 256 * 2; break;
    case BIV_GGML_F32: qrow = row_bytes; srow = row_bytes; break; // chain layout + row-major copy
    default: qrow = row_bytes; break;
    }
    // the chain layouts (layout.hpp) need whole groups of blocks per row
    if ((ty == BIV_GGML_Q8_0 || ty == BIV_GGML_Q4_K) && cols % 256)
        return fail(ctx, BIV_HIP_E_INVALID, "width %zu: Q8_0/Q4_K rows must be a multiple of 256", cols);
    if (ty == BIV_GGML_Q6_K && cols % 512)
        return fail(ctx, BIV_HIP_E_INVALID, "width %zu: Q6_K rows must be a multiple of 512", cols);
    if ((ty == BIV_GGML_F32 || ty == BIV_GGML_BF16) && cols % 128)
        return fail(ctx, BIV_HIP_E_INVALID, "width %zu: F32/BF16 rows must be a multiple of 128", cols);
    const int K = (int)cols;
    std::vector<uint8_t> q(nr * qrow), s(nr * srow), d(nr * drow);
    // rows i0 .. i1 - 1 of the n * rows (disjoint ranges on several host threads)
    auto repack = [&](size_t i0, size_t i1) {
        for (size_t i = i0; i < i1; i++) {
            const size_t e = i / rows, r = i % rows;
            const uint8_t *src = src_row(e, r);
            uint8_t *qd = &q[i * qrow], *sd = srow ? &s[i * srow] : nullptr, *dd = drow ? &d[i * drow] : nullptr;
            switch (ty) {
            case BIV_GGML_Q8_0:
                for (int b = 0; b < K / 32; b++) {
                    const uint8_t *blk = src + 34 * b;
                    memcpy(sd + 2 * biv::lay::q8_scale(K, b), blk, 2);
                    for (int l = 0; l < 8; l++) memcpy(qd + 4 * biv::lay::q8_word(b, l), blk + 2 + 4 * l, 4);
                }
                break;
            case BIV_GGML_Q4_K:
                for (int sb = 0; sb < K / 256; sb++) {
                    const uint8_t *blk = src + 144 * sb;
                    memcpy(sd + 16 * sb, blk, 16); // d, dmin, the 12 scale bytes
                    for (int j = 0; j < 4; j++)
                        for (int l = 0; l < 8; l++)
                            memcpy(qd + 4 * biv::lay::q4k_word(4 * sb + j, l), blk + 16 + 32 * j + 4 * l, 4);
                }
                break;
            case BIV_GGML_Q6_K: {
                const int nsb = K / 256;
                uint8_t *qh = qd + 128 * nsb;
                for (int sb = 0; sb < nsb; sb++) {
                    const uint8_t *blk = src + 210 * sb;
                    for (int h = 0; h < 2; h++) {
                        const int qq = 2 * sb + h;
                        for (int l = 0; l < 8; l++) {
                            for (int pi = 0; pi < 2; pi++)
                                memcpy(qd + 4 * biv::lay::q6k_ql_word(qq, pi, l), blk + 64 * h + 32 * pi + 4 * l, 4);
                            memcpy(qh + 4 * biv::lay::q6k_qh_word(qq, l), blk + 128 + 32 * h + 4 * l, 4);
                        }
                        // sub-scale sc[8h + 2k + hsel] belongs to chain pi = k & 1 at
                        // step s = 2 qq + (k >> 1)
                        for (int k = 0; k < 4; k++)
                            for (int hsel = 0; hsel < 2; hsel++)
                                sd[biv::lay::q6k_sc(K, k & 1, hsel, 2 * qq + (k >> 1))] = blk[192 + 8 * h + 2 * k + hsel];
                    }
                    memcpy(dd + 2 * sb, blk + 208, 2);
                }
                break;
            }
            case BIV_GGML_F32:
                for (int e2 = 0; e2 < K; e2++)
                    memcpy(qd + 4 * biv::lay::f32_elem(e2 / 32, e2 % 32), src + 4 * e2, 4);
                memcpy(sd, src, row_bytes);
                break;
            case BIV_GGML_BF16: {
                // element 128 g + 16 m + L goes to (16 g + L) * 8 + m (lay::bf16_elem)
                uint16_t *dst16 = reinterpret_cast<uint16_t *>(qd);
                for (int g = 0; g < K / 128; g++)
                    for (int m = 0; m < 8; m++) {
                        uint16_t v[16];
                        memcpy(v, src + 2 * (128 * g + 16 * m), 32);
                        for (int L = 0; L < 16; L++) dst16[(16 * g + L) * 8 + m] = v[L];
                    }
                break;
            }
            default:
                memcpy(qd, src, row_bytes);
                break;
            }
        }
    };
    {
        const size_t nt = std::min<size_t>((nr + 255) / 256, std::max(1u, std::min(16u, std::thread::hardware_concurrency())));
        std::vector<std::thread> pool;
        for (size_t t = 1; t < nt; t++) pool.emplace_back(repack, nr * t / nt, nr * (t + 1) / nt);
        repack(0, nr / nt);
        for (auto &th : pool) th.join();
    }
    int rc;
    if ((rc = dev_alloc(ctx, q.size(), &m.q))) return rc;
    HIP_TRY(ctx, hipMemcpy(m.q, q.data(), q.size(), hipMemcpyHostToDevice), "upload");
    if (srow) {
        if ((rc = dev_alloc(ctx, s.size(), &m.s))) return rc;
        HIP_TRY(ctx, hipMemcpy(m.s, s.data(), s.size(), hipMemcpyHostToDevice), "upload");
    }
    if (drow) {
        if ((rc = dev_alloc(ctx, d.size(), &m.d))) return rc;
        HIP_TRY(ctx, hipMemcpy(m.d, d.data(), d.size(), hipMemcpyHostToDevice), "upload");
    }
    return 0;
}

template <class T> int sc_alloc(biv_hip_ctx *ctx, size_t count, T **out, std::vector<void *> *bufs = nullptr)
{
    void *p = nullptr;
    hipError_t e = hipMalloc(&p, count * sizeof(T) + 16);
    if (e != hipSuccess)
        return fail(ctx, BIV_HIP_E_NOMEM, "scratch hipMalloc(%zu): %s", count * sizeof(T), hipGetErrorString(e));
    (bufs ? bufs : &ctx->sc.bufs)->push_back(p);
    *out = static_cast<T *>(p);
    return 0;
}

void dense_scratch_free(biv_hip_ctx *ctx)
{
    for (void *p : ctx->dsc.bufs) (void)hipFree(p);
    ctx->dsc = DenseScratch{};
}

// Make the dense scratch fit T rows of a layer of E x ff.
int dense_scratch_fit(biv_hip_ctx *ctx, const biv_hip_dense *d, int T)
{
    DenseScratch &s = ctx->dsc;
    if (T <= s.cap_T && d->E <= s.E && d->ff <= s.ff) return 0;
    HIP_TRY(ctx, hipStreamSynchronize(ctx->stream), "sync");
    const int cap = std::max(T, std::max(s.cap_T, 8)), E = std::max(d->E, s.E), ff = std::max(d->ff, s.ff);
    dense_scratch_free(ctx);
    const size_t Tc = cap;
    auto *b = &s.bufs;
    int rc = 0;
    rc = rc ? rc : sc_alloc(ctx, Tc * E, &s.xq, b);
    rc = rc ? rc : sc_alloc(ctx, Tc * E / 32, &s.xd, b);
    rc = rc ? rc : sc_alloc(ctx, Tc * E / 32, &s.xs, b);
    rc = rc ? rc : sc_alloc(ctx, Tc * ff, &s.act, b);
    rc = rc ? rc : sc_alloc(ctx, Tc * ff, &s.aq, b);
    rc = rc ? rc : sc_alloc(ctx, Tc * ff / 32, &s.ad, b);
    rc = rc ? rc : sc_alloc(ctx, Tc * ff / 32, &s.as, b);
    rc = rc ? rc : sc_alloc(ctx, Tc * E, &s.h_stage, b);
    rc = rc ? rc : sc_alloc(ctx, Tc * E, &s.o_stage, b);
    if (rc) {
        dense_scratch_free(ctx);
        return rc;
    }
    s.cap_T = cap;
    s.E = E;
    s.ff = ff;
    return 0;
}

// dense_ffn (model.rs:1118-1126) of T rows on the context's stream:
// Input::q8 of h (for quantised gate/up), gate/up with the SwiGLU, Q8 of
// the intermediate (for a quantised down), down into out or added to it.
int dense_forward(biv_hip_ctx *ctx, const biv_hip_dense *d, const float *h, int T, float *out, unsigned flags)
{
    if (T == 0) return 0;
    int rc = dense_scratch_fit(ctx, d, T);
    if (rc) return rc;
    DenseScratch &s = ctx->dsc;
    hipStream_t st = ctx->stream;
    const int E = d->E, ff = d->ff;
    const DevMat &G = d->gate->m, &U = d->up->m, &D = d->down->m;
    if (G.ty != biv::T_BF16)
        HIP_TRY(ctx, biv::launch_quant_rows(h, T * E / 32, E, s.xq, s.xd, s.xs, st), "quantise h");
    biv::LongArgs g{};
    g.a = G;
    g.b = U;
    g.xq = s.xq;
    g.xd = s.xd;
    g.xs = s.xs;
    g.xf = h;
    g.out = s.act;
    g.T = T;
    g.K = E;
    HIP_TRY(ctx, biv::launch_long_mv(g, 1, st), "dense gate/up");
    if (D.ty != biv::T_BF16)
        HIP_TRY(ctx, biv::launch_quant_rows(s.act, T * ff / 32, ff, s.aq, s.ad, s.as, st), "quantise act");
    biv::LongArgs dn{};
    dn.a = D;
    dn.xq = s.aq;
    dn.xd = s.ad;
    dn.xs = s.as;
    dn.xf = s.act;
    dn.out = out;
    dn.T = T;
    dn.K = ff;
    dn.add = (flags & BIV_HIP_ADD) != 0;
    HIP_TRY(ctx, biv::launch_long_mv(dn, 0, st), "dense down");
    return 0;
}

void scratch_free(biv_hip_ctx *ctx)
{
    for (void *p : ctx->sc.bufs) (void)hipFree(p);
    ctx->sc = Scratch{};
}

// The buffers of one forward of up to cap tokens of a layer of the given
// shape: take(ptr, count) is called for each, in one fixed order.
template <class Take>
int scratch_plan(Scratch &s, size_t cap, size_t E, size_t ff, size_t ne, size_t k, Take take)
{
    const size_t P = cap * k, R = P + cap;
    int rc = 0;
    rc = rc ? rc : take(s.xq, cap * E);
    rc = rc ? rc : take(s.xd, cap * E / 32);
    rc = rc ? rc : take(s.xs, cap * E / 32);
    rc = rc ? rc : take(s.logits, cap * ne);
    rc = rc ? rc : take(s.glogit, cap);
    rc = rc ? rc : take(s.act, R * ff);
    rc = rc ? rc : take(s.aq, R * ff);
    rc = rc ? rc : take(s.ad, R * ff / 32);
    rc = rc ? rc : take(s.as, R * ff / 32);
    rc = rc ? rc : take(s.y, R * E);
    rc = rc ? rc : take(s.h_stage, cap * E);
    // bf16 halves of h or of the intermediate, whichever is larger
    rc = rc ? rc : take(s.xh, 2 * std::max(cap * E, R * ff));
    rc = rc ? rc : take(s.xl, 2 * std::max(cap * E, R * ff));
    rc = rc ? rc : take(s.o_stage, cap * E);
    rc = rc ? rc : take(s.dp.slots, ne + P); // >= max_slots(ne, P, chunk)
    rc = rc ? rc : take(s.dp.pair_tok, P);
    rc = rc ? rc : take(s.dp.pair_exp, P);
    rc = rc ? rc : take(s.dp.pair_w, P);
    rc = rc ? rc : take(s.dp.tok_pairs, P);
    rc = rc ? rc : take(s.dp.ids, P);
    rc = rc ? rc : take(s.dp.wts, P);
    rc = rc ? rc : take(s.counters, biv::route_work_ints((int)cap));
    return rc;
}

// Make the scratch fit T tokens of layer m.
int scratch_fit(biv_hip_ctx *ctx, const biv_hip_moe *m, int T)
{
    Scratch &s = ctx->sc;
    if (T <= s.cap_T && m->E <= ctx->sc_E && m->ff <= ctx->sc_ff && m->n_expert <= ctx->sc_ne && m->k <= ctx->sc_k)
        return 0;
    // wait for queued work before freeing what it may use
    HIP_TRY(ctx, hipStreamSynchronize(ctx->stream), "sync");
    scratch_free(ctx);
    const int cap = T < 16 ? 16 : T;
    ctx->sc_E = std::max(ctx->sc_E, m->E);
    ctx->sc_ff = std::max(ctx->sc_ff, m->ff);
    ctx->sc_ne = std::max(ctx->sc_ne, m->n_expert);
    ctx->sc_k = std::max(ctx->sc_k, m->k);
    int rc = scratch_plan(s, cap, ctx->sc_E, ctx->sc_ff, ctx->sc_ne, ctx->sc_k,
                          [&](auto *&p, size_t count) { return sc_alloc(ctx, count, &p); });
    if (rc) {
        scratch_free(ctx);
        return rc;
    }
    s.cap_T = cap;
    return 0;
}

// The scratch of biv_hip_moe_forward_device_noalloc: device memory the
// library holds from load to process end, one copy per GPU, so that this
// entry point calls no allocator.  Host code never passes `scratch` itself
// (on the host it names a stand-in, not a device address): each context
// resolves its GPU's copy with hipGetSymbolAddress at creation and uses that.
constexpr size_t NOALLOC_BYTES = (size_t)48 << 20;
static __device__ __align__(256) uint8_t scratch[NOALLOC_BYTES];

// The context that holds each GPU's copy of `scratch`: the first to call the
// no-allocation entry point on that device, until it is destroyed.  Another
// context calling it on the same device gets BIV_HIP_E_BUSY rather than a
// silent race over the same bytes.
constexpr int NOALLOC_MAX_DEVICES = 64;
std::atomic<biv_hip_ctx *> g_noalloc_owner[NOALLOC_MAX_DEVICES];

int noalloc_claim(biv_hip_ctx *ctx)
{
    if (ctx->device >= NOALLOC_MAX_DEVICES)
        return fail(ctx, BIV_HIP_E_INVALID, "no-allocation scratch: device %d past %d", ctx->device,
                    NOALLOC_MAX_DEVICES);
    biv_hip_ctx *owner = nullptr;
    if (g_noalloc_owner[ctx->device].compare_exchange_strong(owner, ctx) || owner == ctx) return 0;
    return fail(ctx, BIV_HIP_E_BUSY, "the no-allocation scratch of device %d is held by another context",
                ctx->device);
}

void noalloc_release(biv_hip_ctx *ctx)
{
    if (ctx->device < NOALLOC_MAX_DEVICES) {
        biv_hip_ctx *mine = ctx;
        g_noalloc_owner[ctx->device].compare_exchange_strong(mine, nullptr);
    }
}

// Carve the buffers of a forward of T tokens of layer m out of the context's
// copy of `scratch` (256-byte aligned pieces).  No allocation.
int noalloc_scratch(biv_hip_ctx *ctx, const biv_hip_moe *m, int T, Scratch &s);

int noalloc_scratch(biv_hip_ctx *ctx, const biv_hip_moe *m, int T, Scratch &s)
{
    size_t off = 0;
    bool fits = true;
    auto take = [&](auto *&p, size_t count) {
        using Elem = std::remove_reference_t<decltype(*p)>;
        off = (off + 255) & ~(size_t)255;
        const size_t bytes = count * sizeof(Elem) + 16;
        if (off + bytes > NOALLOC_BYTES) fits = false;
        p = fits ? reinterpret_cast<Elem *>(ctx->noalloc + off) : nullptr;
        off += bytes;
        return 0;
    };
    s = Scratch{};
    scratch_plan(s, (size_t)T, m->E, m->ff, m->n_expert, m->k, take);
    if (!fits)
        return fail(ctx, BIV_HIP_E_INVALID,
                    "%d tokens of this layer need %zu bytes of scratch; the no-allocation entry point has %zu", T, off,
                    NOALLOC_BYTES);
    s.cap_T = T;
    return 0;
}

struct Dumps {
    int32_t *gate = nullptr, *up = nullptr, *down = nullptr;
    bool act = false; // the quantised intermediate is read back
};

// T from which BF16 layers use the matrix cores
constexpr int MFMA_MIN_T = 64;

constexpr int N_STAGES = 6; // router (+ quantise h), route + dispatch, gate/up, quantise act, down, combine

// The stage markers of one forward when timing is on.
struct StageMarks {
    biv_hip_ctx *ctx;
    std::vector<hipEvent_t> ev;
    explicit StageMarks(biv_hip_ctx *c) : ctx(c) {}
    hipError_t mark()
    {
        if (!ctx->timing) return hipSuccess;
        hipEvent_t e;
        if (!ctx->ev_pool.empty()) {
            e = ctx->ev_pool.back();
            ctx->ev_pool.pop_back();
        } else {
            hipError_t err = hipEventCreate(&e);
            if (err != hipSuccess) return err;
        }
        ev.push_back(e);
        return hipEventRecord(e, ctx->stream);
    }
    ~StageMarks()
    {
        if (!ctx->timing) return;
        if (ev.size() == N_STAGES + 1) ctx->ev_fwd.push_back(ev);
        else
            for (auto e : ev) ctx->ev_pool.push_back(e);
    }
};

// Queue the whole block: h and out are device pointers.  With only >= 0,
// queue stage `only` alone (for measurement: the scratch holds a forward's
// routing of the same T).
// With norm_w, h is the residual x and the block takes rms_norm(x) with
// these weights (the post_norm of model.rs:786-790), formed by the router
// launch into the scratch row block h_stage.
// ext: run in these scratch buffers (sized for T) instead of the context's.
int forward(biv_hip_ctx *ctx, const biv_hip_moe *m, const float *h, int T, float *out, unsigned flags,
            const Dumps &dm, int only = -1, const float *norm_w = nullptr, float eps = 0.0f, Scratch *ext = nullptr)
{
    if (T == 0) return 0;
    int rc = ext ? 0 : scratch_fit(ctx, m, T);
    if (rc) return rc;
    StageMarks mk(ctx);
#define MARK() HIP_TRY(ctx, only < 0 ? mk.mark() : hipSuccess, "timing event")
    auto run = [&](int stage) { return only < 0 || only == stage; };
    Scratch &s = ext ? *ext : ctx->sc;
    hipStream_t st = ctx->stream;
    const int E = m->E, ff = m->ff, ne = m->n_expert, k = m->k;
    const int P = T * k;
    const bool has_shared = m->sg != nullptr;
    int *ctr_rs = s.counters;
    // BF16 matrices at prefill sizes run on the matrix cores (mfma.hip), when
    // the routed and shared matrices of that half are all BF16
    const bool mf_gu = T >= MFMA_MIN_T && m->gate->m.ty == biv::T_BF16 && (!has_shared || m->sg->m.ty == biv::T_BF16);
    const bool mf_dn = T >= MFMA_MIN_T && m->down->m.ty == biv::T_BF16 && (!has_shared || m->sd->m.ty == biv::T_BF16);
    // pairs per slot: decode keeps an expert's tokens together; larger passes
    // cut them so that hot experts and the shared expert spread over the GPU
    // (a matrix-core workgroup takes a whole slot: 256 BF16 pairs, 16 Q8_0)
    // quantised matrices at prefill sizes run on the int8 matrix cores: gate/up
    // when gate and up are Q8_0 or Q4_K (each pair of one type, routed and
    // shared), down when the routed and shared down matrices are Q8_0 or Q6_K
    auto gu_ok = [](int g, int u) { return g == u && (g == biv::T_Q8_0 || g == biv::T_Q4K); };
    const bool mq_gu = T >= MFMA_MIN_T && gu_ok(m->gate->m.ty, m->up->m.ty) &&
                       (!has_shared || gu_ok(m->sg->m.ty, m->su->m.ty));
    auto dn_ok = [](int t) { return t == biv::T_Q8_0 || t == biv::T_Q6K; };
    const bool mq_dn = T >= MFMA_MIN_T && dn_ok(m->down->m.ty) && (!has_shared || dn_ok(m->sd->m.ty));
    const int chunk = mq_gu || mq_dn ? biv::MFMA_Q8_TILE : mf_gu || mf_dn ? biv::MFMA_TOK_TILE : T <= 64 ? 64 : 16;
    const int u_max = biv::max_slots(ne, P, chunk);
    s.dp.slot_cap = u_max;

    biv::RouterArgs ra{};
    ra.router = reinterpret_cast<const float *>(m->router->m.q);
    ra.router_rm = reinterpret_cast<const float *>(m->router->m.s);
    ra.gate_inp = has_shared ? reinterpret_cast<const float *>(m->gi->m.q) : nullptr;
    ra.gate_rm = has_shared ? reinterpret_cast<const float *>(m->gi->m.s) : nullptr;
    ra.n_expert = ne;
    ra.E = E;
    ra.T = T;
    ra.h = h;
    ra.logits = s.logits;
    ra.glogit = s.glogit;
    ra.xq = s.xq;
    ra.xd = s.xd;
    ra.xs = s.xs;
    ra.norm_w = norm_w;
    ra.eps = eps;
    ra.hn = s.h_stage;
    // BF16 gate/up on the matrix cores from the pre-pass's bf16 halves of h
    const bool prep_split = mf_gu && T >= biv::prep_min_t();
    if (prep_split) {
        ra.xh = reinterpret_cast<uint4 *>(s.xh);
        ra.xl = reinterpret_cast<uint4 *>(s.xl);
    }
    // BF16 gate/up (routed and shared) read h as f32 or as its bf16 halves:
    // nothing reads the Q8 of h, so the router launch leaves it out
    if (m->gate->m.ty == biv::T_BF16 && (!has_shared || m->sg->m.ty == biv::T_BF16)) ra.xq = nullptr;
    if (norm_w) {
        if (h == s.h_stage) return fail(ctx, BIV_HIP_E_INVALID, "post_norm input aliases its output");
        h = s.h_stage; // every later use of h takes the normalised rows
    }
    // Small batches (decode): every gate/up workgroup derives its slot from
    // the logits (the same in each) and a routing workgroup in the same
    // launch writes the routes and dispatch records, so there is no route
    // launch.  Up to GU_ROUTE_T tokens: each workgroup's own routing delays
    // its weight loads, which past 3 tokens costs more than the launch
    // (measured: T = 1, 2, 3 20.5 / 26.8 / 34.4 against 21.0 / 29.9 / 35.1 us
    // per Q8_0 layer with the route launch; T = 4, 5, 8 42.6 / 55 / 78
    // against 40.3 / 45.7 / 58).  At most 4 (a wave per token).  BF16
    // gate/up, which stages f32 rows, for one token.  The taps take the
    // separate launches.
    const bool bf_gu = m->gate->m.ty == biv::T_BF16;
    const bool gu_route = ctx->gu_route && T <= ctx->gu_route_t && (T == 1 || !bf_gu) && !mf_gu && !mq_gu &&
                          !dm.gate && !dm.up && !dm.down && k <= 8 && ne >= k && ne <= 256 && chunk == 64;
    MARK();
    if (run(0)) HIP_TRY(ctx, biv::launch_router(ra, st), "router");
    MARK();
    if (run(1) && !gu_route) HIP_TRY(ctx, biv::launch_route_sort(s.logits, ne, k, T, chunk, s.dp, ctr_rs, st), "route and dispatch");
    MARK();

    biv::MvArgs a{};
    a.a = m->gate->m;
    a.b = m->up->m;
    if (has_shared) {
        a.sa = m->sg->m;
        a.sb = m->su->m;
    }
    a.xq = s.xq;
    a.xd = s.xd;
    a.xs = s.xs;
    a.xf = h; // BF16 matrices take the f32 rows (Input::F32, ops.rs:45-60)
    a.dp = s.dp;
    a.out = s.act;
    a.dump_a = dm.gate;
    a.dump_b = dm.up;
    a.T = T;
    a.P = P;
    a.u_max = u_max;
    if (gu_route) {
        a.logits = s.logits;
        a.n_expert = ne;
        a.k = k;
    }
    if (run(2)) {
        if (mf_gu) {
            biv::MfArgs g{};
            g.a = a.a;
            g.b = a.b;
            g.sa = a.sa;
            g.sb = a.sb;
            g.xh = reinterpret_cast<const uint4 *>(s.xh);
            g.xl = reinterpret_cast<const uint4 *>(s.xl);
            g.dp = s.dp;
            g.out = s.act;
            if (mf_dn) {
                // the intermediate goes out as the bf16 halves the down
                // kernel reads, in the f32 intermediate's bytes (no split launch)
                g.out = nullptr;
                g.xo_h = reinterpret_cast<uint4 *>(s.act);
                g.xo_l = g.xo_h + (size_t)(has_shared ? P + T : P) * ff / 8;
            }
            g.T = T;
            g.P = P;
            g.u_max = u_max;
            g.chunk = chunk;
            g.sh_chunk = biv::MFMA_TOK_TILE;
            if (!prep_split) HIP_TRY(ctx, biv::launch_split_bf16(h, T, E, s.xh, s.xl, st), "split h");
            HIP_TRY(ctx, biv::launch_mfma_gateup(g, st), "expert gate/up (mfma)");
        } else if (mq_gu) {
            a.sh_chunk = biv::MFMA_Q8_TILE;
            HIP_TRY(ctx, biv::launch_mfma_gateup_exact(a, st), "expert gate/up (int8 mfma)");
        } else {
            HIP_TRY(ctx, biv::launch_gateup(a, st), "expert gate/up");
        }
    }
    MARK();
    const int rows_act = has_shared ? P + T : P;
    // For small T the down kernel quantises its rows itself, saving a launch
    // (every workgroup of a slot quantises the slot's rows: past a few tokens
    // that costs more than it saves), unless a down matrix is Q4_K, whose
    // mins need the block sums.  The taps still want the rows apart.
    // BF16 down matrices take the f32 intermediate as it is (no Q8, as
    // uses_f32_act, quant.rs:75-77).
    const bool down_f32 = m->down->m.ty == biv::T_BF16 && (!has_shared || m->sd->m.ty == biv::T_BF16);
    const bool down_q8 = m->down->m.ty != biv::T_BF16 || (has_shared && m->sd->m.ty != biv::T_BF16);
    const bool fused_quant = T <= 16 && !down_f32 && m->down->m.ty != biv::T_Q4K &&
                             (!has_shared || (m->sd->m.ty != biv::T_Q4K && m->sd->m.ty != biv::T_BF16));
    // Decode sizes: down and combine in one launch (each expert's pairs in
    // one slot; Q8_0 or Q6_K down matrices, the shared one of the same kind)
    const int dty = m->down->m.ty;
    const bool fused_dc = ctx->fused_dc && T <= 16 && T <= chunk && (dty == biv::T_Q8_0 || dty == biv::T_Q6K) &&
                          m->down->m.rows % 8 == 0 &&
                          (!has_shared || (m->sd->m.ty == dty && m->sd->m.cols == m->down->m.cols &&
                                           m->sd->m.rows == m->down->m.rows));
    if (down_q8 && (!(fused_quant || fused_dc) || dm.act) && run(3))
        HIP_TRY(ctx, biv::launch_quant_rows(s.act, rows_act * ff / 32, ff, s.aq, s.ad, s.as, st), "quantise act");
    MARK();

    biv::MvArgs d{};
    d.a = m->down->m;
    if (has_shared) d.sa = m->sd->m;
    d.xq = s.aq;
    d.xd = s.ad;
    d.xs = s.as;
    d.xf = s.act;
    d.qx = fused_quant;
    d.dp = s.dp;
    d.out = s.y;
    d.dump_a = dm.down;
    d.T = T;
    d.P = P;
    d.u_max = u_max;
    if (fused_dc) {
        if (run(4)) {
            biv::DownCombineArgs c{};
            c.a = m->down->m;
            if (has_shared) c.sa = m->sd->m;
            c.xf = s.act;
            c.dp = s.dp;
            c.glogit = s.glogit;
            c.out = out;
            c.dump = dm.down;
            c.T = T;
            c.P = P;
            c.k = k;
            c.add = (flags & BIV_HIP_ADD) != 0;
            HIP_TRY(ctx, biv::launch_down_combine(c, st), "expert down + combine");
        }
        MARK();
        MARK();
        return 0;
    }
    if (run(4)) {
        if (mf_dn) {
            biv::MfArgs g{};
            g.a = d.a;
            g.sa = d.sa;
            if (mf_gu) {
                // gate/up wrote the halves (in the intermediate's bytes)
                g.xh = reinterpret_cast<const uint4 *>(s.act);
                g.xl = g.xh + (size_t)(has_shared ? P + T : P) * ff / 8;
            } else {
                g.xh = reinterpret_cast<const uint4 *>(s.xh);
                g.xl = reinterpret_cast<const uint4 *>(s.xl);
            }
            g.dp = s.dp;
            g.out = s.y;
            g.T = T;
            g.P = P;
            g.u_max = u_max;
            g.chunk = chunk;
            g.sh_chunk = biv::MFMA_TOK_TILE;
            if (!mf_gu)
                HIP_TRY(ctx, biv::launch_split_bf16(s.act, has_shared ? P + T : P, ff, s.xh, s.xl, st), "split act");
            HIP_TRY(ctx, biv::launch_mfma_down(g, st), "expert down (mfma)");
        } else if (mq_dn) {
            d.sh_chunk = biv::MFMA_Q8_TILE;
            HIP_TRY(ctx, biv::launch_q8_mfma_down(d, st), "expert down (int8 mfma)");
        } else {
            HIP_TRY(ctx, biv::launch_down(d, st), "expert down");
        }
    }
    MARK();
    if (run(5))
        HIP_TRY(ctx,
                biv::launch_combine(s.y, s.dp, s.glogit, has_shared, T, P, k, E, out, (flags & BIV_HIP_ADD) != 0,
                                    st),
                "combine");
    MARK();
#undef MARK
    return 0;
}

} // namespace

extern "C" {

int biv_hip_create(int device, biv_hip_ctx **out)
{
    if (!out) return fail(nullptr, BIV_HIP_E_INVALID, "null output pointer");
    *out = nullptr;
    int n = 0;
    hipError_t e = hipGetDeviceCount(&n);
    if (e != hipSuccess || n == 0) return fail(nullptr, BIV_HIP_E_DEVICE, "no HIP device (%s)", hipGetErrorString(e));
    if (device < 0 || device >= n) return fail(nullptr, BIV_HIP_E_INVALID, "device %d of %d", device, n);
    hipDeviceProp_t prop;
    e = hipGetDeviceProperties(&prop, device);
    if (e != hipSuccess) return fail(nullptr, BIV_HIP_E_DEVICE, "device properties: %s", hipGetErrorString(e));
    if (strncmp(prop.gcnArchName, "gfx950", 6) != 0)
        return fail(nullptr, BIV_HIP_E_DEVICE, "device %d is %s; this library is built for gfx950", device,
                    prop.gcnArchName);
    e = hipSetDevice(device);
    if (e != hipSuccess) return fail(nullptr, BIV_HIP_E_DEVICE, "hipSetDevice: %s", hipGetErrorString(e));
    auto *ctx = new biv_hip_ctx();
    ctx->device = device;
    e = hipStreamCreateWithFlags(&ctx->own, hipStreamNonBlocking);
    if (e != hipSuccess) {
        delete ctx;
        return fail(nullptr, BIV_HIP_E_DEVICE, "stream: %s", hipGetErrorString(e));
    }
    ctx->stream = ctx->own;
    // the device address of this GPU's no-allocation scratch (device is current)
    e = hipGetSymbolAddress(reinterpret_cast<void **>(&ctx->noalloc), HIP_SYMBOL(scratch));
    if (e != hipSuccess) {
        (void)hipStreamDestroy(ctx->own);
        delete ctx;
        return fail(nullptr, BIV_HIP_E_DEVICE, "no-allocation scratch address: %s", hipGetErrorString(e));
    }
    const char *fdc = getenv("BIV_HIP_FUSED_DC");
    ctx->fused_dc = !(fdc && fdc[0] == '0');
    const char *gur = getenv("BIV_HIP_GU_ROUTE");
    ctx->gu_route = !(gur && gur[0] == '0');
    if (const char *gt = getenv("BIV_HIP_GU_ROUTE_T")) ctx->gu_route_t = std::max(1, std::min(4, atoi(gt)));
    *out = ctx;
    return 0;
}

void biv_hip_destroy(biv_hip_ctx *ctx)
{
    if (!ctx) return;
    (void)hipSetDevice(ctx->device);
    (void)hipStreamSynchronize(ctx->stream);
    noalloc_release(ctx);
    scratch_free(ctx);
    for (auto &v : ctx->ev_fwd)
        for (auto e : v) (void)hipEventDestroy(e);
    for (auto e : ctx->ev_pool) (void)hipEventDestroy(e);
    for (void *p : ctx->allocs) (void)hipFree(p);
    for (auto *w : ctx->weights) delete w;
    for (auto *x : ctx->experts) delete x;
    for (auto *l : ctx->layers) delete l;
    for (auto *l : ctx->denses) delete l;
    dense_scratch_free(ctx);
    if (ctx->own) (void)hipStreamDestroy(ctx->own);
    delete ctx;
}

const char *biv_hip_last_error(const biv_hip_ctx *ctx) { return ctx ? ctx->err.c_str() : g_create_error.c_str(); }

int biv_hip_set_stream(biv_hip_ctx *ctx, void *stream)
{
    if (!ctx) return BIV_HIP_E_INVALID;
    ctx->stream = stream ? static_cast<hipStream_t>(stream) : ctx->own;
    return 0;
}

int biv_hip_sync(biv_hip_ctx *ctx)
{
    if (!ctx) return BIV_HIP_E_INVALID;
    HIP_TRY(ctx, hipStreamSynchronize(ctx->stream), "sync");
    return 0;
}

int biv_hip_upload_weight(biv_hip_ctx *ctx, int ggml_type, size_t cols, size_t rows, const void *data,
                          biv_hip_weight **out)
{
    if (!ctx || !out) return BIV_HIP_E_INVALID;
    HIP_TRY(ctx, hipSetDevice(ctx->device), "hipSetDevice");
    auto *w = new biv_hip_weight();
    int rc = upload_mat(ctx, ggml_type, cols, rows, 1, static_cast<const uint8_t *>(data), 0, 0, w->m);
    if (rc) {
        delete w;
        return rc;
    }
    ctx->weights.push_back(w);
    *out = w;
    return 0;
}

int biv_hip_upload_experts(biv_hip_ctx *ctx, int ggml_type, size_t cols, size_t rows, size_t n_expert,
                           const void *data, size_t stride, size_t offset, biv_hip_experts **out)
{
    if (!ctx || !out) return BIV_HIP_E_INVALID;
    HIP_TRY(ctx, hipSetDevice(ctx->device), "hipSetDevice");
    size_t be, bb;
    if (!block_of(ggml_type, be, bb)) return fail(ctx, BIV_HIP_E_TYPE, "no kernel for ggml type %d", ggml_type);
    if (cols % be == 0 && stride < offset + rows * (cols / be * bb) && n_expert > 1)
        return fail(ctx, BIV_HIP_E_INVALID, "expert stride %zu is smaller than a matrix", stride);
    auto *x = new biv_hip_experts();
    int rc = upload_mat(ctx, ggml_type, cols, rows, n_expert, static_cast<const uint8_t *>(data), stride, offset,
                        x->m);
    if (rc) {
        delete x;
        return rc;
    }
    ctx->experts.push_back(x);
    *out = x;
    return 0;
}

int biv_hip_moe_create(biv_hip_ctx *ctx, const biv_hip_weight *router, const biv_hip_experts *gate,
                       const biv_hip_experts *up, const biv_hip_experts *down, const biv_hip_weight *shared_gate,
                       const biv_hip_weight *shared_up, const biv_hip_weight *shared_down,
                       const biv_hip_weight *gate_inp, int k, biv_hip_moe **out)
{
    if (!ctx || !out) return BIV_HIP_E_INVALID;
    if (!router || !gate || !up || !down) return fail(ctx, BIV_HIP_E_INVALID, "router and experts are required");
    const int n_shared = !!shared_gate + !!shared_up + !!shared_down + !!gate_inp;
    if (n_shared != 0 && n_shared != 4)
        return fail(ctx, BIV_HIP_E_INVALID, "the shared expert needs gate, up, down and gate_inp");
    const DevMat &g = gate->m, &u = up->m, &d = down->m, &r = router->m;
    const int E = g.cols, ff = g.rows, ne = g.n;
    if (r.ty != BIV_GGML_F32) return fail(ctx, BIV_HIP_E_TYPE, "router type %d: only F32 routers", r.ty);
    if (!expert_type_ok(g.ty) || !expert_type_ok(u.ty) || !expert_type_ok(d.ty))
        return fail(ctx, BIV_HIP_E_TYPE, "expert types %d/%d/%d: kernels exist for Q8_0, Q4_K, Q6_K, BF16", g.ty,
                    u.ty, d.ty);
    if (g.ty != u.ty) return fail(ctx, BIV_HIP_E_TYPE, "gate and up experts must share a type");
    if (u.cols != E || u.rows != ff || u.n != ne || d.cols != ff || d.rows != E || d.n != ne)
        return fail(ctx, BIV_HIP_E_INVALID, "expert shapes disagree: gate %dx%dx%d up %dx%dx%d down %dx%dx%d", g.cols,
                    g.rows, g.n, u.cols, u.rows, u.n, d.cols, d.rows, d.n);
    if (r.cols != E || r.rows != ne) return fail(ctx, BIV_HIP_E_INVALID, "router is %dx%d, want %dx%d", r.cols, r.rows, E, ne);
    auto width_ok = [](int K) { return K == 512 || K == 1024 || K == 2048; };
    if (!width_ok(E) || !width_ok(ff))
        return fail(ctx, BIV_HIP_E_INVALID, "n_embd %d / n_ff %d: the matvec kernels take 512, 1024 or 2048", E, ff);
    if (ne > 256) return fail(ctx, BIV_HIP_E_INVALID, "%d experts: at most 256", ne);
    if (k < 1 || k > 16 || k > ne) return fail(ctx, BIV_HIP_E_INVALID, "k = %d not in 1..min(16, n_expert)", k);
    if (n_shared) {
        const DevMat &sg = shared_gate->m, &su = shared_up->m, &sd = shared_down->m, &gi = gate_inp->m;
        if (!expert_type_ok(sg.ty) || !expert_type_ok(su.ty) || !expert_type_ok(sd.ty) || sg.ty != su.ty)
            return fail(ctx, BIV_HIP_E_TYPE, "shared expert types %d/%d/%d", sg.ty, su.ty, sd.ty);
        if (gi.ty != BIV_GGML_F32) return fail(ctx, BIV_HIP_E_TYPE, "gate_inp type %d: only F32", gi.ty);
        if (sg.cols != E || su.cols != E || sd.rows != E || sg.rows != ff || su.rows != ff || sd.cols != ff ||
            gi.cols != E || gi.rows != 1)
            return fail(ctx, BIV_HIP_E_INVALID, "shared expert must be %dx%d (gate/up), %dx%d (down), gate_inp %d", E,
                        ff, ff, E, E);
    }
    auto *m = new biv_hip_moe();
    m->router = router;
    m->gate = gate;
    m->up = up;
    m->down = down;
    m->sg = shared_gate;
    m->su = shared_up;
    m->sd = shared_down;
    m->gi = gate_inp;
    m->k = k;
    m->n_expert = ne;
    m->E = E;
    m->ff = ff;
    ctx->layers.push_back(m);
    *out = m;
    return 0;
}

static int check_fwd(biv_hip_ctx *ctx, const biv_hip_moe *moe, const void *h, int n, const void *out)
{
    if (!ctx) return BIV_HIP_E_INVALID;
    if (!moe) return fail(ctx, BIV_HIP_E_INVALID, "null layer");
    if (n < 0) return fail(ctx, BIV_HIP_E_INVALID, "n = %d", n);
    if (n > 0 && (!h || !out)) return fail(ctx, BIV_HIP_E_INVALID, "null h or out");
    if ((long long)n * moe->k >= (1 << 20)) return fail(ctx, BIV_HIP_E_INVALID, "n * k = %lld pairs: too many", (long long)n * moe->k);
    return 0;
}

int biv_hip_moe_forward_device(biv_hip_ctx *ctx, const biv_hip_moe *moe, const float *h_dev, int n, float *out_dev,
                               unsigned flags)
{
    int rc = check_fwd(ctx, moe, h_dev, n, out_dev);
    if (rc) return rc;
    HIP_TRY(ctx, hipSetDevice(ctx->device), "hipSetDevice");
    return forward(ctx, moe, h_dev, n, out_dev, flags, Dumps{});
}

int biv_hip_moe_forward_device_noalloc(biv_hip_ctx *ctx, const biv_hip_moe *moe, const float *h_dev, int n,
                                       float *out_dev, unsigned flags)
{
    int rc = check_fwd(ctx, moe, h_dev, n, out_dev);
    if (rc) return rc;
    if (n == 0) return 0;
    // stage timing would create events (an allocation)
    if (ctx->timing) return fail(ctx, BIV_HIP_E_INVALID, "the no-allocation entry point runs with timing off");
    if ((rc = noalloc_claim(ctx))) return rc;
    HIP_TRY(ctx, hipSetDevice(ctx->device), "hipSetDevice");
    Scratch s;
    if ((rc = noalloc_scratch(ctx, moe, n, s))) return rc;
    return forward(ctx, moe, h_dev, n, out_dev, flags, Dumps{}, -1, nullptr, 0.0f, &s);
}

int biv_hip_moe_forward_taps(biv_hip_ctx *ctx, const biv_hip_moe *moe, const float *h, int n, float *out,
                             unsigned flags, const biv_hip_taps *taps)
{
    int rc = check_fwd(ctx, moe, h, n, out);
    if (rc) return rc;
    if (n == 0) return 0;
    HIP_TRY(ctx, hipSetDevice(ctx->device), "hipSetDevice");
    if ((rc = scratch_fit(ctx, moe, n))) return rc;
    Scratch &s = ctx->sc;
    const size_t E = moe->E, ff = moe->ff, k = moe->k, P = (size_t)n * k, R = P + n;
    HIP_TRY(ctx, hipMemcpyAsync(s.h_stage, h, sizeof(float) * n * E, hipMemcpyHostToDevice, ctx->stream), "copy h");
    if (flags & BIV_HIP_ADD)
        HIP_TRY(ctx, hipMemcpyAsync(s.o_stage, out, sizeof(float) * n * E, hipMemcpyHostToDevice, ctx->stream),
                "copy x");
    Dumps dm;
    bool permuted_acts = false;
    std::vector<void *> tmp;
    auto dev = [&](size_t bytes) -> int32_t * {
        void *p = nullptr;
        if (hipMalloc(&p, bytes) != hipSuccess) return nullptr;
        tmp.push_back(p);
        return static_cast<int32_t *>(p);
    };
    if (taps && taps->gate_idots) dm.gate = dev(sizeof(int32_t) * R * ff * (E / 32));
    if (taps && taps->up_idots) dm.up = dev(sizeof(int32_t) * R * ff * (E / 32));
    if (taps && taps->down_idots) dm.down = dev(sizeof(int32_t) * R * E * (ff / 32));
    dm.act = taps && (taps->act_q || taps->act_d);
    rc = forward(ctx, moe, s.h_stage, n, s.o_stage, flags, dm);
    auto d2h = [&](void *dst, const void *src, size_t bytes) {
        if (!rc && dst && src) {
            hipError_t e = hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, ctx->stream);
            if (e != hipSuccess) rc = hip_fail(ctx, e, "copy taps");
        }
    };
    d2h(out, s.o_stage, sizeof(float) * n * E);
    if (taps) {
        d2h(taps->ids, s.dp.ids, sizeof(int32_t) * P);
        d2h(taps->weights, s.dp.wts, sizeof(float) * P);
        d2h(taps->logits, s.logits, sizeof(float) * n * moe->n_expert);
        d2h(taps->shared_logit, moe->sg ? s.glogit : nullptr, sizeof(float) * n);
        d2h(taps->pair_token, s.dp.pair_tok, sizeof(int32_t) * P);
        d2h(taps->pair_expert, s.dp.pair_exp, sizeof(int32_t) * P);
        d2h(taps->gate_idots, dm.gate, sizeof(int32_t) * R * ff * (E / 32));
        d2h(taps->up_idots, dm.up, sizeof(int32_t) * R * ff * (E / 32));
        d2h(taps->act_q, s.aq, R * ff);
        d2h(taps->act_d, s.ad, sizeof(float) * R * ff / 32);
        permuted_acts = taps->act_q || taps->act_d;
        d2h(taps->down_idots, dm.down, sizeof(int32_t) * R * E * (ff / 32));
    }
    hipError_t e = hipStreamSynchronize(ctx->stream);
    for (void *p : tmp) (void)hipFree(p);
    if (!rc && e != hipSuccess) rc = hip_fail(ctx, e, "forward");
    if (!rc && permuted_acts) {
        // the intermediate is stored in the chain layout: back to row order
        const int K = (int)ff;
        std::vector<int8_t> qrow(ff);
        std::vector<float> drow(ff / 32);
        for (size_t r = 0; r < R; r++) {
            if (taps->act_q) {
                int8_t *row = taps->act_q + r * ff;
                memcpy(qrow.data(), row, ff);
                for (int b = 0; b < K / 32; b++)
                    for (int l = 0; l < 8; l++) memcpy(row + 32 * b + 4 * l, &qrow[4 * biv::lay::q8_word(b, l)], 4);
            }
            if (taps->act_d) {
                float *row = taps->act_d + r * (ff / 32);
                memcpy(drow.data(), row, sizeof(float) * (ff / 32));
                for (int b = 0; b < K / 32; b++) row[b] = drow[biv::lay::q8_scale(K, b)];
            }
        }
    }
    return rc;
}

int biv_hip_moe_forward(biv_hip_ctx *ctx, const biv_hip_moe *moe, const float *h, int n, float *out, unsigned flags)
{
    return biv_hip_moe_forward_taps(ctx, moe, h, n, out, flags, nullptr);
}

int biv_hip_malloc(biv_hip_ctx *ctx, size_t bytes, void **out)
{
    if (!ctx || !out) return BIV_HIP_E_INVALID;
    HIP_TRY(ctx, hipSetDevice(ctx->device), "hipSetDevice");
    hipError_t e = hipMalloc(out, bytes ? bytes : 1);
    if (e != hipSuccess) return fail(ctx, BIV_HIP_E_NOMEM, "hipMalloc(%zu): %s", bytes, hipGetErrorString(e));
    return 0;
}

int biv_hip_free(biv_hip_ctx *ctx, void *p)
{
    if (!ctx) return BIV_HIP_E_INVALID;
    HIP_TRY(ctx, hipFree(p), "hipFree");
    return 0;
}

int biv_hip_memcpy_h2d(biv_hip_ctx *ctx, void *dst, const void *src, size_t bytes)
{
    if (!ctx) return BIV_HIP_E_INVALID;
    HIP_TRY(ctx, hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, ctx->stream), "h2d");
    HIP_TRY(ctx, hipStreamSynchronize(ctx->stream), "h2d");
    return 0;
}

int biv_hip_memcpy_d2h(biv_hip_ctx *ctx, void *dst, const void *src, size_t bytes)
{
    if (!ctx) return BIV_HIP_E_INVALID;
    HIP_TRY(ctx, hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, ctx->stream), "d2h");
    HIP_TRY(ctx, hipStreamSynchronize(ctx->stream), "d2h");
    return 0;
}

int biv_hip_numerics(const biv_hip_ctx *ctx, char *buf, size_t len)
{
    if (!buf || len == 0) return BIV_HIP_E_INVALID;
    snprintf(buf, len,
             "kind=hip;arch=gfx950;act=q8_32_f32scale;router=f32_avx2_order;route=softmax_topk_lowidx;"
             "experts=int32_block_dot_f32_scale;combine=fma_ascending_expert;deterministic=1");
    return 0;
}

size_t biv_hip_device_bytes(const biv_hip_ctx *ctx) { return ctx ? ctx->bytes : 0; }

int biv_hip_set_timing(biv_hip_ctx *ctx, int enable)
{
    if (!ctx) return BIV_HIP_E_INVALID;
    ctx->timing = enable != 0;
    return 0;
}

int biv_hip_stage_times(biv_hip_ctx *ctx, double *ms, int n_stages, int *n_forwards)
{
    if (!ctx || !ms || n_stages < N_STAGES) return BIV_HIP_E_INVALID;
    HIP_TRY(ctx, hipStreamSynchronize(ctx->stream), "sync");
    for (int i = 0; i < n_stages; i++) ms[i] = 0.0;
    for (auto &v : ctx->ev_fwd) {
        for (int i = 0; i < N_STAGES; i++) {
            float t = 0.0f;
            HIP_TRY(ctx, hipEventElapsedTime(&t, v[i], v[i + 1]), "event time");
            ms[i] += t;
        }
        for (auto e : v) ctx->ev_pool.push_back(e);
    }
    if (n_forwards) *n_forwards = (int)ctx->ev_fwd.size();
    ctx->ev_fwd.clear();
    return 0;
}

int biv_hip_rms_norm(biv_hip_ctx *ctx, float *x_dev, const float *w_dev, int rows, int n, float eps)
{
    if (!ctx) return BIV_HIP_E_INVALID;
    if (rows < 0 || n <= 0 || n % 32 || (rows > 0 && (!x_dev || !w_dev)))
        return fail(ctx, BIV_HIP_E_INVALID, "rms_norm: %d rows of %d (n a positive multiple of 32)", rows, n);
    HIP_TRY(ctx, hipSetDevice(ctx->device), "hipSetDevice");
    HIP_TRY(ctx, biv::launch_rms_norm(x_dev, x_dev, w_dev, rows, n, eps, ctx->stream), "rms_norm");
    return 0;
}

int biv_hip_moe_ffn_step(biv_hip_ctx *ctx, const biv_hip_moe *moe, float *x_dev, const float *norm_dev, float eps,
                         int n)
{
    int rc = check_fwd(ctx, moe, x_dev, n, x_dev);
    if (rc) return rc;
    if (!norm_dev) return fail(ctx, BIV_HIP_E_INVALID, "null norm weights");
    if (n == 0) return 0;
    HIP_TRY(ctx, hipSetDevice(ctx->device), "hipSetDevice");
    if ((rc = scratch_fit(ctx, moe, n))) return rc;
    return forward(ctx, moe, x_dev, n, x_dev, BIV_HIP_ADD, Dumps{}, -1, norm_dev, eps);
}

int biv_hip_time_stage(biv_hip_ctx *ctx, const biv_hip_moe *const *moes, int n_moes, const float *h_dev, int n,
                       float *out_dev, int stage, int reps, double *ms_per_launch)
{
    if (!ctx || !moes || n_moes < 1 || !h_dev || !out_dev || n < 1 || stage < 0 || stage >= N_STAGES || reps < 1 ||
        !ms_per_launch)
        return fail(ctx, BIV_HIP_E_INVALID, "time_stage: bad arguments");
    const biv_hip_moe *m0 = moes[0];
    for (int i = 0; i < n_moes; i++) {
        const biv_hip_moe *m = moes[i];
        if (!m || m->E != m0->E || m->ff != m0->ff || m->n_expert != m0->n_expert || m->k != m0->k ||
            (m->sg == nullptr) != (m0->sg == nullptr) || m->gate->m.ty != m0->gate->m.ty ||
            m->down->m.ty != m0->down->m.ty)
            return fail(ctx, BIV_HIP_E_INVALID, "time_stage: layers differ in shape or types");
    }
    HIP_TRY(ctx, hipSetDevice(ctx->device), "hipSetDevice");
    const bool timing = ctx->timing;
    ctx->timing = false;
    int rc = forward(ctx, m0, h_dev, n, out_dev, 0, Dumps{}); // the routing the stage runs on
    hipEvent_t e0 = nullptr, e1 = nullptr;
    if (!rc && hipEventCreate(&e0) != hipSuccess) rc = fail(ctx, BIV_HIP_E_DEVICE, "event");
    if (!rc && hipEventCreate(&e1) != hipSuccess) rc = fail(ctx, BIV_HIP_E_DEVICE, "event");
    if (!rc && hipEventRecord(e0, ctx->stream) != hipSuccess) rc = fail(ctx, BIV_HIP_E_DEVICE, "event");
    for (int r = 0; r < reps && !rc; r++) rc = forward(ctx, moes[r % n_moes], h_dev, n, out_dev, 0, Dumps{}, stage);
    float ms = 0.0f;
    if (!rc && hipEventRecord(e1, ctx->stream) != hipSuccess) rc = fail(ctx, BIV_HIP_E_DEVICE, "event");
    if (!rc && hipEventSynchronize(e1) != hipSuccess) rc = fail(ctx, BIV_HIP_E_DEVICE, "event sync");
    if (!rc && hipEventElapsedTime(&ms, e0, e1) != hipSuccess) rc = fail(ctx, BIV_HIP_E_DEVICE, "event time");
    if (e0) (void)hipEventDestroy(e0);
    if (e1) (void)hipEventDestroy(e1);
    ctx->timing = timing;
    if (!rc) *ms_per_launch = ms / reps;
    return rc;
}

} // extern "C"

extern "C" {

int biv_hip_dense_create(biv_hip_ctx *ctx, const biv_hip_weight *gate, const biv_hip_weight *up,
                         const biv_hip_weight *down, biv_hip_dense **out)
{
    if (!ctx) return BIV_HIP_E_INVALID;
    if (!out || !gate || !up || !down) return fail(ctx, BIV_HIP_E_INVALID, "null argument");
    *out = nullptr;
    const DevMat &G = gate->m, &U = up->m, &D = down->m;
    const int E = G.cols, ff = G.rows;
    if (U.cols != E || U.rows != ff || D.cols != ff || D.rows != E)
        return fail(ctx, BIV_HIP_E_INVALID, "dense shapes: gate %dx%d, up %dx%d, down %dx%d", G.rows, G.cols, U.rows,
                    U.cols, D.rows, D.cols);
    auto ok = [](int t) { return t == biv::T_Q8_0 || t == biv::T_Q4K || t == biv::T_Q6K || t == biv::T_BF16; };
    if (!ok(G.ty) || !ok(D.ty) || U.ty != G.ty)
        return fail(ctx, BIV_HIP_E_TYPE,
                    "dense types gate %d, up %d, down %d: gate and up of one type, each Q8_0, Q4_K, Q6_K or BF16", G.ty,
                    U.ty, D.ty);
    if (E % 512 || ff % 512) return fail(ctx, BIV_HIP_E_INVALID, "n_embd %d and n_ff %d must be multiples of 512", E, ff);
    auto *d = new biv_hip_dense{gate, up, down, E, ff};
    ctx->denses.push_back(d);
    *out = d;
    return 0;
}

int biv_hip_dense_forward_device(biv_hip_ctx *ctx, const biv_hip_dense *d, const float *h_dev, int n, float *out_dev,
                                 unsigned flags)
{
    if (!ctx) return BIV_HIP_E_INVALID;
    if (!d) return fail(ctx, BIV_HIP_E_INVALID, "null layer");
    if (n < 0) return fail(ctx, BIV_HIP_E_INVALID, "n = %d", n);
    if (n > 0 && (!h_dev || !out_dev)) return fail(ctx, BIV_HIP_E_INVALID, "null h or out");
    HIP_TRY(ctx, hipSetDevice(ctx->device), "hipSetDevice");
    return dense_forward(ctx, d, h_dev, n, out_dev, flags);
}

int biv_hip_dense_forward(biv_hip_ctx *ctx, const biv_hip_dense *d, const float *h, int n, float *out, unsigned flags)
{
    if (!ctx) return BIV_HIP_E_INVALID;
    if (!d) return fail(ctx, BIV_HIP_E_INVALID, "null layer");
    if (n < 0) return fail(ctx, BIV_HIP_E_INVALID, "n = %d", n);
    if (n == 0) return 0;
    if (!h || !out) return fail(ctx, BIV_HIP_E_INVALID, "null h or out");
    HIP_TRY(ctx, hipSetDevice(ctx->device), "hipSetDevice");
    int rc = dense_scratch_fit(ctx, d, n);
    if (rc) return rc;
    DenseScratch &s = ctx->dsc;
    const size_t bytes = sizeof(float) * (size_t)n * d->E;
    HIP_TRY(ctx, hipMemcpyAsync(s.h_stage, h, bytes, hipMemcpyHostToDevice, ctx->stream), "copy h");
    if (flags & BIV_HIP_ADD)
        HIP_TRY(ctx, hipMemcpyAsync(s.o_stage, out, bytes, hipMemcpyHostToDevice, ctx->stream), "copy x");
    rc = dense_forward(ctx, d, s.h_stage, n, s.o_stage, flags);
    if (rc) return rc;
    HIP_TRY(ctx, hipMemcpyAsync(out, s.o_stage, bytes, hipMemcpyDeviceToHost, ctx->stream), "copy out");
    HIP_TRY(ctx, hipStreamSynchronize(ctx->stream), "forward");
    return 0;
}

} // extern "C"
