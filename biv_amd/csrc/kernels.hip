// gfx950 kernels of the qwen35moe MoE block: activation quantiser, router,
// route, dispatch sort, grouped expert matvecs and the fixed-order combine.
//
// Numerics follow biv's CPU path (engine/src/quant.rs, ops.rs, model.rs) to
// the bit where it can be restated: activations are quantised exactly as
// Q8Act::quantize_into does, every dot product (router, gate, up, down) is
// summed in the accumulation order of biv's x86 kernels (see layout.hpp),
// and the combine uses the reference's FMA order.  Nothing uses a
// floating-point atomic, so a forward is bit-identical from run to run.
#include "common.hpp"
#include "expf_ref.h"
#include "layout.hpp"
#include "lds_dma.hpp"

#include <hip/hip_fp16.h>

namespace biv {

namespace {

constexpr int WAVE = 64;

__device__ inline int dot4(int a, int b, int c) { return __builtin_amdgcn_sdot4(a, b, c, false); }

// f32::exp of the reference: glibc's expf, restated bit for bit (expf_ref.h)
__device__ inline float exp_f32(float x) { return biv_expf_ref(x); }

// glibc's expf table (expf_ref.h) in global memory, for kernels that copy it
// into LDS first: exp_lds then costs one LDS read, where exp_f32 costs a
// dependent global (L2) load
__device__ const uint64_t exp_tab_g[32] = BIV_EXPF_TAB_INIT;
__device__ inline float exp_lds(float x, const uint64_t *tab)
{
    double r;
    uint64_t ki;
    const uint32_t i = biv_expf_reduce(x, &r, &ki);
    return biv_expf_finish_sel(x, r, ki, tab[i]);
}

// ops::sigmoid (ops.rs:159-162)
__device__ inline float sigmoid(float x) { return 1.0f / (1.0f + exp_f32(-x)); }

// ops::silu(g) * u (ops.rs:159-167, model.rs:1121-1124)
__device__ inline float silu_mul(float g, float u) { return (g * sigmoid(g)) * u; }

// byte i (0..15) of a 16-byte vector, without indexing a private array
__device__ inline int byte_at(const int4 &v, int i)
{
    const int w = i < 4 ? v.x : i < 8 ? v.y : i < 12 ? v.z : v.w;
    return ((unsigned)w >> (8 * (i & 3))) & 0xFF;
}

// N consecutive 32-bit words from 16-byte aligned memory (8-byte aligned when
// N is 2): 128-bit loads.
template <int N> __device__ inline void ld_words(const void *p, int (&out)[N])
{
    if constexpr (N % 4 == 0) {
        const int4 *q = reinterpret_cast<const int4 *>(p);
#pragma unroll
        for (int i = 0; i < N / 4; i++) {
            int4 v = q[i];
            out[4 * i] = v.x;
            out[4 * i + 1] = v.y;
            out[4 * i + 2] = v.z;
            out[4 * i + 3] = v.w;
        }
    } else {
        static_assert(N == 2, "word count");
        const int2 *q = reinterpret_cast<const int2 *>(p);
        int2 v = q[0];
        out[0] = v.x;
        out[1] = v.y;
    }
}

// ---------------------------------------------------------------------------
// Q8Act::quantize_into (quant.rs:368-394) of one 32-element block v of row
// `row`: amax, d = amax / 127, id = 1/d (0 when d is 0), q =
// round-half-away(v * id), s = d * sum(q); IEEE division and no contraction
// keep it bit-exact.  Written in the chain layout (layout.hpp).
// The row's quant words, block scales and block sums are at qrow, drow, srow
// (srow may be null); generic pointers, so the row may be in LDS.
__device__ inline void quant_block_at(const float (&v)[32], int K, int b, int *qrow, float *drow, float *srow)
{
    // the largest magnitude as a tree: max is exact, so any order gives the
    // sequential loop's value (NaNs skipped by fmaxf alike; 0 if all are)
    float m[16];
#pragma unroll
    for (int j = 0; j < 16; j++) m[j] = fmaxf(fabsf(v[2 * j]), fabsf(v[2 * j + 1]));
#pragma unroll
    for (int w = 8; w >= 1; w >>= 1)
#pragma unroll
        for (int j = 0; j < w; j++) m[j] = fmaxf(m[j], m[j + w]);
    const float amax = fmaxf(0.0f, m[0]);
    const float db = amax / 127.0f;
    const float id = db != 0.0f ? 1.0f / db : 0.0f;
    int sum = 0;
#pragma unroll
    for (int l = 0; l < 8; l++) {
        unsigned w = 0;
#pragma unroll
        for (int c = 0; c < 4; c++) {
            int r = (int)roundf(v[4 * l + c] * id);
            sum += r;
            w |= (unsigned)(r & 0xFF) << (8 * c);
        }
        qrow[lay::q8_word(b, l)] = (int)w;
    }
    drow[lay::q8_scale(K, b)] = db;
    if (srow) srow[lay::q8_scale(K, b)] = db * (float)sum;
}

// The same from a block in LDS, read twice (amax, then the quants) so that
// few registers are live; 16-byte word l of the block at v[l ^ sw].
__device__ inline void quant_block_lds(const float4 *v, int K, int b, int *qrow, float *drow, float *srow = nullptr,
                                       int sw = 0)
{
    float amax = 0.0f;
#pragma unroll
    for (int q = 0; q < 8; q++) {
        const float4 f = v[q ^ sw];
        amax = fmaxf(amax, fabsf(f.x));
        amax = fmaxf(amax, fabsf(f.y));
        amax = fmaxf(amax, fabsf(f.z));
        amax = fmaxf(amax, fabsf(f.w));
    }
    const float db = amax / 127.0f;
    const float id = db != 0.0f ? 1.0f / db : 0.0f;
    int sum = 0;
#pragma unroll
    for (int l = 0; l < 8; l++) {
        const float4 f = v[l ^ sw];
        const int r0 = (int)roundf(f.x * id), r1 = (int)roundf(f.y * id), r2 = (int)roundf(f.z * id),
                  r3 = (int)roundf(f.w * id);
        sum += r0;
        sum += r1;
        sum += r2;
        sum += r3;
        const unsigned w = ((unsigned)r0 & 0xFF) | (((unsigned)r1 & 0xFF) << 8) | (((unsigned)r2 & 0xFF) << 16) |
                           (((unsigned)r3 & 0xFF) << 24);
        qrow[lay::q8_word(b, l)] = (int)w;
    }
    drow[lay::q8_scale(K, b)] = db;
    if (srow) srow[lay::q8_scale(K, b)] = db * (float)sum;
}

__device__ inline void quant_block(const float (&v)[32], int K, size_t row, int b, int8_t *qs, float *d, float *s)
{
    quant_block_at(v, K, b, reinterpret_cast<int *>(qs + row * K), d + row * (K / 32), s + row * (K / 32));
}

// 32 consecutive floats, 16-byte aligned
__device__ inline void load32(const float *p, float (&v)[32])
{
    const float4 *q = reinterpret_cast<const float4 *>(p);
#pragma unroll
    for (int j = 0; j < 8; j++) {
        float4 f = q[j];
        v[4 * j] = f.x;
        v[4 * j + 1] = f.y;
        v[4 * j + 2] = f.z;
        v[4 * j + 3] = f.w;
    }
}

// The x86 kernels' tree over the 16 chains of a (row, token) that a 16-lane
// group of the chain kernels holds, lane by lane acc0 + acc1, the two
// 128-bit halves, movehl, movehdup (partners 8, 4, 2 and 1 lanes on), into
// the group's first lane (the other lanes' results are not used): DPP
// row_shl moves within the 16-lane row, not LDS permutes.
#define BIV_ROW_SHL(x, n) __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x100 + (n), 0xF, 0xF, true))
__device__ inline float row_tree16(float acc)
{
    float t = acc + BIV_ROW_SHL(acc, 8); // acc0 + acc1, lane by lane
    t = t + BIV_ROW_SHL(t, 4);           // the two 128-bit halves
    t = t + BIV_ROW_SHL(t, 2);           // movehl
    t = t + BIV_ROW_SHL(t, 1);           // movehdup
    return t;
}
// The same tree for the 32 chains of dot_f32 on a 32-lane half wave
// (quant.rs:1149-1153): lanes 8 apart (acc0 + acc1, acc2 + acc3), then 16
// ((acc0 + acc1) + (acc2 + acc3)), then 4, 2, 1; into lane 0 of the half
__device__ inline float half_tree32(float v)
{
    v = v + BIV_ROW_SHL(v, 8);
    v = v + __uint_as_float(__builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false)[1]);
    v = v + BIV_ROW_SHL(v, 4);
    v = v + BIV_ROW_SHL(v, 2);
    v = v + BIV_ROW_SHL(v, 1);
    return v;
}
#undef BIV_ROW_SHL

// lane l's x from lane l + 16 (lanes 0-15 and 32-47, the first groups of
// each 32-lane half: v_permlane16_swap, not an LDS permute)
__device__ inline float from_lane_plus16(float x)
{
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return __uint_as_float(r[1]);
}

// ---------------------------------------------------------------------------
// Router logits (and the shared expert's gate logit, row n_expert) in the
// order of biv's AVX2 dot_f32 (quant.rs:1177-1207): lane L of a 32-lane half
// wave runs FMA chain L over elements L, L+32, ... of one row; then the tree
// (acc0+acc1)+(acc2+acc3) and hsum (quant.rs:1149-1153).  Rows are stored in
// the f32 chain layout, so each lane's 4-value steps are one 128-bit load.
//
// A workgroup holds 8 rows in registers and meets TC tokens, staged in LDS;
// tokens go two at a time, two independent chains per lane.
// The RMS scale of ops::rms_norm (ops.rs:136-144) of a row of 32 NS floats
// from the sum of squares of lane L's chain (elements L, L + 32, ...), in
// every lane of the 32-lane half wave: dot_f32's tree, / n, 1 / sqrt(. + eps).
__device__ inline float rms_scale(float acc, int n, float eps)
{
    float v = acc;
    v = v + __shfl_xor(v, 8);  // acc0+acc1 (lanes 0-7), acc2+acc3 (16-23)
    v = v + __shfl_xor(v, 16); // (acc0+acc1)+(acc2+acc3)
    v = v + __shfl_xor(v, 4);  // the two 128-bit halves
    v = v + __shfl_xor(v, 2);  // movehl
    v = v + __shfl_xor(v, 1);  // movehdup
    const float ss = v / (float)n;
    return 1.0f / sqrtf(ss + eps);
}

template <int NS, int TC, int NTH = 256> __global__ __launch_bounds__(NTH) void k_router(RouterArgs a)
{
    constexpr int RPW = NTH / 32; // rows per workgroup (a half wave each)
    constexpr int E = 32 * NS;
    const float *__restrict__ router = a.router;
    const float *__restrict__ h = a.h;
    const int n_expert = a.n_expert, T = a.T;
    // Workgroups past the row groups quantise h for the experts (Q8 rows in
    // the chain layout): one 32-element block per thread and turn.  With no
    // xq (BF16 layers, which read h as f32) there are none, or, with the
    // post_norm, they write hn only.
    const int n_rw = (n_expert + 1 + RPW - 1) / RPW;
    if ((int)blockIdx.x >= n_rw && a.norm_w) {
        // post_norm first: a half wave per token forms its RMS scale (the
        // row in registers), then quantises the normalised row, two blocks
        // per lane, and writes it to hn
        const int L = threadIdx.x & 31, nhw = NTH / 32;
        const int nq = gridDim.x - n_rw;
        for (int t = ((blockIdx.x - n_rw) * gridDim.y + blockIdx.y) * nhw + (threadIdx.x >> 5); t < T;
             t += nq * gridDim.y * nhw) {
            const float *g = h + (size_t)t * E;
            float gv[NS];
#pragma unroll
            for (int k = 0; k < NS; k++) gv[k] = g[L + 32 * k];
            float acc = 0.0f;
#pragma unroll
            for (int k = 0; k < NS; k++) acc = fmaf(gv[k], gv[k], acc);
            const float scale = rms_scale(acc, E, a.eps);
            for (int b = L; b < E / 32; b += 32) {
                float v[32];
                load32(g + 32 * b, v);
                const float4 *w4 = reinterpret_cast<const float4 *>(a.norm_w + 32 * b);
                float4 *o4 = reinterpret_cast<float4 *>(a.hn + (size_t)t * E + 32 * b);
#pragma unroll
                for (int j = 0; j < 8; j++) {
                    const float4 w = w4[j];
                    v[4 * j] = v[4 * j] * (scale * w.x);
                    v[4 * j + 1] = v[4 * j + 1] * (scale * w.y);
                    v[4 * j + 2] = v[4 * j + 2] * (scale * w.z);
                    v[4 * j + 3] = v[4 * j + 3] * (scale * w.w);
                    o4[j] = make_float4(v[4 * j], v[4 * j + 1], v[4 * j + 2], v[4 * j + 3]);
                }
                if (a.xq) quant_block(v, E, t, b, a.xq, a.xd, a.xs);
            }
        }
        return;
    }
    if ((int)blockIdx.x >= n_rw) {
        const int nq = gridDim.x - n_rw, nthreads = nq * gridDim.y * blockDim.x;
        for (int i = ((blockIdx.x - n_rw) * gridDim.y + blockIdx.y) * blockDim.x + threadIdx.x; i < T * (E / 32);
             i += nthreads) {
            float v[32];
            load32(h + 32 * (size_t)i, v);
            quant_block(v, E, i / (E / 32), i % (E / 32), a.xq, a.xd, a.xs);
        }
        return;
    }
    const int L = threadIdx.x & 31;
    const int row = blockIdx.x * (blockDim.x / 32) + (threadIdx.x >> 5);
    const bool valid = row < n_expert || (row == n_expert && a.gate_inp != nullptr);
    // gate_inp as an offset from the router: one pointer, a per-lane offset
    const float *w = router + (row < n_expert ? (ptrdiff_t)row * E : (valid ? a.gate_inp - router : 0));
    // this workgroup's tokens into LDS first (row-major, straight from
    // global memory by DMAs the compiler does not track; pieces past the
    // last token reread it into unused LDS), then the row into registers:
    // the chains start once the tokens are in, the row's later words still
    // arriving
    __shared__ float xs[TC][E];
    const int t0 = blockIdx.y * TC, nt = min(TC, T - t0);
    {
        constexpr int NP = TC * (E / 4) / NTH; // 16-byte pieces per thread
        const float4 *src = reinterpret_cast<const float4 *>(h + (size_t)t0 * E);
        const unsigned dst = lds_addr(&xs[0][0]) + 16 * (threadIdx.x & ~(WAVE - 1));
#pragma unroll
        for (int c = 0; c < NP; c++) {
            if (c * NTH >= nt * (E / 4)) break; // uniform
            const int idx0 = c * NTH + (int)threadIdx.x, idx = idx0 < nt * (E / 4) ? idx0 : nt * (E / 4) - 1;
            lds_dma16_at(src + idx, dst + 16 * c * NTH);
        }
    }
    float wv[NS];
    {
        const float4 *p = reinterpret_cast<const float4 *>(w);
#pragma unroll
        for (int i = 0; i < NS / 4; i++) {
            float4 v = p[i * 32 + L];
            wv[4 * i] = v.x;
            wv[4 * i + 1] = v.y;
            wv[4 * i + 2] = v.z;
            wv[4 * i + 3] = v.w;
        }
    }
    // post_norm: this thread's norm weights
    constexpr int NWPT = E / NTH > 0 ? E / NTH : 1;
    float nw[NWPT];
    if (a.norm_w) {
#pragma unroll
        for (int j = 0; j < NWPT; j++) nw[j] = (int)threadIdx.x + NTH * j < E ? a.norm_w[threadIdx.x + NTH * j] : 0.0f;
    }
    // the tokens are in once at most the row's loads are outstanding (loads
    // complete in order); then every thread's
    __builtin_amdgcn_sched_barrier(0);
    wait_vm<NS / 4>();
    rm_barrier();
    if (a.norm_w) {
        // rms_norm of the staged tokens in place: a half wave per token forms
        // the scale, then every thread scales its elements, v * (scale * w)
        __shared__ float scl[TC];
        const int L = threadIdx.x & 31;
        for (int t = threadIdx.x >> 5; t < nt; t += NTH / 32) {
            float acc = 0.0f;
#pragma unroll
            for (int k = 0; k < NS; k++) acc = fmaf(xs[t][L + 32 * k], xs[t][L + 32 * k], acc);
            const float scale = rms_scale(acc, E, a.eps);
            if (L == 0) scl[t] = scale;
        }
        __syncthreads();
        for (int t = 0; t < nt; t++) {
            const float scale = scl[t];
#pragma unroll
            for (int j = 0; j < NWPT; j++) {
                const int e = threadIdx.x + NTH * j;
                if (e < E) xs[t][e] = xs[t][e] * (scale * nw[j]);
            }
        }
        __syncthreads();
    }
    auto finish = [&](float acc, int t) {
        const float v = half_tree32(acc); // valid in lane 0 of the half wave
        if (valid && L == 0) {
            if (row < n_expert) a.logits[(size_t)t * n_expert + row] = v;
            else a.glogit[t] = v;
        }
    };
    // chain L meets elements L, L + 32, ... (conflict-free 32-bit reads)
    int t = 0;
    for (; t + 1 < nt; t += 2) {
        float acc0 = 0.0f, acc1 = 0.0f;
#pragma unroll
        for (int i = 0; i < NS; i++) {
            acc0 = fmaf(wv[i], xs[t][32 * i + L], acc0);
            acc1 = fmaf(wv[i], xs[t + 1][32 * i + L], acc1);
        }
        finish(acc0, t0 + t);
        finish(acc1, t0 + t + 1);
    }
    if (t < nt) {
        float acc = 0.0f;
#pragma unroll
        for (int i = 0; i < NS; i++) acc = fmaf(wv[i], xs[t][32 * i + L], acc);
        finish(acc, t0 + t);
    }
}

#ifndef BIV_RT_MIN_T
#define BIV_RT_MIN_T 256
#endif
constexpr int RT_MIN_T = BIV_RT_MIN_T; // tokens from which launch_router takes the matrix-core router
// tokens from which it takes 32-row tiles of 32 tokens, of 64 tokens
#ifndef BIV_RM_M_T
#define BIV_RM_M_T 1024
#endif
#ifndef BIV_RM_L_T
#define BIV_RM_L_T 2048
#endif

// The router at prefill sizes on the matrix cores.  v_mfma_f32_*x1f32 (one
// product per output, k = 1) rounds each output exactly as fmaf does, so a
// block of it is one FMA step of one chain of dot_f32 (quant.rs:1177-1207)
// for a whole tile of (row, token) pairs: chain L's accumulator for (r, t)
// takes w[r][32 s + L] * h[t][32 s + L] at step s = 0, 1, ..., in the
// reference's order, and the tree (quant.rs:1149-1153) follows at the end.
//
// Both operands are staged row-major (the router's row-major copy), so one
// 16-byte LDS read gives chains 4 c .. 4 c + 3 at one step: component m feeds
// the m-th MFMA of the step.  Each MFMA's two chain blocks (lanes of cs = 0
// and 1) take chains L and L + 8, which the tree adds first, so that level
// is an add within the lane; a wave's chain group c is one of 0, 1, 4, 5.
// Eight waves: four chain groups times two (halves of m when MI = 2, two
// 32-token sub-tiles when MI = 4).  SH = 32: v_mfma_f32_32x32x1f32, a
// 32-row x 32-token block; SH = 16: v_mfma_f32_16x16x1f32 with blocks
// (chain, 16-token group), a 16-row x 32-token block.
//
// A stage is 4 steps (128 elements) of the tile's rows and tokens, NB stages
// in flight.  The gate logit and the Q8 of h come from k_prep, before.
typedef float f32x32_t __attribute__((ext_vector_type(32)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));
template <int SH> struct RmAcc;
template <> struct RmAcc<32> {
    using T = f32x32_t;
    static __device__ T step(float x, float y, T c) { return __builtin_amdgcn_mfma_f32_32x32x1f32(x, y, c, 0, 0, 0); }
};
template <> struct RmAcc<16> {
    using T = f32x16_t;
    static __device__ T step(float x, float y, T c) { return __builtin_amdgcn_mfma_f32_16x16x1f32(x, y, c, 0, 0, 0); }
};

constexpr int RM_NTH = 512;
template <int SH, int MI> constexpr int rm_tokens() { return 32 * (MI / 2); }
template <int SH, int MI> constexpr int rm_nbuf() { return SH == 32 && MI == 4 ? 3 : 4; }

// stage st of a thread's NLD words: word q * RM_NTH + tid lands at that
// index of the buffer (global_load_lds writes a wave's 64 words in lane
// order); the first NW are router words (offsets from wb), the rest token
// words (from xb)
template <int NLD, int NW>
__device__ inline void rm_issue(const float *wb, const float *xb, const unsigned (&off)[NLD], int st, float4 *base, int w)
{
#pragma unroll
    for (int q = 0; q < NLD; q++) lds_dma16((q < NW ? wb : xb) + off[q] + 128 * st, base + q * RM_NTH + w * WAVE);
}

// slot of a workgroup's tile: the tiles are dealt round-robin over the 8
// XCDs by workgroup id, so give XCD x a run of consecutive tiles (row tiles
// fastest): the row tiles of one token tile then share that XCD's L2
__device__ inline int rm_tile(int b, int n)
{
    const int q = n >> 3, r = n & 7, x = b & 7, i = b >> 3;
    return x * q + min(x, r) + i;
}

template <int SH, int MI> __global__ __launch_bounds__(RM_NTH) void k_router_mfma(RouterArgs a, int n_tr, int n_tt)
{
    constexpr int RT = SH, TT = rm_tokens<SH, MI>(), NB = rm_nbuf<SH, MI>();
    constexpr int WORDS = (RT + TT) * 32; // 16-byte words of one stage
    constexpr int NLD = WORDS / RM_NTH;   // words each thread stages
    constexpr int NW = RT * 32 / RM_NTH;  // of them router words
    constexpr int EP = 32 * (RT + 1);     // floats of one chain plane of the epilogue (padded)
    constexpr int STAGE_W = NB * WORDS, EPI_W = 16 * EP / 4;
    static_assert(NLD * RM_NTH == WORDS && NW * RM_NTH == RT * 32, "whole stages");
    __shared__ float4 lds[STAGE_W > EPI_W ? STAGE_W : EPI_W];
    const int E = a.E, ne = a.n_expert, T = a.T, tid = threadIdx.x;
    const int tile = rm_tile(blockIdx.x, n_tr * n_tt);
    const int tr = tile % n_tr, tt = tile / n_tr;
    const int r0 = tr * RT, t0 = tt * TT;
    const int lane = tid & 63, w = tid >> 6, cg = w & 3, ws = w >> 2;
    const int c = (cg & 1) | ((cg >> 1) << 2); // chains 4 c .. 4 c + 3 and 4 c + 8 ..
    const int sp = MI == 4 ? ws : 0;           // token sub-tile
    const int m0 = MI == 4 ? 0 : 2 * ws;       // first of the MI steps' components
    // this lane's operand rows: A row ar of the tile, B token bt of the sub-tile
    const int cs = SH == 32 ? lane >> 5 : (lane >> 4) & 1;
    const int ar = SH == 32 ? (lane & 31) : (lane & 15);
    const int bt = SH == 32 ? (lane & 31) : (lane & 15) + 16 * (lane >> 5);
    const int wd = c ^ (2 * cs);
    // a stage row (RT router rows, then TT tokens) holds 32 words, word x at
    // x ^ (row & 15), which spreads a column of rows over the banks
    const int arow = ar, brow = RT + 32 * sp + bt;
    unsigned off[NLD];
#pragma unroll
    for (int q = 0; q < NLD; q++) {
        const int g = q * RM_NTH + tid, row = g >> 5, word = (g & 31) ^ (row & 15);
        off[q] = q < NW ? (unsigned)(min(r0 + row, ne - 1) * E + 4 * word)
                        : (unsigned)((size_t)min(t0 + row - RT, T - 1) * E + 4 * word);
    }
    using Acc = typename RmAcc<SH>::T;
    Acc acc[MI];
#pragma unroll
    for (int m = 0; m < MI; m++)
#pragma unroll
        for (int k = 0; k < (int)(sizeof(Acc) / 4); k++) acc[m][k] = 0.0f;
    const int nst = E / 128;
    for (int p = 0; p < NB - 1 && p < nst; p++) rm_issue<NLD, NW>(a.router_rm, a.h, off, p, lds + p * WORDS, w);
    for (int st = 0; st < nst; st++) {
        // this stage's words; the later stages' loads stay in flight
        const int ahead = min(nst - 1 - st, NB - 2);
        if (NB > 3 && ahead >= 2) wait_vm<2 * NLD>();
        else if (ahead >= 1) wait_vm<NLD>();
        else wait_vm<0>();
        rm_barrier();
        if (st + NB - 1 < nst) rm_issue<NLD, NW>(a.router_rm, a.h, off, st + NB - 1, lds + ((st + NB - 1) % NB) * WORDS, w);
        const float4 *base = lds + (st % NB) * WORDS;
#pragma unroll
        for (int k = 0; k < 4; k++) {
            const int x = 8 * k + wd;
            if constexpr (MI == 4) {
                const float4 A = base[arow * 32 + (x ^ (arow & 15))];
                const float4 B = base[brow * 32 + (x ^ (brow & 15))];
                acc[0] = RmAcc<SH>::step(A.x, B.x, acc[0]);
                acc[1] = RmAcc<SH>::step(A.y, B.y, acc[1]);
                acc[2] = RmAcc<SH>::step(A.z, B.z, acc[2]);
                acc[3] = RmAcc<SH>::step(A.w, B.w, acc[3]);
            } else {
                const float2 A = reinterpret_cast<const float2 *>(base + arow * 32 + (x ^ (arow & 15)))[ws];
                const float2 B = reinterpret_cast<const float2 *>(base + brow * 32 + (x ^ (brow & 15)))[ws];
                acc[0] = RmAcc<SH>::step(A.x, B.x, acc[0]);
                acc[1] = RmAcc<SH>::step(A.y, B.y, acc[1]);
            }
        }
    }
    // epilogue, one 32-token sub-tile at a time: the chain-L-plus-L+8 sums
    // (chains L in 0..7, 16..23) to LDS planes [16][token][row], then a
    // thread per (row, token) finishes the tree: + L ^ 16, ^ 4, ^ 2, ^ 1
    float *pl = reinterpret_cast<float *>(lds);
    constexpr int NSUB = MI == 4 ? 2 : 1;
#pragma unroll
    for (int sub = 0; sub < NSUB; sub++) {
        __syncthreads(); // the stages (or the previous sub-tile's planes) are read
        if (sp == sub) {
#pragma unroll
            for (int m = 0; m < MI; m++) {
                const int L16 = (c & 1) * 4 + m0 + m + 8 * (c >> 2);
                float *plane = pl + L16 * EP;
                if constexpr (SH == 32) {
#pragma unroll
                    for (int k = 0; k < 16; k++) {
                        const int i = 8 * (k >> 2) + 4 * (lane >> 5) + (k & 3), j = lane & 31;
                        plane[j * (RT + 1) + i] = acc[m][k] + acc[m][k + 16];
                    }
                } else {
#pragma unroll
                    for (int g = 0; g < 2; g++)
#pragma unroll
                        for (int r = 0; r < 4; r++) {
                            const int i = 4 * (lane >> 4) + r, j = (lane & 15) + 16 * g;
                            plane[j * (RT + 1) + i] = acc[m][8 * g + r] + acc[m][8 * g + 4 + r];
                        }
                }
            }
        }
        __syncthreads();
        for (int o = tid; o < 32 * RT; o += RM_NTH) {
            const int row = o % RT, tok = o / RT;
            float p[16];
#pragma unroll
            for (int l = 0; l < 16; l++) p[l] = pl[l * EP + tok * (RT + 1) + row];
            float s2[8];
#pragma unroll
            for (int l = 0; l < 8; l++) s2[l] = p[l] + p[l + 8];
            const float s30 = s2[0] + s2[4], s31 = s2[1] + s2[5], s32 = s2[2] + s2[6], s33 = s2[3] + s2[7];
            const float v = (s30 + s32) + (s31 + s33);
            const int gr = r0 + row, gt = t0 + 32 * sub + tok;
            if (gr < ne && gt < T) a.logits[(size_t)gt * ne + gr] = v;
        }
    }
}

// ---------------------------------------------------------------------------
// ops::rms_norm (ops.rs:136-144) of each row of n: ss = dot_f32(g, g) / n in
// the 32-chain order above, scale = 1 / sqrt(ss + eps), v *= scale * w.  A
// 32-lane half wave per row; n a multiple of 32.
// y may be x (in place).
template <int NPL>
__global__ __launch_bounds__(256) void k_rms_norm(const float *x, float *y, const float *__restrict__ w, int rows, int n,
                                                  float eps)
{
    // NPL > 0: n = 32 NPL, the row held in registers (all loads issued before
    // the chain); NPL = 0: any n (a multiple of 32), read twice
    const int L = threadIdx.x & 31;
    const int row = blockIdx.x * (blockDim.x / 32) + (threadIdx.x >> 5);
    const float *g = x + (size_t)row * n;
    float *o = y + (size_t)row * n;
    float acc = 0.0f;
    float gv[NPL > 0 ? NPL : 1];
    // NPL > 0: the norm weights staged in LDS once per workgroup, read
    // after the chain (a short LDS latency rather than an L2 one)
    __shared__ float wl[NPL > 0 ? 32 * NPL : 1];
    if constexpr (NPL > 0) {
        if (row < rows) {
#pragma unroll
            for (int k = 0; k < NPL; k++) gv[k] = g[L + 32 * k];
        }
        for (int i = threadIdx.x; i < 32 * NPL; i += blockDim.x) wl[i] = w[i];
        __syncthreads();
    }
    if (row >= rows) return; // uniform over the half wave; no shuffles cross halves
    if constexpr (NPL > 0) {
#pragma unroll
        for (int k = 0; k < NPL; k++) acc = fmaf(gv[k], gv[k], acc);
    } else {
        for (int i = L; i < n; i += 32) acc = fmaf(g[i], g[i], acc);
    }
    float v = acc;
    v = v + __shfl_xor(v, 8);  // acc0+acc1 (lanes 0-7), acc2+acc3 (16-23)
    v = v + __shfl_xor(v, 16); // (acc0+acc1)+(acc2+acc3)
    v = v + __shfl_xor(v, 4);  // the two 128-bit halves
    v = v + __shfl_xor(v, 2);  // movehl
    v = v + __shfl_xor(v, 1);  // movehdup
    const float ss = v / (float)n;
    const float scale = 1.0f / sqrtf(ss + eps);
    if constexpr (NPL > 0) {
#pragma unroll
        for (int k = 0; k < NPL; k++) o[L + 32 * k] = gv[k] * (scale * wl[L + 32 * k]);
    } else {
        for (int i = L; i < n; i += 32) o[i] = g[i] * (scale * w[i]);
    }
}

// ---------------------------------------------------------------------------
// route (model.rs:256-268): softmax over the token's logits (ops.rs:192-201),
// the k highest probabilities with the lower expert first among equals, and
// weights p / max(sum of the k in rank order, 1/16384).  One wavefront per
// token, up to 8 logits per lane.
constexpr int MAX_EXPERTS_PER_LANE = 4; // 256 experts over a wavefront

// f32 <-> unsigned with the same order (for finite values and infinities)
__device__ inline unsigned f32_to_ordered(float x)
{
    const unsigned b = __float_as_uint(x);
    return b & 0x80000000u ? ~b : b | 0x80000000u;
}
__device__ inline float ordered_to_f32(unsigned u) { return __uint_as_float(u & 0x80000000u ? u & 0x7FFFFFFFu : ~u); }

// Max over the wavefront of an unsigned value, in every lane: DPP within
// rows of 16 lanes, then the four row results through scalar registers.
// Inclusive prefix sum of v over the wavefront's 64 lanes by DPP: shifts
// of 1, 2, 4, 8 within each row of 16, then row 0's and row 2's totals into
// rows 1 and 3 (row_bcast:15) and rows 0-1's total into rows 2-3
// (row_bcast:31); lanes a shift leaves without a source add 0
__device__ inline int wave_incl_scan(int v)
{
    v += __builtin_amdgcn_update_dpp(0, v, 0x111, 0xF, 0xF, false); // row_shr:1
    v += __builtin_amdgcn_update_dpp(0, v, 0x112, 0xF, 0xF, false); // row_shr:2
    v += __builtin_amdgcn_update_dpp(0, v, 0x114, 0xF, 0xF, false); // row_shr:4
    v += __builtin_amdgcn_update_dpp(0, v, 0x118, 0xF, 0xF, false); // row_shr:8
    v += __builtin_amdgcn_update_dpp(0, v, 0x142, 0xA, 0xF, false); // row_bcast:15 into rows 1, 3
    v += __builtin_amdgcn_update_dpp(0, v, 0x143, 0xC, 0xF, false); // row_bcast:31 into rows 2, 3
    return v;
}

__device__ inline unsigned wave_max_u32(unsigned v)
{
    v = max(v, (unsigned)__builtin_amdgcn_mov_dpp((int)v, 0xB1, 0xF, 0xF, false));  // quad_perm [1,0,3,2]
    v = max(v, (unsigned)__builtin_amdgcn_mov_dpp((int)v, 0x4E, 0xF, 0xF, false));  // quad_perm [2,3,0,1]
    v = max(v, (unsigned)__builtin_amdgcn_mov_dpp((int)v, 0x124, 0xF, 0xF, false)); // row_ror:4
    v = max(v, (unsigned)__builtin_amdgcn_mov_dpp((int)v, 0x128, 0xF, 0xF, false)); // row_ror:8
    const unsigned r0 = __builtin_amdgcn_readlane(v, 0), r1 = __builtin_amdgcn_readlane(v, 16);
    const unsigned r2 = __builtin_amdgcn_readlane(v, 32), r3 = __builtin_amdgcn_readlane(v, 48);
    return max(max(r0, r1), max(r2, r3));
}

// Top-k selection keys (k <= TOPK_FAST): the TOPK_FAST largest of the
// wavefront's RPER keys per lane, as a list sorted in descending order, the
// same in every lane.  Equal keys stay separate entries.
constexpr int TOPK_FAST = 8;

__device__ inline void cas_desc(unsigned &a, unsigned &b)
{
    const unsigned hi = max(a, b), lo = min(a, b);
    a = hi;
    b = lo;
}

// The top TOPK_FAST of two descending lists, descending: the top half of a
// bitonic merge (a against b reversed), then the half-cleaners that sort it.
__device__ inline void merge_top(const unsigned (&a)[TOPK_FAST], const unsigned (&b)[TOPK_FAST], unsigned (&out)[TOPK_FAST])
{
    unsigned m[TOPK_FAST];
#pragma unroll
    for (int i = 0; i < TOPK_FAST; i++) m[i] = max(a[i], b[TOPK_FAST - 1 - i]);
#pragma unroll
    for (int d = TOPK_FAST / 2; d >= 1; d >>= 1)
#pragma unroll
        for (int i = 0; i < TOPK_FAST; i++)
            if ((i & d) == 0) cas_desc(m[i], m[i + d]);
#pragma unroll
    for (int i = 0; i < TOPK_FAST; i++) out[i] = m[i];
}

// N keys per lane (N = 2 or 4)
template <int N> __device__ inline void topk_lists(const unsigned (&key)[N], unsigned (&lst)[TOPK_FAST])
{
    static_assert((N == 2 || N == 4) && TOPK_FAST == 8, "list shapes");
#pragma unroll
    for (int i = 0; i < TOPK_FAST; i++) lst[i] = i < N ? key[i] : 0u;
    if constexpr (N == 4) {
        cas_desc(lst[0], lst[1]);
        cas_desc(lst[2], lst[3]);
        cas_desc(lst[0], lst[2]);
        cas_desc(lst[1], lst[3]);
        cas_desc(lst[1], lst[2]);
    } else {
        cas_desc(lst[0], lst[1]);
    }
    // six levels; each lane meets a partner holding a list of other keys:
    // within a row of 16 lanes by DPP (quad_perm [1,0,3,2], [2,3,0,1], then
    // row_ror 4 and 8: after the second level a lane group of four is
    // uniform, and rotating by one group, then by two, meets disjoint
    // groups); then rows 16 lanes apart and halves 32 apart, swapped between
    // two copies of each entry (v_permlane16_swap / v_permlane32_swap): each
    // lane then holds both lists of its pair of rows (halves), one in each
    // copy, and merges them (the merge is symmetric)
#pragma unroll
    for (int lvl = 0; lvl < 6; lvl++) {
        unsigned A[TOPK_FAST], B[TOPK_FAST];
#pragma unroll
        for (int i = 0; i < TOPK_FAST; i++) {
            if (lvl < 4) {
                A[i] = lst[i];
                const int v = (int)lst[i];
                B[i] = (unsigned)(lvl == 0   ? __builtin_amdgcn_mov_dpp(v, 0xB1, 0xF, 0xF, false)
                                  : lvl == 1 ? __builtin_amdgcn_mov_dpp(v, 0x4E, 0xF, 0xF, false)
                                  : lvl == 2 ? __builtin_amdgcn_mov_dpp(v, 0x124, 0xF, 0xF, false)
                                             : __builtin_amdgcn_mov_dpp(v, 0x128, 0xF, 0xF, false));
            } else {
                const auto r = lvl == 4 ? __builtin_amdgcn_permlane16_swap(lst[i], lst[i], false, false)
                                        : __builtin_amdgcn_permlane32_swap(lst[i], lst[i], false, false);
                A[i] = r[0];
                B[i] = r[1];
            }
        }
        merge_top(A, B, lst);
    }
}

// route (model.rs:256-268) of token t by one wavefront: softmax over the
// logits (ops.rs:192-201), the k highest probabilities with the lower expert
// first among equals, weights p / max(sum of the k in rank order, 1/16384).
// `es` is this wave's LDS scratch of n_expert floats.  Ids and weights go to
// ids/wts and, when given, to the LDS copies lds_ids/lds_wts.
constexpr int RPER = MAX_EXPERTS_PER_LANE;

// LDS writes of this wavefront visible to all its lanes
__device__ inline void wave_lds_sync()
{
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// The prefill pre-pass of the matrix-core router, a wave per token:
//   with norm_w, ops::rms_norm (ops.rs:136-144): ss in dot_f32's 32-chain
//     order (chain L in lane L, as k_rms_norm), scale, v = x * (scale * w),
//     written to hn;
//   the shared expert's gate logit gate_inp . h in dot_f32's order
//     (quant.rs:1177-1207), chain L in lane L, then the tree;
//   with xq, the Q8 for the experts of the (normalised) row: it goes
//     through LDS (32-element blocks at a 36-float pitch) so that lane b
//     quantises block b (BF16 layers, which never read it, pass none);
//   with xh, the bf16 hi / lo halves of the row for BF16 experts (from the
//     LDS copy, as k_split_bf16 forms them).
// Lanes 32-63 repeat the chains of lanes 0-31 (the shuffle tree stays within
// each half); each half writes half of the row (to hn and LDS).  The norm
// weights and the gate row, the chains' operands, are staged in LDS once per
// workgroup.
constexpr int PREP_TOK = 4, PREP_PITCH = 36; // tokens (waves) per workgroup; LDS floats per block
template <int NS> __global__ __launch_bounds__(64 * PREP_TOK) void k_prep(RouterArgs a)
{
    constexpr int E = 32 * NS;
    __shared__ __align__(16) float wn[E];
    __shared__ __align__(16) float wg[E];
    __shared__ __align__(16) float rows[PREP_TOK][NS * PREP_PITCH];
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, L = lane & 31, hi = lane >> 5;
    const int t = blockIdx.x * PREP_TOK + w;
    // the weights go straight to LDS (DMA), the token's row to registers;
    // then all of it is waited for
    {
        float4 *wn4 = reinterpret_cast<float4 *>(wn), *wg4 = reinterpret_cast<float4 *>(wg);
#pragma unroll
        for (int q = 0; q * 64 * PREP_TOK < E / 4; q++) {
            const int i0 = q * 64 * PREP_TOK + 64 * w; // this wave's 64 words
            if (i0 < E / 4) {
                if (a.norm_w) lds_dma16(a.norm_w + 4 * (i0 + lane), wn4 + i0);
                if (a.gate_rm) lds_dma16(a.gate_rm + 4 * (i0 + lane), wg4 + i0);
            }
        }
    }
    const float *g = a.h + (size_t)min(t, a.T - 1) * E;
    float v[NS];
#pragma unroll
    for (int k = 0; k < NS; k++) v[k] = g[L + 32 * k];
    wait_vm<0>();
    __syncthreads();
    if (t >= a.T) return; // uniform over the wave, which syncs only itself from here
    if (a.norm_w) {
        float acc = 0.0f;
#pragma unroll
        for (int k = 0; k < NS; k++) acc = fmaf(v[k], v[k], acc);
        const float scale = rms_scale(acc, E, a.eps);
        float *o = a.hn + (size_t)t * E;
#pragma unroll
        for (int k = 0; k < NS; k++) {
            v[k] = v[k] * (scale * wn[L + 32 * k]);
            if ((k < NS / 2) == (hi == 0)) o[L + 32 * k] = v[k];
        }
    }
    if (a.gate_rm) {
        float acc = 0.0f;
#pragma unroll
        for (int k = 0; k < NS; k++) acc = fmaf(wg[L + 32 * k], v[k], acc);
        acc = half_tree32(acc); // valid in lane 0
        if (lane == 0) a.glogit[t] = acc;
    }
    float *r = &rows[w][0];
#pragma unroll
    for (int k = 0; k < NS; k++)
        if ((k < NS / 2) == (hi == 0)) r[k * PREP_PITCH + L] = v[k];
    wave_lds_sync();
    if (a.xq && lane < NS)
        quant_block_lds(reinterpret_cast<const float4 *>(r + lane * PREP_PITCH), E, lane,
                        reinterpret_cast<int *>(a.xq + (size_t)t * E), a.xd + (size_t)t * (E / 32),
                        a.xs + (size_t)t * (E / 32));
    if (a.xh) {
        // the bf16 halves for the matrix-core gate/up: 16-byte chunk 16 g + c
        // of the row holds elements 128 g + 16 m + c, m = 0..7
        for (int ch = lane; ch < E / 8; ch += 64) {
            const int g = ch >> 4, c = ch & 15;
            uint32_t hb[8], lb[8];
#pragma unroll
            for (int m = 0; m < 8; m++) {
                const int e = 128 * g + 16 * m + c;
                const float x = r[(e >> 5) * PREP_PITCH + (e & 31)];
                bf16_split(x, &hb[m], &lb[m]);
            }
            a.xh[(size_t)t * (E / 8) + ch] = make_uint4(hb[0] | hb[1] << 16, hb[2] | hb[3] << 16, hb[4] | hb[5] << 16,
                                                        hb[6] | hb[7] << 16);
            a.xl[(size_t)t * (E / 8) + ch] = make_uint4(lb[0] | lb[1] << 16, lb[2] | lb[3] << 16, lb[4] | lb[5] << 16,
                                                        lb[6] | lb[7] << 16);
        }
    }
}


// token t's logits, RPER per lane (-inf past n_expert)
__device__ inline void load_logits(const float *__restrict__ logits, int n_expert, int t, float (&v)[RPER])
{
    const int lane = threadIdx.x & 63;
#pragma unroll
    for (int j = 0; j < RPER; j++) {
        const int i = lane + WAVE * j;
        v[j] = i < n_expert ? logits[(size_t)t * n_expert + i] : -INFINITY;
    }
}

__device__ void route_select(unsigned (&key)[RPER], const unsigned (&lst)[TOPK_FAST], int n_expert, int k, int t,
                             float *es, int *__restrict__ ids, float *__restrict__ wts, int *lds_ids, float *lds_wts);

// v: the token's logits (load_logits); tab: the exp table in LDS; ids / wts
// (global, may be null) and lds_ids / lds_wts (may be null) take the routes
__device__ void route_token(float (&v)[RPER], const uint64_t *tab, int n_expert, int k, int t, float *es,
                            int *__restrict__ ids, float *__restrict__ wts, int *lds_ids, float *lds_wts)
{
    const int lane = threadIdx.x & 63;
    float mx = -INFINITY;
#pragma unroll
    for (int j = 0; j < RPER; j++) mx = fmaxf(mx, v[j]);
    if (mx != mx) mx = -INFINITY; // f32::max skips NaN
    mx = ordered_to_f32(wave_max_u32(f32_to_ordered(mx)));
#pragma unroll
    for (int j = 0; j < RPER; j++) {
        const int i = lane + WAVE * j;
        const float ev = exp_lds(v[j] - mx, tab); // every lane: no branch around the table read
        v[j] = i < n_expert ? ev : 0.0f;
        es[i] = v[j]; // zeros past n_expert: adding +0 leaves the positive sum's bits alone
    }
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
    // the sum in index order, as the reference's loop adds it: one chain, the
    // same in every lane; the reads well ahead of the adds
    float sum = 0.0f;
    const float4 *e4 = reinterpret_cast<const float4 *>(es);
    constexpr int NQ = MAX_EXPERTS_PER_LANE * WAVE / 4;
    // 12 reads (48 values) kept in flight ahead of the adds: the chain,
    // not the LDS latency, sets the pace
    constexpr int LA = 12;
    float4 q[NQ];
#pragma unroll
    for (int i = 0; i < LA; i++) q[i] = e4[i];
#pragma unroll
    for (int i = 0; i < NQ; i++) {
        if (i + LA < NQ) q[i + LA] = e4[i + LA];
        sum = sum + q[i].x;
        sum = sum + q[i].y;
        sum = sum + q[i].z;
        sum = sum + q[i].w;
    }
    const float inv = 1.0f / sum;
    // probabilities as keys: bits + 1 orders like the float (p >= 0), 0 once taken
    unsigned key[RPER];
#pragma unroll
    for (int j = 0; j < RPER; j++) key[j] = lane + WAVE * j < n_expert ? __float_as_uint(v[j] * inv) + 1u : 0u;
    // The k largest keys as a sorted list in every lane: each lane sorts its
    // own, then six butterfly levels merge a lane's list with its partner's,
    // keeping the top TOPK_FAST (bitonic merge).
    unsigned lst[TOPK_FAST];
    if (k <= TOPK_FAST) topk_lists<RPER>(key, lst);
    route_select(key, lst, n_expert, k, t, es, ids, wts, lds_ids, lds_wts);
}

// The set of one token's k routed experts without the softmax's sum, when
// the exps alone decide it: with e = exp(x - max) (e <= 1, sum <= 256, so
// inv = 1 / sum lies in [1/256, 1]), the probabilities p = e * inv round
// monotonically, and two exps at least 16 ulps apart, both at least 2^-100
// (the smaller may be +0 instead), give distinct p.  So when the k-th
// largest exp stands that far above the next one, the k largest p are the
// k largest exps, whatever the sum.  Returns false (decide by route_token)
// for NaN or infinite logits, a narrower gap, or equal exps at the k-th
// place; on success m[j] bit l is set for expert l + 64 j of the set.
// v: the token's logits (load_logits), unchanged; tab: this wave's exp
// table in LDS; k <= 8.
__device__ bool route_set_masks(const float (&v)[RPER], const uint64_t *tab, int n_expert, int k,
                                unsigned long long (&m)[RPER])
{
    const int lane = threadIdx.x & 63;
    float mx = -INFINITY;
#pragma unroll
    for (int j = 0; j < RPER; j++) mx = fmaxf(mx, v[j]);
    if (mx != mx) mx = -INFINITY;
    mx = ordered_to_f32(wave_max_u32(f32_to_ordered(mx)));
    unsigned ek[RPER], lst[TOPK_FAST];
#pragma unroll
    for (int j = 0; j < RPER; j++) {
        const float ev = exp_lds(v[j] - mx, tab);
        ek[j] = lane + WAVE * j < n_expert ? __float_as_uint(ev) + 1u : 0u;
    }
    topk_lists<RPER>(ek, lst);
    unsigned kth = lst[0];
#pragma unroll
    for (int r = 1; r < TOPK_FAST; r++) kth = r == k - 1 ? lst[r] : kth;
    unsigned below = 0u;
    int cnt = 0;
#pragma unroll
    for (int j = 0; j < RPER; j++) {
        m[j] = __ballot(ek[j] >= kth);
        cnt += __popcll(m[j]);
        below = max(below, ek[j] < kth ? ek[j] : 0u);
    }
    const unsigned next = wave_max_u32(below);
    constexpr unsigned ONE = 0x3F800000u + 1u, TINY = 0x0D800000u + 1u; // keys of 1.0 and 2^-100
    return lst[0] <= ONE && cnt == k && kth >= TINY && (next <= 1u || (next >= TINY && kth - next >= 16u));
}

// The selection from the probabilities: key[j] = bits(p) + 1 of expert
// lane + 64 j (0 past n_expert) and, for k <= TOPK_FAST, lst, the top
// TOPK_FAST keys in descending order (equal keys as separate entries).  The
// expert of rank r: the keys equal to the r-th, in index order, skipping
// those equal keys already ranked (lower index first); weights p / max(sum
// of the k in rank order, 1/16384).  es: this wave's LDS scratch.
__device__ void route_select(unsigned (&key)[RPER], const unsigned (&lst)[TOPK_FAST], int n_expert, int k, int t,
                             float *es, int *__restrict__ ids, float *__restrict__ wts, int *lds_ids, float *lds_wts)
{
    const int lane = threadIdx.x & 63;
    float sel_p = 0.0f, s = 0.0f;
    int sel_i = 0;
    if (k <= TOPK_FAST) {
        // Every lane holds the same list.  Without equal keys among the k
        // largest (nor between the k-th and the next), exactly k keys are at
        // least the k-th, and each one's rank is the number of listed keys
        // above it: those lanes write their experts to LDS by rank (es is
        // free again: the sum has read it).  Equal keys take the ballot
        // walk below, which breaks ties by the lower index.
        unsigned kth = lst[0];
#pragma unroll
        for (int r = 1; r < TOPK_FAST; r++) kth = r == k - 1 ? lst[r] : kth;
        int ncand = 0;
#pragma unroll
        for (int j = 0; j < RPER; j++) ncand += __popcll(__ballot(key[j] >= kth));
        bool ties = ncand != k;
#pragma unroll
        for (int r = 0; r + 1 < TOPK_FAST; r++) ties |= r + 1 < k && lst[r] == lst[r + 1];
        if (!ties) {
            int *sel = reinterpret_cast<int *>(es);
#pragma unroll
            for (int j = 0; j < RPER; j++) {
                if (key[j] >= kth) {
                    int rank = 0;
#pragma unroll
                    for (int r = 0; r < TOPK_FAST; r++) rank += r < k && lst[r] > key[j];
                    sel[rank] = lane + WAVE * j;
                }
            }
            wave_lds_sync();
            // weights' numerators and their sum in rank order (the
            // reference's iterator sum)
#pragma unroll
            for (int r = 0; r < TOPK_FAST; r++) {
                if (r >= k) break;
                const float bp = __uint_as_float(lst[r] - 1u);
                if (r == lane) sel_p = bp;
                s += bp;
            }
            if (lane < k) sel_i = sel[lane];
        }
        // every lane holds the same list: scalar values from here on
        unsigned prev = 0u;
        int before = 0; // earlier ranks holding the current key
#pragma unroll
        for (int r = 0; r < TOPK_FAST; r++) {
            if (!ties) break; // uniform
            if (r >= k) break;
            const unsigned kr = (unsigned)__builtin_amdgcn_readfirstlane((int)lst[r]);
            before = r > 0 && prev == kr ? before + 1 : 0;
            prev = kr;
            // the before-th lowest index holding kr, rows j in index order
            unsigned long long m[RPER];
#pragma unroll
            for (int j = 0; j < RPER; j++) m[j] = __ballot(key[j] == kr);
            int bi = 0, need = before;
            int row = 0;
            unsigned long long mm = m[0];
            if (need >= __popcll(mm)) {
                need -= __popcll(mm);
                row = 1;
                mm = m[1];
                if (need >= __popcll(mm)) {
                    need -= __popcll(mm);
                    row = 2;
                    mm = m[2];
                    if (need >= __popcll(mm)) {
                        need -= __popcll(mm);
                        row = 3;
                        mm = m[3];
                    }
                }
            }
            for (int q = 0; q < need; q++) mm &= mm - 1ull;
            bi = WAVE * row + __ffsll((long long)mm) - 1;
            const float bp = __uint_as_float(kr - 1u); // kr >= 1: k <= n_expert valid keys
            if (r == lane) {
                sel_p = bp;
                sel_i = bi;
            }
            s += bp; // the sum in rank order, as the reference's iterator sum
        }
    } else {
        for (int r = 0; r < k; r++) {
            unsigned best = 0;
#pragma unroll
            for (int j = 0; j < RPER; j++) best = max(best, key[j]);
            best = wave_max_u32(best);
            // the lowest index holding it: first row j, lowest lane
            int bi = -1;
#pragma unroll
            for (int j = 0; j < RPER; j++) {
                const unsigned long long m = __ballot(key[j] == best && best != 0);
                if (bi < 0 && m) bi = WAVE * j + __ffsll((long long)m) - 1;
            }
            float bp;
            if (bi < 0) {
                // NaN probabilities (non-finite h) give no candidate: the lowest
                // expert not yet chosen keeps the ids in range
                bi = 0;
#pragma unroll
                for (int j = RPER - 1; j >= 0; j--) {
                    const unsigned long long m = __ballot(lane + WAVE * j < n_expert && key[j] != 0);
                    if (m) bi = WAVE * j + __ffsll((long long)m) - 1;
                }
                bp = 0.0f;
            } else {
                bp = __uint_as_float(best - 1u);
            }
#pragma unroll
            for (int j = 0; j < RPER; j++)
                if (lane + WAVE * j == bi) key[j] = 0;
            if (r == lane) {
                sel_p = bp;
                sel_i = bi;
            }
            s += bp; // the sum in rank order, as the reference's iterator sum
        }
    }
    s = fmaxf(s, 1.0f / 16384.0f);
    if (lane < k) {
        const float w = sel_p / s;
        if (ids) {
            ids[(size_t)t * k + lane] = sel_i;
            wts[(size_t)t * k + lane] = w;
        }
        if (lds_ids) {
            lds_ids[t * k + lane] = sel_i;
            lds_wts[t * k + lane] = w;
        }
    }
}

// ---------------------------------------------------------------------------
// Dispatch: a counting sort of the T*k pairs by expert, tokens ascending
// within an expert (the `routed` lists of model.rs:866-873; Metal's moe_sort,
// kernels.metal:1675-1739).  Counts are integer atomics in LDS, whose result
// does not depend on their order; a pair's place among its expert's pairs is
// the number of earlier tokens with that expert, read from a token bitmap, so
// the order is deterministic.  Run by one workgroup of NT threads.
constexpr int MAX_EXPERTS = 256;
constexpr int RS_THREADS = 1024;


// The same dispatch as sort_pairs for P <= 4 * WAVE pairs, by one wavefront
// and without workgroup barriers.  A pair's place among its expert's pairs is
// the number of earlier tokens with that expert (a token names an expert at
// most once), read from a token bitmap per expert; so T <= 64.  cnt is an
// LDS array of 2 * MAX_EXPERTS ints (the bitmap reuses it), first and
// sfirst of MAX_EXPERTS.
__device__ void sort_pairs_wave(const int *ids, const float *wts, int n_expert, int k, int T, int chunk,
                                const Dispatch &dp, int *cnt, int *first, int *sfirst)
{
    const int lane = threadIdx.x & (WAVE - 1);
    const int P = T * k;
    for (int e = lane; e < MAX_EXPERTS; e += WAVE) cnt[e] = 0;
    wave_lds_sync();
    for (int i = lane; i < P; i += WAVE) atomicAdd(&cnt[ids[i]], 1);
    wave_lds_sync();
    // lane owns experts 4 lane .. 4 lane + 3: their pairs and slots, then a
    // wave scan of the lane totals
    constexpr int EPL = MAX_EXPERTS / WAVE;
    int c[EPL], ns[EPL], tot = 0, stot = 0;
#pragma unroll
    for (int j = 0; j < EPL; j++) {
        const int e = EPL * lane + j;
        c[j] = e < n_expert ? cnt[e] : 0;
        ns[j] = (c[j] + chunk - 1) / chunk;
        tot += c[j];
        stot += ns[j];
    }
    const int x = wave_incl_scan(tot), y = wave_incl_scan(stot);
    const int n_used = __builtin_amdgcn_readlane(y, WAVE - 1);
    int pos = x - tot, spos = y - stot;
#pragma unroll
    for (int j = 0; j < EPL; j++) {
        const int e = EPL * lane + j;
        if (e < n_expert) {
            first[e] = pos;
            sfirst[e] = spos;
            for (int q = 0; q < ns[j]; q++)
                reinterpret_cast<int4 *>(&dp.slots[spos + q])[0] =
                    make_int4(e, pos + q * chunk, min(chunk, c[j] - q * chunk), n_used);
        }
        pos += c[j];
        spos += ns[j];
    }
    for (int u = n_used + lane; u < dp.slot_cap; u += WAVE) reinterpret_cast<int4 *>(&dp.slots[u])[0] = make_int4(0, 0, 0, 0);
    wave_lds_sync();
    // a pair's place among its expert's pairs: the earlier tokens with that
    // expert, from a token bitmap per expert (T <= 4 * WAVE / k <= 64 here)
    unsigned long long *bm = reinterpret_cast<unsigned long long *>(cnt); // cnt is read out above
    for (int e = lane; e < MAX_EXPERTS; e += WAVE) bm[e] = 0ull;
    wave_lds_sync();
    for (int i = lane; i < P; i += WAVE) atomicOr(&bm[ids[i]], 1ull << (i / k));
    wave_lds_sync();
    for (int i = lane; i < P; i += WAVE) {
        const int e = ids[i], t = i / k;
        const int r = __popcll(bm[e] & ((1ull << t) - 1ull));
        const int p = first[e] + r;
        dp.pair_tok[p] = t;
        dp.pair_exp[p] = e;
        dp.pair_w[p] = wts[i];
        // positions ascend with the expert id: the pair's place among the
        // token's k is the number of its experts below e
        int rank = 0;
        for (int j2 = 0; j2 < k; j2++) rank += ids[t * k + j2] < e;
        dp.tok_pairs[(size_t)t * k + rank] = p;
        if (r % chunk < SLOT_TOKS) dp.slots[sfirst[e] + r / chunk].tok[r % chunk] = t;
    }
}

// The same dispatch for P <= WAVE pairs with every expert's pairs in one
// slot (T <= chunk), by one wavefront with no per-expert arrays: lane i takes
// pair i and counts, over all pairs j, those of a lower expert, those of its
// expert from earlier tokens (a token names an expert once) and those of its
// own token with a lower expert.  Its dispatch position is the first two
// counts, the first count its expert's first position; a first pair marks
// that position, and the marks below it, as a ballot, number the expert's
// slot.  mark is an LDS array of WAVE ints.
#ifndef BIV_SMALL_SORT_P
#define BIV_SMALL_SORT_P 16 // pairs up to which the route takes sort_pairs_small (measured: faster up to T = 2)
#endif
__device__ void sort_pairs_small(const int *ids, const float *wts, int k, int T, const Dispatch &dp, int *mark)
{
    const int lane = threadIdx.x & (WAVE - 1);
    const int P = T * k;
    const bool act = lane < P;
    const int e = act ? ids[lane] : 0x7FFFFFFF;
    const int t = lane / k, t0 = t * k;
    int lt = 0, eqb = 0, eqt = 0, rk = 0;
    // every id first (P is a multiple of 4 here), then the counts
    int4 q[WAVE / 4];
#pragma unroll
    for (int r = 0; r < WAVE / 4; r++)
        if (4 * r < P) q[r] = *reinterpret_cast<const int4 *>(ids + 4 * r); // uniform
#pragma unroll
    for (int r = 0; r < WAVE / 4; r++) {
        if (4 * r >= P) break; // uniform
        const int ej[4] = {q[r].x, q[r].y, q[r].z, q[r].w};
#pragma unroll
        for (int u = 0; u < 4; u++) {
            const int j = 4 * r + u;
            const bool below = ej[u] < e, eq = ej[u] == e;
            lt += below;
            eqt += eq;
            eqb += eq && j < t0;
            rk += below && j >= t0 && j < t0 + k;
        }
    }
    const int pos = lt + eqb;
    mark[lane] = 0;
    wave_lds_sync();
    if (act && eqb == 0) mark[pos] = 1;
    wave_lds_sync();
    const unsigned long long firsts = __ballot(mark[lane] != 0);
    const int n_used = __popcll(firsts);
    if (act) {
        const int slot = __popcll(firsts & ((1ull << lt) - 1ull)); // lt: the expert's first position
        dp.pair_tok[pos] = t;
        dp.pair_exp[pos] = e;
        dp.pair_w[pos] = wts[lane];
        dp.tok_pairs[t0 + rk] = pos;
        if (eqb == 0) reinterpret_cast<int4 *>(&dp.slots[slot])[0] = make_int4(e, pos, eqt, n_used);
        if (eqb < SLOT_TOKS) dp.slots[slot].tok[eqb] = t;
    }
    for (int u = n_used + lane; u < dp.slot_cap; u += WAVE) reinterpret_cast<int4 *>(&dp.slots[u])[0] = make_int4(0, 0, 0, 0);
}

// The counting sort past one workgroup (the `routed` lists of
// model.rs:866-873, Metal's moe_sort): tokens in blocks of RS_WAVES.
// route_block_counts: block b's per-expert pair counts, work[b * 256 + e].
// k_dispatch_scan (one workgroup): turns them, in place, into each block's
// first rank within the expert; each expert's first dispatch position and
// first slot (work[nb * 256 + e], work[(nb + 1) * 256 + e]); the slot
// records.  k_dispatch_place: every pair to its position, a pair's place
// among its expert's pairs being its block's first rank plus the earlier
// tokens of its block with that expert (a token bitmap in LDS).  No atomics
// on values: the order is that of the single-workgroup sort.
constexpr int RB_TOKS = RS_THREADS / WAVE; // tokens per block

__device__ inline void block_masks(const int *ids, int n_expert, int k, int T, int b, unsigned *mask)
{
    const int t0 = b * RB_TOKS, nt = min(RB_TOKS, T - t0);
    for (int e = threadIdx.x; e < MAX_EXPERTS; e += blockDim.x) mask[e] = 0u;
    __syncthreads();
    for (int i = threadIdx.x; i < nt * k; i += blockDim.x) atomicOr(&mask[ids[(size_t)t0 * k + i]], 1u << (i / k));
    __syncthreads();
}

__device__ void route_block_counts(const int *ids, int n_expert, int k, int T, int b, int *work)
{
    __shared__ unsigned mask[MAX_EXPERTS];
    block_masks(ids, n_expert, k, T, b, mask);
    for (int e = threadIdx.x; e < MAX_EXPERTS; e += blockDim.x) work[(size_t)b * MAX_EXPERTS + e] = __popc(mask[e]);
}

// The experts' exclusive scans, one thread per expert e (lane, wave w of
// MAX_EXPERTS / WAVE; every thread of the workgroup calls it, `writer` those
// of the first MAX_EXPERTS): its first dispatch position (pairs in expert
// order) and its first slot.  Slots are numbered with the experts whose
// pairs fill at most half a slot last: their cheap units then go out last
// and fill the grid's tail.  An expert's slots stay consecutive (their
// workgroups share its weights through L2).  n_used: the slots in use.
__device__ inline void expert_scan(int tot, int chunk, bool writer, int (&wsum)[3][MAX_EXPERTS / WAVE], int &first,
                                   int &sfirst, int &n_used)
{
    const int lane = threadIdx.x & (WAVE - 1), w = (threadIdx.x & (MAX_EXPERTS - 1)) >> 6;
    const int nsl = (tot + chunk - 1) / chunk;
    const bool light = tot > 0 && 2 * tot <= chunk;
    const int x = wave_incl_scan(tot), yh = wave_incl_scan(light ? 0 : nsl), yl = wave_incl_scan(light ? nsl : 0);
    if (writer && lane == WAVE - 1) {
        wsum[0][w] = x;
        wsum[1][w] = yh;
        wsum[2][w] = yl;
    }
    __syncthreads();
    int px = 0, ph = 0, pl = 0, n_heavy = 0, n_light = 0;
    for (int i = 0; i < MAX_EXPERTS / WAVE; i++) {
        if (i < w) {
            px += wsum[0][i];
            ph += wsum[1][i];
            pl += wsum[2][i];
        }
        n_heavy += wsum[1][i];
        n_light += wsum[2][i];
    }
    first = px + x - tot;
    sfirst = light ? n_heavy + pl + yl - nsl : ph + yh - nsl;
    n_used = n_heavy + n_light;
}

constexpr int DS_SPLIT = 4; // threads per expert column in k_dispatch_scan
// Up to DS_RUNS * 16 blocks (T <= 4096) a thread of k_dispatch_scan takes
// four adjacent experts (one 16-byte load per block) over a run of at most
// 16 blocks, all its loads in flight at once.
constexpr int DS_RUNS = MAX_EXPERTS * DS_SPLIT / (MAX_EXPERTS / 4);
__global__ __launch_bounds__(MAX_EXPERTS *DS_SPLIT) void k_dispatch_scan(int n_expert, int nb, int chunk, Dispatch dp,
                                                                         int *work)
{
    // Each block's exclusive prefix per expert, in place, and each expert's
    // total (integer sums: the result does not depend on how the blocks are
    // split between threads)
    const int e = threadIdx.x & (MAX_EXPERTS - 1), qs = threadIdx.x / MAX_EXPERTS;
    int run = 0;
    if (nb <= DS_RUNS * 16) {
        __shared__ int part[DS_RUNS][MAX_EXPERTS];
        const int q4 = threadIdx.x % (MAX_EXPERTS / 4), r = threadIdx.x / (MAX_EXPERTS / 4);
        const int nbr = (nb + DS_RUNS - 1) / DS_RUNS, lo = min(nb, r * nbr), hi = min(nb, lo + nbr);
        int4 *w4 = reinterpret_cast<int4 *>(work);
        int4 v[16];
#pragma unroll
        for (int j = 0; j < 16; j++)
            v[j] = lo + j < hi ? w4[(size_t)(lo + j) * (MAX_EXPERTS / 4) + q4] : make_int4(0, 0, 0, 0);
        int4 sm = make_int4(0, 0, 0, 0);
#pragma unroll
        for (int j = 0; j < 16; j++) {
            sm.x += v[j].x;
            sm.y += v[j].y;
            sm.z += v[j].z;
            sm.w += v[j].w;
        }
        reinterpret_cast<int4 *>(&part[r][0])[q4] = sm;
        __syncthreads();
        int4 rn = make_int4(0, 0, 0, 0);
        for (int i = 0; i < r; i++) {
            const int4 pv = reinterpret_cast<const int4 *>(&part[i][0])[q4];
            rn.x += pv.x;
            rn.y += pv.y;
            rn.z += pv.z;
            rn.w += pv.w;
        }
#pragma unroll
        for (int j = 0; j < 16; j++) {
            if (lo + j < hi) w4[(size_t)(lo + j) * (MAX_EXPERTS / 4) + q4] = rn;
            rn.x += v[j].x;
            rn.y += v[j].y;
            rn.z += v[j].z;
            rn.w += v[j].w;
        }
        for (int i = 0; i < DS_RUNS; i++) run += part[i][e];
    } else {
        // DS_SPLIT threads per expert, each over a run of the blocks: its
        // sum, the runs' offsets, then its blocks' prefixes (16 loads in
        // flight at a time, twice)
        __shared__ int part[DS_SPLIT][MAX_EXPERTS];
        const int nbq = (nb + DS_SPLIT - 1) / DS_SPLIT, b_lo = min(nb, qs * nbq), b_hi = min(nb, b_lo + nbq);
        int sum = 0;
        for (int b0 = b_lo; b0 < b_hi; b0 += 16) {
            int v[16];
#pragma unroll
            for (int j = 0; j < 16; j++) v[j] = b0 + j < b_hi ? work[(size_t)(b0 + j) * MAX_EXPERTS + e] : 0;
#pragma unroll
            for (int j = 0; j < 16; j++) sum += v[j];
        }
        part[qs][e] = sum;
        __syncthreads();
        for (int i = 0; i < qs; i++) run += part[i][e];
        for (int b0 = b_lo; b0 < b_hi; b0 += 16) {
            int v[16];
#pragma unroll
            for (int j = 0; j < 16; j++) v[j] = b0 + j < b_hi ? work[(size_t)(b0 + j) * MAX_EXPERTS + e] : 0;
#pragma unroll
            for (int j = 0; j < 16; j++) {
                if (b0 + j < b_hi) work[(size_t)(b0 + j) * MAX_EXPERTS + e] = run;
                run += v[j];
            }
        }
        run = 0;
        for (int i = 0; i < DS_SPLIT; i++) run += part[i][e];
    }
    const int tot = e < n_expert ? run : 0, nsl = (tot + chunk - 1) / chunk;
    __shared__ int wsum[3][MAX_EXPERTS / WAVE];
    int first, sfirst, n_used;
    expert_scan(tot, chunk, qs == 0, wsum, first, sfirst, n_used);
    if (qs != 0) return; // the records: one thread per expert
    work[(size_t)nb * MAX_EXPERTS + e] = first;
    work[(size_t)(nb + 1) * MAX_EXPERTS + e] = sfirst;
    for (int j = 0; j < nsl; j++)
        reinterpret_cast<int4 *>(&dp.slots[sfirst + j])[0] =
            make_int4(e, first + j * chunk, min(chunk, tot - j * chunk), n_used);
    for (int u = n_used + e; u < dp.slot_cap; u += MAX_EXPERTS) reinterpret_cast<int4 *>(&dp.slots[u])[0] = make_int4(0, 0, 0, 0);
}

// Up to DP_FUSE_NB blocks, k_dispatch_place<true> runs k_dispatch_scan's
// arithmetic itself (one launch fewer): every workgroup reads the whole
// count table (a column of at most DP_FUSE_NB counts per thread, all loads
// in flight at once) for its block's first ranks and the experts' first
// positions and slots; workgroup 0 writes the slot records.  The same
// integer sums, so the same dispatch.
constexpr int DP_FUSE_NB = 32;

template <bool FUSED>
__global__ __launch_bounds__(MAX_EXPERTS) void k_dispatch_place(int n_expert, int k, int T, int nb, int chunk,
                                                                Dispatch dp, const int *work)
{
    __shared__ unsigned mask[MAX_EXPERTS];
    __shared__ int base_s[FUSED ? MAX_EXPERTS : 1], first_s[FUSED ? MAX_EXPERTS : 1],
        sfirst_s[FUSED ? MAX_EXPERTS : 1];
    const int b = blockIdx.x, t0 = b * RB_TOKS, nt = min(RB_TOKS, T - t0);
    const int *base, *first, *sfirst;
    if constexpr (FUSED) {
        const int e = threadIdx.x;
        int v[DP_FUSE_NB];
#pragma unroll
        for (int j = 0; j < DP_FUSE_NB; j++) v[j] = j < nb ? work[(size_t)j * MAX_EXPERTS + e] : 0;
        int tot = 0, bse = 0;
#pragma unroll
        for (int j = 0; j < DP_FUSE_NB; j++) {
            if (j == b) bse = tot;
            tot += v[j];
        }
        if (e >= n_expert) tot = 0;
        const int nsl = (tot + chunk - 1) / chunk;
        __shared__ int wsum[3][MAX_EXPERTS / WAVE];
        int fst, sfst, n_used;
        expert_scan(tot, chunk, true, wsum, fst, sfst, n_used);
        base_s[e] = bse;
        first_s[e] = fst;
        sfirst_s[e] = sfst;
        if (b == 0) {
            for (int j = 0; j < nsl; j++)
                reinterpret_cast<int4 *>(&dp.slots[sfst + j])[0] =
                    make_int4(e, fst + j * chunk, min(chunk, tot - j * chunk), n_used);
            for (int u = n_used + e; u < dp.slot_cap; u += MAX_EXPERTS)
                reinterpret_cast<int4 *>(&dp.slots[u])[0] = make_int4(0, 0, 0, 0);
        }
        base = base_s;
        first = first_s;
        sfirst = sfirst_s;
    } else {
        base = work + (size_t)b * MAX_EXPERTS;
        first = work + (size_t)nb * MAX_EXPERTS;
        sfirst = work + (size_t)(nb + 1) * MAX_EXPERTS;
    }
    block_masks(dp.ids, n_expert, k, T, b, mask);
    for (int i = threadIdx.x; i < nt * k; i += blockDim.x) {
        const int tl = i / k, t = t0 + tl;
        const int e = dp.ids[(size_t)t0 * k + i];
        const int r = base[e] + __popc(mask[e] & ((1u << tl) - 1u)); // rank among the expert's pairs
        const int p = first[e] + r;
        dp.pair_tok[p] = t;
        dp.pair_exp[p] = e;
        dp.pair_w[p] = dp.wts[(size_t)t0 * k + i];
        int rank = 0; // among the token's experts, ascending id
        for (int j = 0; j < k; j++) rank += dp.ids[(size_t)t * k + j] < e;
        dp.tok_pairs[(size_t)t * k + rank] = p;
        if (r % chunk < SLOT_TOKS) dp.slots[sfirst[e] + r / chunk].tok[r % chunk] = t;
    }
}

// One wavefront per token routes it, then the pairs are sorted: with a
// single workgroup (T <= RS_WAVES, so at most 4 * WAVE pairs as k <= 16) by
// one wavefront from LDS, else by the counting sort above (each routing
// workgroup counts its block; k_dispatch_scan and k_dispatch_place follow).
constexpr int RS_WAVES = RS_THREADS / WAVE;

__global__ __launch_bounds__(RS_THREADS) void k_route_sort(const float *__restrict__ logits, int n_expert, int k,
                                                           int T, int chunk, Dispatch dp, int *work)
{
    __shared__ float es[RS_WAVES][MAX_EXPERTS];
    __shared__ __align__(16) int lds_ids[RS_WAVES * 16];
    __shared__ float lds_wts[RS_WAVES * 16];
    const int wave = threadIdx.x >> 6, nw = blockDim.x >> 6;
    const bool single = gridDim.x == 1;
    // the first token's logits and the exp table go out together
    __shared__ uint64_t tab[32];
    const int t0 = blockIdx.x * nw + wave;
    float lg[RPER];
    if (t0 < T) load_logits(logits, n_expert, t0, lg);
    if (threadIdx.x < 32) tab[threadIdx.x] = exp_tab_g[threadIdx.x];
    __syncthreads();
    for (int t = t0; t < T; t += gridDim.x * nw) {
        if (t != t0) load_logits(logits, n_expert, t, lg);
        route_token(lg, tab, n_expert, k, t, es[wave], dp.ids, dp.wts, single ? lds_ids : nullptr,
                    single ? lds_wts : nullptr);
    }
    if (single) {
        // the routes from LDS, sorted by one wavefront
        __shared__ int cnt[2 * MAX_EXPERTS], first[MAX_EXPERTS], sfirst[MAX_EXPERTS]; // cnt: later a u64 bitmap
        __syncthreads();
        if (wave == 0) {
            if (T * k <= BIV_SMALL_SORT_P && (T * k) % 4 == 0 && T <= chunk)
                sort_pairs_small(lds_ids, lds_wts, k, T, dp, cnt);
            else sort_pairs_wave(lds_ids, lds_wts, n_expert, k, T, chunk, dp, cnt, first, sfirst);
        }
        return;
    }
    if (single) return;
    // past one workgroup: this block's expert counts for the counting sort
    // (k_dispatch_scan, k_dispatch_place); block b holds tokens 16 b .. 16 b + 15
    __syncthreads();
    route_block_counts(dp.ids, n_expert, k, T, blockIdx.x, work);
}

// ---------------------------------------------------------------------------
// Expert rows as 16 FMA chains.  Chain<TY, K> holds, in registers, what lane
// (pi, l) of a 16-lane group needs of one weight row: word l of the blocks of
// parity pi and their scales.  partial(s, x) is the i32 the reference's ymm
// lane l holds for block 2s + pi; wscale(s) the weight half of the block's
// f32 scale.

template <int TY, int K> struct Chain;

// Q8_0: dot_i8_i8 lane l = bytes 4l..4l+3 of the block; scale f16(d)
// (quant.rs:1368-1382)
template <int K> struct Chain<T_Q8_0, K> {
    static constexpr int S = K / 64;
    static constexpr int NLOAD_MIN = S / 4; // vector loads of a load_chunk, at least
    int w[S];
    int hw[S / 2]; // the f16 scales, two per register
    // chunk c (elements cK .. cK + K - 1) of a row of KF elements: the
    // quants of a chunk are contiguous, its scales sit at step cS of each
    // parity's run
    __device__ inline void load_chunk(const DevMat &M, size_t mrow, int KF, int c, int pi, int l)
    {
        const int4 *q = reinterpret_cast<const int4 *>(M.q + mrow * KF + (size_t)c * K);
#pragma unroll
        for (int i = 0; i < S / 4; i++) {
            int4 v = q[i * 16 + pi * 8 + l];
            w[4 * i] = v.x;
            w[4 * i + 1] = v.y;
            w[4 * i + 2] = v.z;
            w[4 * i + 3] = v.w;
        }
        ld_words(M.s + 2 * (mrow * (KF / 32) + pi * (KF / 64) + (size_t)c * S), hw);
    }
    __device__ inline void load(const DevMat &M, size_t mrow, int pi, int l) { load_chunk(M, mrow, K, 0, pi, l); }
    __device__ inline int partial(int s, int x) const { return dot4(w[s], x, 0); }
    __device__ inline float wscale(int s) const
    {
        const unsigned h = (unsigned)hw[s >> 1] >> (16 * (s & 1));
        return __half2float(__ushort_as_half((unsigned short)(h & 0xFFFF)));
    }
};

// Q4_K: dot_u8_i8 of the low (pi 0) or high (pi 1) nibbles; scale d * sc
// of sub-block 2s + pi (quant.rs:1384-1423)
template <int K> struct Chain<T_Q4K, K> {
    static constexpr int S = K / 64;
    static constexpr int NLOAD_MIN = S / 4; // vector loads of a load_chunk, at least
    // the nibbles of steps 2m (low) and 2m + 1 (high) of each byte in wp[m];
    // per super-block its f32 d and the four sub-scales of this parity as
    // bytes: half the registers of whole words and f32 scales, for more
    // waves per SIMD
    int wp[S / 2];
    float ds[S / 4];
    int scp[S / 4];
    __device__ inline void load(const DevMat &M, size_t mrow, int pi, int l) { load_chunk(M, mrow, K, 0, pi, l); }
    __device__ inline void load_chunk(const DevMat &M, size_t mrow, int KF, int c, int pi, int l)
    {
        const int4 *q = reinterpret_cast<const int4 *>(M.q + mrow * (KF / 2) + (size_t)c * (K / 2));
        const int sh = 4 * pi;
#pragma unroll
        for (int i = 0; i < S / 4; i++) {
            int4 v = q[i * 8 + l];
            const unsigned w0 = ((unsigned)v.x >> sh) & 0x0F0F0F0Fu, w1 = ((unsigned)v.y >> sh) & 0x0F0F0F0Fu;
            const unsigned w2 = ((unsigned)v.z >> sh) & 0x0F0F0F0Fu, w3 = ((unsigned)v.w >> sh) & 0x0F0F0F0Fu;
            wp[2 * i] = (int)(w0 | (w1 << 4));
            wp[2 * i + 1] = (int)(w2 | (w3 << 4));
        }
        const int4 *hd = reinterpret_cast<const int4 *>(M.s + 16 * (mrow * (KF / 256) + (size_t)c * (K / 256)));
#pragma unroll
        for (int i = 0; i < S / 4; i++) {
            const int4 h = hd[i];
            ds[i] = __half2float(__ushort_as_half((unsigned short)(h.x & 0xFFFF)));
            unsigned packed = 0;
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const int sb = 2 * j + pi;
                int sc;
                if (sb < 4) sc = byte_at(h, 4 + sb) & 63;
                else sc = (byte_at(h, 4 + sb + 4) & 0xF) | ((byte_at(h, 4 + sb - 4) >> 6) << 4);
                packed |= (unsigned)sc << (8 * j);
            }
            scp[i] = (int)packed;
        }
    }
    __device__ inline int partial(int s, int x) const
    {
        const unsigned w = (unsigned)wp[s >> 1];
        return dot4((int)((s & 1) ? (w >> 4) & 0x0F0F0F0Fu : w & 0x0F0F0F0Fu), x, 0);
    }
    // d * sc of the step's sub-block, the product the reference forms
    __device__ inline float wscale(int s) const
    {
        return ds[s >> 2] * (float)(((unsigned)scp[s >> 2] >> (8 * (s & 3))) & 0xFF);
    }
};

// Q6_K: lanes of madd(maddubs(q, x) - maddubs(32, x), sc), lanes 0-3 under
// the block's first sub-scale and 4-7 under its second; scale d
// (quant.rs:1475-1533)
template <int K> struct Chain<T_Q6K, K> {
    static constexpr int S = K / 64;
    static constexpr int NLOAD_MIN = S / 4; // vector loads of a load_chunk, at least
    int ql[S / 2], qh[S / 2];
    int sc[S];
    float dd[S / 4];
    int pi_;
    __device__ inline void load(const DevMat &M, size_t mrow, int pi, int l) { load_chunk(M, mrow, K, 0, pi, l); }
    __device__ inline void load_chunk(const DevMat &M, size_t mrow, int KF, int c, int pi, int l)
    {
        const uint8_t *base = M.q + mrow * (KF / 256) * 192;
        const int4 *pl = reinterpret_cast<const int4 *>(base + (size_t)c * (K / 256) * 128);
        const int4 *ph = reinterpret_cast<const int4 *>(base + (KF / 256) * 128 + (size_t)c * (K / 256) * 64);
#pragma unroll
        for (int i = 0; i < S / 8; i++) {
            int4 v = pl[i * 16 + pi * 8 + l];
            ql[4 * i] = v.x;
            ql[4 * i + 1] = v.y;
            ql[4 * i + 2] = v.z;
            ql[4 * i + 3] = v.w;
            int4 u = ph[i * 8 + l];
            qh[4 * i] = u.x;
            qh[4 * i + 1] = u.y;
            qh[4 * i + 2] = u.z;
            qh[4 * i + 3] = u.w;
        }
        int sw[S / 4];
        ld_words(M.s + mrow * (KF / 16) + lay::q6k_sc(KF, pi, l >= 4, c * S), sw);
#pragma unroll
        for (int i = 0; i < S / 4; i++)
#pragma unroll
            for (int c = 0; c < 4; c++) sc[4 * i + c] = (int)(signed char)(((unsigned)sw[i] >> (8 * c)) & 0xFF);
        const unsigned short *dp = reinterpret_cast<const unsigned short *>(M.d + 2 * (mrow * (KF / 256) + (size_t)c * (K / 256)));
#pragma unroll
        for (int i = 0; i < S / 4; i++) dd[i] = __half2float(__ushort_as_half(dp[i]));
        pi_ = pi;
    }
    __device__ inline int partial(int s, int x) const
    {
        const int qq = s >> 1, hi = s & 1, k = pi_ + 2 * hi;
        const unsigned lo = hi ? (((unsigned)ql[qq] >> 4) & 0x0F0F0F0Fu) : ((unsigned)ql[qq] & 0x0F0F0F0Fu);
        const unsigned hb = (((unsigned)qh[qq] >> (2 * k)) & 0x03030303u) << 4;
        // a 24-bit product (full rate; a 32-bit multiply is quarter rate):
        // |dot| <= 4 * 63 * 128 + 32 * 512 and sc is int8, so it is the same
        // integer.  In asm: for __mul24 the compiler sign-extends both
        // operands and, in some kernels, still emits the 32-bit multiply.
        const int d = dot4((int)(lo | hb), x, 0) - 32 * dot4(0x01010101, x, 0);
        int r;
        asm("v_mul_i32_i24 %0, %1, %2" : "=v"(r) : "v"(sc[s]), "v"(d));
        return r;
    }
    __device__ inline float wscale(int s) const { return dd[s >> 2]; }
};

// BF16: dot_bf16 (quant.rs:1228-1256) with f32 activations; chain L = 8 pi + l
// holds elements L, L + 16, ... (layout.hpp bf16_elem), two per register.
template <int K> struct Chain<T_BF16, K> {
    static constexpr int S = K / 16;
    static constexpr int NLOAD_MIN = S / 8; // vector loads of a load_chunk, at least
    int w[S / 2];
    __device__ inline void load(const DevMat &M, size_t mrow, int pi, int l) { load_chunk(M, mrow, K, 0, pi, l); }
    __device__ inline void load_chunk(const DevMat &M, size_t mrow, int KF, int c, int pi, int l)
    {
        const int4 *q = reinterpret_cast<const int4 *>(M.q + (mrow * KF + (size_t)c * K) * 2);
#pragma unroll
        for (int g = 0; g < S / 8; g++) {
            const int4 v = q[g * 16 + pi * 8 + l];
            w[4 * g] = v.x;
            w[4 * g + 1] = v.y;
            w[4 * g + 2] = v.z;
            w[4 * g + 3] = v.w;
        }
    }
    __device__ inline float wval(int s) const
    {
        const unsigned u = (unsigned)w[s >> 1];
        return __uint_as_float(s & 1 ? (u & 0xFFFF0000u) : (u << 16));
    }
};

// What lane (pi, l) needs of one Q8 activation row: word l of the blocks of
// parity pi and their scales.
template <int K> struct XChain {
    static constexpr int S = K / 64;
    int x[S];
    float d[S];
    __device__ inline void load(const int8_t *xq, const float *xd, size_t xrow, int pi, int l)
    {
        const int4 *q = reinterpret_cast<const int4 *>(xq + xrow * K);
#pragma unroll
        for (int i = 0; i < S / 4; i++) {
            int4 v = q[i * 16 + pi * 8 + l];
            x[4 * i] = v.x;
            x[4 * i + 1] = v.y;
            x[4 * i + 2] = v.z;
            x[4 * i + 3] = v.w;
        }
        const float4 *dq = reinterpret_cast<const float4 *>(xd + xrow * (K / 32) + pi * S);
#pragma unroll
        for (int i = 0; i < S / 4; i++) {
            float4 v = dq[i];
            d[4 * i] = v.x;
            d[4 * i + 1] = v.y;
            d[4 * i + 2] = v.z;
            d[4 * i + 3] = v.w;
        }
    }
};

// Q4_K mins, summed apart and subtracted last (quant.rs:1418-1422):
// mins += dmin * (m_a * s_a + m_b * s_b) over the sub-block pairs in order.
template <int K>
__device__ inline float q4k_mins(const DevMat &M, size_t mrow, const float *xs, size_t xrow)
{
    constexpr int S = K / 64;
    const int4 *hd = reinterpret_cast<const int4 *>(M.s + 16 * (mrow * (K / 256)));
    const float *sr = xs + xrow * (K / 32);
    float mins = 0.0f;
    for (int i = 0; i < S / 4; i++) {
        const int4 h = hd[i];
        const float dmin = __half2float(__ushort_as_half((unsigned short)((unsigned)h.x >> 16)));
        for (int j = 0; j < 4; j++) {
            const int sa = 2 * j, sb = 2 * j + 1;
            const int ma = sa < 4 ? byte_at(h, 4 + sa + 4) & 63
                                  : (byte_at(h, 4 + sa + 4) >> 4) | ((byte_at(h, 4 + sa) >> 6) << 4);
            const int mb = sb < 4 ? byte_at(h, 4 + sb + 4) & 63
                                  : (byte_at(h, 4 + sb + 4) >> 4) | ((byte_at(h, 4 + sb) >> 6) << 4);
            const int s = 4 * i + j;
            mins = mins + dmin * ((float)ma * sr[lay::q8_scale(K, 2 * s)] +
                                  (float)mb * sr[lay::q8_scale(K, 2 * s + 1)]);
        }
    }
    return mins;
}

// q4k_mins by the 16 lanes of a group (lane ln of the group, every lane
// calling it for the same row and input row): lane ln forms the terms s =
// ln, ln + 16, ... (the loads of all terms in flight at once, where one lane
// would wait on them in turn), then the group's first lane adds them in
// index order, so its sum is q4k_mins's to the bit (the other lanes' are
// not: only the first lane's result is used).
template <int K>
__device__ inline float q4k_mins_group(const DevMat &M, size_t mrow, const float *xs, size_t xrow, int ln)
{
    constexpr int S = K / 64;          // sub-block pairs: the terms
    constexpr int R = (S + 15) / 16;   // terms per lane
    const int4 *hd = reinterpret_cast<const int4 *>(M.s + 16 * (mrow * (K / 256)));
    const float *sr = xs + xrow * (K / 32);
    float term[R];
#pragma unroll
    for (int r = 0; r < R; r++) {
        const int s = ln + 16 * r;
        term[r] = 0.0f;
        if (s < S) {
            const int4 h = hd[s >> 2];
            const int j = s & 3;
            const float dmin = __half2float(__ushort_as_half((unsigned short)((unsigned)h.x >> 16)));
            const int sa = 2 * j, sb = 2 * j + 1;
            const int ma = sa < 4 ? byte_at(h, 4 + sa + 4) & 63
                                  : (byte_at(h, 4 + sa + 4) >> 4) | ((byte_at(h, 4 + sa) >> 6) << 4);
            const int mb = sb < 4 ? byte_at(h, 4 + sb + 4) & 63
                                  : (byte_at(h, 4 + sb + 4) >> 4) | ((byte_at(h, 4 + sb) >> 6) << 4);
            term[r] = dmin * ((float)ma * sr[lay::q8_scale(K, 2 * s)] + (float)mb * sr[lay::q8_scale(K, 2 * s + 1)]);
        }
    }
    // the sum in index order in the group's first lane: its term r of lane
    // k reaches it through k single-lane rotations within the 16-lane row
    // (DPP row_shl:1, no LDS)
    float mins = 0.0f;
#pragma unroll
    for (int r = 0; r < R; r++) {
        float x = term[r];
#pragma unroll
        for (int k = 0; k < 16; k++) {
            if (16 * r + k >= S) break;
            mins = mins + x;
            if (k < 15) x = __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(x), 0x101, 0xF, 0xF, false));
        }
    }
    return mins; // in the group's first lane
}

// The Q4_K mins of chunk c of a row of KF (q4k_mins over that chunk's
// sub-block pairs), added to `mins` in the reference's order.
template <int K>
__device__ inline float q4k_mins_chunk(const DevMat &M, size_t mrow, int KF, int c, const float *xs, size_t xrow,
                                       float mins)
{
    constexpr int S = K / 64;
    const int4 *hd = reinterpret_cast<const int4 *>(M.s + 16 * (mrow * (KF / 256) + (size_t)c * (K / 256)));
    const float *sr = xs + xrow * (KF / 32);
    for (int i = 0; i < S / 4; i++) {
        const int4 h = hd[i];
        const float dmin = __half2float(__ushort_as_half((unsigned short)((unsigned)h.x >> 16)));
        for (int j = 0; j < 4; j++) {
            const int sa = 2 * j, sb = 2 * j + 1;
            const int ma = sa < 4 ? byte_at(h, 4 + sa + 4) & 63
                                  : (byte_at(h, 4 + sa + 4) >> 4) | ((byte_at(h, 4 + sa) >> 6) << 4);
            const int mb = sb < 4 ? byte_at(h, 4 + sb + 4) & 63
                                  : (byte_at(h, 4 + sb + 4) >> 4) | ((byte_at(h, 4 + sb) >> 6) << 4);
            const int sg = c * S + 4 * i + j; // sub-block pair of the whole row
            mins = mins + dmin * ((float)ma * sr[lay::q8_scale(KF, 2 * sg)] + (float)mb * sr[lay::q8_scale(KF, 2 * sg + 1)]);
        }
    }
    return mins;
}

// ---------------------------------------------------------------------------
// Matvecs over rows of any length (a multiple of LK): dense_ffn's gate/up
// and down (model.rs:1118-1126) for the qwen35 dense FFN, whose rows are
// longer than the experts'.  The row streams through in chunks of LK
// elements; the 16 chains of a (row, token) run on across chunks, so every
// sum is the reference's x86 order over the whole row.  A workgroup takes
// LXT tokens and a block of rows: 8 of gate and up (the SwiGLU formed in
// registers) or 16 of down.  Chunk c + 1's weights (registers) and
// activations (LDS) load while chunk c computes.
constexpr int LK = 512;
constexpr int LXT = 8;
#ifndef BIV_LONG_FULL_LDS
#define BIV_LONG_FULL_LDS (96 * 1024)
#endif
constexpr size_t LONG_FULL_LDS = BIV_LONG_FULL_LDS; // LDS bytes up to which a workgroup stages every chunk

// FULL: every chunk of the workgroup's activation rows is staged in LDS
// (dynamic, nc buffers) before the loop, so the loop only streams weights,
// LPD chunks ahead in a ring of registers whose waits the compiler places
// (gate/up: two for five tokens or more, whose accumulators and staged
// operands leave registers for fewer chunks, the freed ones buying a wave per
// SIMD; down: eight, its 4-row waves being too few for more than one wave
// per SIMD anyway, so that registers go to bytes in flight).
#ifndef BIV_LONG_LPD
#define BIV_LONG_LPD 4
#endif
#ifndef BIV_LONG_LPD_DN
#define BIV_LONG_LPD_DN 8
#endif
template <int XTT, bool GATEUP> constexpr int long_lpd() { return GATEUP ? (XTT >= 5 ? 2 : BIV_LONG_LPD) : BIV_LONG_LPD_DN; }

template <int TY, bool GATEUP, int XTT, int WV>
__global__ __launch_bounds__(WV *WAVE) void k_chain_mv_long_full(LongArgs a)
{
    constexpr int LPD = long_lpd<XTT, GATEUP>();
    constexpr int K = LK, S = K / 64, ROW16 = K / 16 + K / 128, NTH = WV * WAVE;
    constexpr bool BF = TY == T_BF16;
    extern __shared__ int4 dyn[]; // [nc chunks][nt rows][16-byte pieces of a chunk's row]
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int grp = lane >> 4, ln = lane & 15, pi = ln >> 3, l = ln & 7;
    constexpr int RPW = GATEUP ? 2 : 4;
    const int row = (blockIdx.x * WV + wave) * RPW + (GATEUP ? grp >> 1 : grp);
    const int m = GATEUP ? (grp & 1) : 0;
    DevMat M = a.a;
    if (GATEUP && m) {
        M.q += a.b.q - M.q;
        M.s += a.b.s - M.s;
        M.d += a.b.d - M.d;
    }
    const int rows = M.rows, KF = a.K, nc = KF / K;
    const bool row_ok = row < rows;
    const size_t mrow = row_ok ? row : 0;
    const int t0 = blockIdx.y * XTT, nt = min(XTT, a.T - t0);
    // every chunk of the nt rows, piece (c, j, r) at dyn[c * np + j * rp + r],
    // straight into LDS ahead of the weights (DMAs the compiler does not
    // track: its waits for the weights then leave the activations alone)
    const int rp = BF ? K / 4 : ROW16, np = nt * rp, npc = nc * np;
    for (int i0 = 0; i0 < npc; i0 += NTH) {
        const int i = i0 + (int)threadIdx.x;
        if (i >= npc) break;
        const int c = i / np, jr = i - c * np, j = jr / rp, r = jr - j * rp;
        const void *src;
        if constexpr (BF) {
            src = a.xf + (size_t)(t0 + j) * KF + (size_t)c * K + 4 * r;
        } else {
            const size_t x = (size_t)(t0 + j);
            if (r < K / 16) {
                src = a.xq + x * KF + (size_t)c * K + 16 * r;
            } else {
                const int r2 = r - K / 16, ppi = r2 / (S / 4), qq = r2 - ppi * (S / 4);
                src = a.xd + x * (KF / 32) + ppi * (KF / 64) + (size_t)c * S + 4 * qq;
            }
        }
        lds_dma16(static_cast<const float *>(src), reinterpret_cast<const float4 *>(dyn + i0 + wave * WAVE));
    }
    // then the first weight chunks
    Chain<TY, K> w[LPD];
#pragma unroll
    for (int d = 0; d < LPD; d++) w[d].load_chunk(M, mrow, KF, d < nc ? d : 0, pi, l);
    // this thread's DMAs are in once at most the weights' loads are
    // outstanding (loads complete in order); then every thread's
    __builtin_amdgcn_sched_barrier(0); // (the weights' loads stay above the wait)
    wait_vm<LPD * Chain<TY, K>::NLOAD_MIN>();
    rm_barrier();
    float acc[XTT], mins[XTT];
#pragma unroll
    for (int j = 0; j < XTT; j++) {
        acc[j] = 0.0f;
        mins[j] = 0.0f;
    }
    auto compute = [&](const Chain<TY, K> &wc, int c) {
        const int4 *st = dyn + c * np;
#pragma unroll
        for (int j = 0; j < XTT; j++) {
            if (j >= nt) break;
            if constexpr (BF) {
                const float *xr = reinterpret_cast<const float *>(st) + j * K;
#pragma unroll
                for (int s2 = 0; s2 < K / 16; s2++) acc[j] = fmaf(wc.wval(s2), xr[16 * s2 + ln], acc[j]);
            } else {
#pragma unroll
                for (int q = 0; q < S / 4; q++) {
                    const int4 xv = st[j * ROW16 + q * 16 + pi * 8 + l];
                    const float4 xd = *reinterpret_cast<const float4 *>(&st[j * ROW16 + K / 16 + pi * (S / 4) + q]);
                    const int xw[4] = {xv.x, xv.y, xv.z, xv.w};
                    const float xs[4] = {xd.x, xd.y, xd.z, xd.w};
#pragma unroll
                    for (int u = 0; u < 4; u++) {
                        const int s2 = 4 * q + u;
                        acc[j] = fmaf((float)wc.partial(s2, xw[u]), wc.wscale(s2) * xs[u], acc[j]);
                    }
                }
                if (TY == T_Q4K && ln == 0) mins[j] = q4k_mins_chunk<K>(M, mrow, KF, c, a.xs, (size_t)(t0 + j), mins[j]);
            }
        }
    };
    for (int c0 = 0; c0 < nc; c0 += LPD) {
#pragma unroll
        for (int d = 0; d < LPD; d++) {
            const int c = c0 + d;
            if (c < nc) {
                compute(w[d], c);
                if (c + LPD < nc) w[d].load_chunk(M, mrow, KF, c + LPD, pi, l);
            }
        }
    }
#pragma unroll
    for (int j = 0; j < XTT; j++) {
        if (j >= nt) break;
        float t = row_tree16(acc[j]); // valid in the group's first lane
        if (TY == T_Q4K) t = t - mins[j]; // (the first lane formed it)
        const size_t o = (size_t)(t0 + j) * rows + row;
        if (GATEUP) {
            const float up = from_lane_plus16(t); // (read by the gate groups' first lanes)
            if (m == 0 && ln == 0 && row_ok) a.out[o] = silu_mul(t, up);
        } else if (ln == 0 && row_ok) {
            a.out[o] = a.add ? a.out[o] + t : t;
        }
    }
}

template <int TY, bool GATEUP, int XTT, int WV>
__global__ __launch_bounds__(WV *WAVE) void k_chain_mv_long(LongArgs a)
{
    constexpr int K = LK, S = K / 64, ROW16 = K / 16 + K / 128, NTH = WV * WAVE;
    constexpr bool BF = TY == T_BF16;
    constexpr int PIECES = BF ? XTT * K / 4 : XTT * ROW16; // 16-byte pieces of one chunk's rows
    constexpr int NPC = (PIECES + NTH - 1) / NTH;
    __shared__ int4 stage[2][NPC * NTH];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int grp = lane >> 4, ln = lane & 15, pi = ln >> 3, l = ln & 7;
    constexpr int RPW = GATEUP ? 2 : 4;
    const int row = (blockIdx.x * WV + wave) * RPW + (GATEUP ? grp >> 1 : grp);
    const int m = GATEUP ? (grp & 1) : 0;
    DevMat M = a.a;
    if (GATEUP && m) { // up as gate plus a uniform offset (one pointer per plane)
        M.q += a.b.q - M.q;
        M.s += a.b.s - M.s;
        M.d += a.b.d - M.d;
    }
    const int rows = M.rows, KF = a.K, nc = KF / K;
    const bool row_ok = row < rows;
    const size_t mrow = row_ok ? row : 0;
    const int t0 = blockIdx.y * XTT, nt = min(XTT, a.T - t0);
    const int np = BF ? nt * (K / 4) : nt * ROW16;
    auto issue = [&](int c) {
        int4 *dst = &stage[c & 1][0];
#pragma unroll
        for (int q = 0; q < NPC; q++) {
            if (q * NTH >= np) break; // uniform
            const int idx0 = q * NTH + (int)threadIdx.x, idx = idx0 < np ? idx0 : np - 1;
            const void *src;
            if constexpr (BF) {
                const int j = idx / (K / 4), r = idx - j * (K / 4);
                src = a.xf + (size_t)(t0 + j) * KF + (size_t)c * K + 4 * r;
            } else {
                const int j = idx / ROW16, r = idx - j * ROW16;
                const size_t x = (size_t)(t0 + j);
                if (r < K / 16) {
                    src = a.xq + x * KF + (size_t)c * K + 16 * r;
                } else { // scale pieces: parity, then 4 of its scales
                    const int r2 = r - K / 16, ppi = r2 / (S / 4), qq = r2 - ppi * (S / 4);
                    src = a.xd + x * (KF / 32) + ppi * (KF / 64) + (size_t)c * S + 4 * qq;
                }
            }
            __builtin_amdgcn_global_load_lds(src, (__attribute__((address_space(3))) void *)(dst + q * NTH + wave * WAVE),
                                             16, 0, 0);
        }
    };
    float acc[XTT], mins[XTT];
#pragma unroll
    for (int j = 0; j < XTT; j++) {
        acc[j] = 0.0f;
        mins[j] = 0.0f;
    }
    auto compute = [&](const Chain<TY, K> &w, int c) {
        const int4 *st = &stage[c & 1][0];
#pragma unroll
        for (int j = 0; j < XTT; j++) {
            if (j >= nt) break;
            if constexpr (BF) {
                const float *xr = reinterpret_cast<const float *>(st) + j * K;
#pragma unroll
                for (int s2 = 0; s2 < K / 16; s2++) acc[j] = fmaf(w.wval(s2), xr[16 * s2 + ln], acc[j]);
            } else {
#pragma unroll
                for (int q = 0; q < S / 4; q++) {
                    const int4 xv = st[j * ROW16 + q * 16 + pi * 8 + l];
                    const float4 xd = *reinterpret_cast<const float4 *>(&st[j * ROW16 + K / 16 + pi * (S / 4) + q]);
                    const int xw[4] = {xv.x, xv.y, xv.z, xv.w};
                    const float xs[4] = {xd.x, xd.y, xd.z, xd.w};
#pragma unroll
                    for (int u = 0; u < 4; u++) {
                        const int s2 = 4 * q + u;
                        acc[j] = fmaf((float)w.partial(s2, xw[u]), w.wscale(s2) * xs[u], acc[j]);
                    }
                }
                if (TY == T_Q4K && ln == 0) mins[j] = q4k_mins_chunk<K>(M, mrow, KF, c, a.xs, (size_t)(t0 + j), mins[j]);
            }
        }
    };
    Chain<TY, K> w0, w1;
    issue(0);
    w0.load_chunk(M, mrow, KF, 0, pi, l);
    for (int c = 0; c < nc; c += 2) {
        __builtin_amdgcn_s_waitcnt(0);
        __syncthreads();
        if (c + 1 < nc) {
            issue(c + 1);
            w1.load_chunk(M, mrow, KF, c + 1, pi, l);
        }
        compute(w0, c);
        if (c + 1 >= nc) break;
        __builtin_amdgcn_s_waitcnt(0);
        __syncthreads();
        if (c + 2 < nc) {
            issue(c + 2);
            w0.load_chunk(M, mrow, KF, c + 2, pi, l);
        }
        compute(w1, c + 1);
    }
#pragma unroll
    for (int j = 0; j < XTT; j++) {
        if (j >= nt) break;
        float t = row_tree16(acc[j]); // valid in the group's first lane
        if (TY == T_Q4K) t = t - mins[j]; // (the first lane formed it)
        const size_t o = (size_t)(t0 + j) * rows + row;
        if (GATEUP) {
            const float up = from_lane_plus16(t); // (read by the gate groups' first lanes)
            if (m == 0 && ln == 0 && row_ok) a.out[o] = silu_mul(t, up);
        } else if (ln == 0 && row_ok) {
            a.out[o] = a.add ? a.out[o] + t : t;
        }
    }
}

// ---------------------------------------------------------------------------
// Combine for every token (model.rs:884-896): o = 0; for each of t's experts
// in ascending id, o = fma(w, y, o) (quant::axpy, quant.rs:1209-1226); then
// o = fma(sigmoid(g), y_shared, o); then out = o, or out += o (the residual
// add of model.rs:790).
struct CombineArgs {
    const float *y;
    Dispatch dp;
    const float *glogit;
    float *out;
    int T, P, k, E, has_shared, add;
};

// ---------------------------------------------------------------------------
// Grouped expert matvec.  blockIdx.y is a slot: first the shared expert's
// (its tokens in runs of XT, dispatched first as they are the longest-running
// workgroups when T is large), then the routed experts'.  A wave is four 16-lane groups; a group runs the 16
// chains of one (matrix, row): for gate/up, groups (row, gate) and (row, up)
// sit side by side and the SwiGLU is formed in registers; for down each group
// has its own row.  The weight row is loaded once and met by every token of
// the expert.
constexpr int MV_WAVES = 4;
#ifndef MV_NSET_LONG
#define MV_NSET_LONG 1
#endif
#ifndef MV_NSET_SHORT
#define MV_NSET_SHORT 2
#endif
constexpr int XT = 8; // activation rows staged in LDS at a time

// Each wave holds NSET sets of rows (four groups each), all loaded before the
// first token: more bytes in flight per wave.
// WPE: the waves per SIMD the register allocation must allow.
// The routing workgroup of a small-batch gate/up launch (T <= XT, slots of
// 64 pairs): the tokens' routes (route_token, a wave per token in turn) to
// dp.ids / dp.wts and the dispatch records that down + combine read
// (sort_pairs_small or sort_pairs_wave, as k_route_sort), in LDS scratch of
// ROUTE_SCRATCH bytes.
constexpr int ROUTE_SCRATCH = 1024 + 4 * 1024 + 512 + 2048 + 2048;
constexpr int GU_ROUTE_TMAX = 4; // tokens of the routing inside gate/up: a wave each
__device__ inline void route_records(const MvArgs &a, void *scratch)
{
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    char *sc = static_cast<char *>(scratch);
    uint64_t *tab = reinterpret_cast<uint64_t *>(sc) + 32 * wave;
    float *es = reinterpret_cast<float *>(sc + 1024) + MAX_EXPERTS * wave;
    int *ids = reinterpret_cast<int *>(sc + 1024 + 4 * 1024);
    float *wts = reinterpret_cast<float *>(ids + 64);
    int *cnt = reinterpret_cast<int *>(wts + 64), *first = cnt + 2 * MAX_EXPERTS, *sfirst = first + MAX_EXPERTS;
    if (lane < 32) tab[lane] = exp_tab_g[lane];
    wave_lds_sync();
    for (int t = wave; t < a.T; t += MV_WAVES) {
        float lg[RPER];
        load_logits(a.logits, a.n_expert, t, lg);
        route_token(lg, tab, a.n_expert, a.k, t, es, a.dp.ids, a.dp.wts, ids, wts);
    }
    __syncthreads();
    if (wave == 0) {
        const int P = a.T * a.k;
        if (P <= BIV_SMALL_SORT_P && P % 4 == 0) sort_pairs_small(ids, wts, a.k, a.T, a.dp, cnt);
        else sort_pairs_wave(ids, wts, a.n_expert, a.k, a.T, 64, a.dp, cnt, first, sfirst);
    }
}

template <int TY, int K, bool GATEUP, bool DUMP, int NSET, bool QX, int WPE, bool ROUTE = false>
__global__ __launch_bounds__(MV_WAVES *WAVE) __attribute__((amdgpu_waves_per_eu(WPE, 8))) void k_chain_mv(MvArgs a)
{
    static_assert(!ROUTE || (GATEUP && !QX), "the routing runs inside gate/up only");
    constexpr int S = K / 64;
    constexpr int RPW = GATEUP ? 2 : 4; // rows per set of a wave
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int grp = lane >> 4, ln = lane & 15, pi = ln >> 3, l = ln & 7;
    const int u = blockIdx.y;
    const bool shared = u < a.n_sh;
    int e = 0, beg, cnt, tok0 = 0;
    Slot sl;
    if (shared) {
        tok0 = u * a.sh_chunk; // the shared expert's tokens [tok0, tok0 + cnt)
        beg = a.P + tok0;
        cnt = min(a.sh_chunk, a.T - tok0);
    } else if constexpr (ROUTE) {
        // the slot's expert, first position and tokens come from the
        // routing below; meanwhile every token's row is staged (row t =
        // token t)
        beg = 0;
        cnt = a.T;
#pragma unroll
        for (int j = 0; j < SLOT_TOKS; j++) sl.tok[j] = j;
    } else {
        sl = a.dp.slots[u - a.n_sh];
        if (sl.cnt == 0) return; // uniform over the workgroup
        e = sl.expert;
        beg = sl.beg;
        cnt = sl.cnt;
    }
    const int m = GATEUP ? (grp & 1) : 0;
    // The group's matrix: the up matrix is addressed as the gate matrix plus
    // a uniform byte offset, so that each plane is one pointer in scalar
    // registers with a per-lane offset (a pointer chosen per lane would be
    // read from the kernel arguments with vector loads, before any weight).
    DevMat M = shared ? a.sa : a.a;
    if (GATEUP && m) {
        const DevMat &B = shared ? a.sb : a.b;
        M.q += B.q - M.q;
        M.s += B.s - M.s;
        M.d += B.d - M.d;
    }
    const int rows = M.rows;
    const int row0 = (blockIdx.x * MV_WAVES + wave) * RPW * NSET + (GATEUP ? grp >> 1 : grp);
    // The slot's activation rows, XC at a time, staged in LDS by the whole
    // workgroup (every group of every wave reads them from there), loaded
    // straight from global memory into LDS.  Staged row j is ROW16 16-byte
    // pieces: its K/16 quant pieces, then its K/128 scale pieces.  With QX
    // the rows come in as f32 (a.xf) and the workgroup quantises them itself
    // (Q8Act, as the standalone quantiser), XC of them in 16 KB.
    // BF16 matrices meet the f32 rows themselves (a.xf), XC of them in 16 KB.
    static_assert(!QX || (TY != T_Q4K && TY != T_BF16), "Q4_K needs the block sums of a separate quantisation");
    constexpr bool BF = TY == T_BF16, F32IN = QX || BF;
    constexpr int XC = F32IN ? (XT * 512 / K > 0 ? XT * 512 / K : 1) : XT;
    constexpr int ROW16 = K / 16 + K / 128;
    constexpr int NTH = MV_WAVES * WAVE;
    constexpr int NPC = F32IN ? XC * K / 4 / NTH : (XC * ROW16 + NTH - 1) / NTH; // pieces per thread
    constexpr int STAGE16 = BF ? 1 : (XC * ROW16 + NTH - 1) / NTH * NTH;
    constexpr int RS16 = ROUTE ? ROUTE_SCRATCH / 16 : 1;
    __shared__ int4 stage[STAGE16 > RS16 ? STAGE16 : RS16]; // also the routing workgroup's scratch
    __shared__ int s_tok[MV_WAVES][GU_ROUTE_TMAX]; // ROUTE: the slot's tokens (staged rows), a copy per wave
    __shared__ int4 fstage[F32IN ? NPC * NTH : 1];
    // (inline asm: the compiler does not track these DMAs, so its waits for
    // the weights do not cover them; the chunk loop waits for them itself)
    const unsigned stage_a = lds_addr(stage), fstage_a = lds_addr(fstage);
    auto lds_load = [&](const void *src, unsigned dst_wave) { lds_dma16_at(src, dst_wave); };
    // issue the loads of the nt rows of the chunk at i0 (row numbers of the
    // first chunk from the slot record: scalar loads, which do not wait on
    // vector loads); pieces past the chunk reread a valid row into unused LDS
    auto issue_chunk = [&](int i0, int nt) {
        // the input row of staged row j: gate/up reads its pair's token's
        // row (from the slot record for the first chunk), down the pair's own
        int trow[XC];
#pragma unroll
        for (int j = 0; j < XC; j++) {
            const int i = i0 + min(j, nt - 1);
            trow[j] = !GATEUP   ? beg + i
                      : shared  ? tok0 + i
                      : i0 == 0 ? (j < nt ? sl.tok[j] : sl.tok[0])
                                : a.dp.pair_tok[beg + i];
        }
        if constexpr (F32IN) {
#pragma unroll
            for (int c = 0; c < NPC; c++) {
                if (c * NTH >= nt * (K / 4)) break; // uniform
                const int idx0 = (int)threadIdx.x + c * NTH, idx = idx0 < nt * (K / 4) ? idx0 : nt * (K / 4) - 1;
                const int jr = idx / (K / 4);
                int xr = trow[0];
#pragma unroll
                for (int jj = 1; jj < XC; jj++) xr = jr == jj ? trow[jj] : xr;
                lds_load(a.xf + (size_t)xr * K + 4 * (idx - jr * (K / 4)), fstage_a + 16 * (c * NTH + wave * WAVE));
            }
        } else {
#pragma unroll
            for (int c = 0; c < NPC; c++) {
                if (c * NTH >= nt * ROW16) break; // uniform
                const int idx0 = (int)threadIdx.x + c * NTH, idx = idx0 < nt * ROW16 ? idx0 : nt * ROW16 - 1;
                const int jr = idx / ROW16, r = idx - jr * ROW16;
                int xr = trow[0];
#pragma unroll
                for (int jj = 1; jj < XC; jj++) xr = jr == jj ? trow[jj] : xr;
                // quant pieces, then scale pieces (16 bytes each)
                const uint8_t *src = r < K / 16 ? reinterpret_cast<const uint8_t *>(a.xq) + (size_t)xr * K + 16 * r
                                                : reinterpret_cast<const uint8_t *>(a.xd) + (size_t)xr * (K / 8) + 16 * (r - K / 16);
                lds_load(src, stage_a + 16 * (c * NTH + wave * WAVE));
            }
        }
    };
    // The first chunk's loads go out before the weights': loads complete in
    // order, so a gather issued after the weight loads would start only once
    // the weights are in.
    if constexpr (ROUTE) {
        // the row of workgroups past the slots: the routing workgroup's
        if (u >= a.n_sh + a.u_max) {
            if (blockIdx.x == 0) route_records(a, stage);
            return; // uniform over the workgroup
        }
    }
    issue_chunk(0, min(XC, cnt));
    if constexpr (ROUTE) {
        // The slot's record (route, model.rs:256-268, and the dispatch
        // order of model.rs:866-873), the same in every routed workgroup:
        // each token's expert set from its exps when they decide it
        // (route_set_masks, a wave per token in turn), else from its whole
        // routing (route_token, by wave 0); then slot us is the us-th expert
        // of their union in ascending id, its pairs follow those of the
        // lower experts, its tokens ascend (every expert holds at most T <=
        // 32 pairs: one slot each).  The logits and exp's table go out
        // behind the activation rows.  The routing workgroup
        // (route_records) writes the routes and dispatch records.
        __shared__ uint64_t rtab[MV_WAVES][32];
        __shared__ float res[MAX_EXPERTS];
        __shared__ int rids[TOPK_FAST];
        __shared__ float rwts[TOPK_FAST];
        __shared__ unsigned long long rmask[GU_ROUTE_TMAX][RPER];
        __shared__ int rok[GU_ROUTE_TMAX];
        if (!shared) { // uniform over the workgroup
            // a wave per token: exp's table, then its logits go out, then the
            // table's store to LDS (which waits only for the loads before it)
            const uint64_t tv = lane < 32 ? exp_tab_g[lane] : 0ull;
            float lg[RPER];
            if (wave < a.T) load_logits(a.logits, a.n_expert, wave, lg);
            if (lane < 32) rtab[wave][lane] = tv;
            wave_lds_sync();
            if (wave < a.T) {
                unsigned long long mk[RPER];
                const bool ok = route_set_masks(lg, rtab[wave], a.n_expert, a.k, mk);
                if (lane < RPER) {
                    unsigned long long mine = mk[0];
#pragma unroll
                    for (int j = 1; j < RPER; j++) mine = lane == j ? mk[j] : mine;
                    rmask[wave][lane] = mine;
                }
                if (lane == 0) rok[wave] = ok;
            }
            {
                __syncthreads();
                bool all_ok = true;
                for (int t = 0; t < a.T; t++) all_ok &= __builtin_amdgcn_readfirstlane(rok[t]) != 0;
                if (!all_ok) { // uniform, rare: the whole routing of the undecided tokens, by wave 0
                    if (wave == 0) {
                        for (int t = 0; t < a.T; t++) {
                            if (rok[t]) continue; // uniform
                            float lt[RPER];
                            load_logits(a.logits, a.n_expert, t, lt);
                            route_token(lt, rtab[0], a.n_expert, a.k, 0, res, nullptr, nullptr, rids, rwts);
                            wave_lds_sync();
#pragma unroll
                            for (int j = 0; j < RPER; j++) {
                                bool in = false;
                                for (int q = 0; q < a.k; q++) in |= rids[q] == lane + WAVE * j;
                                const unsigned long long mj = __ballot(in);
                                if (lane == 0) rmask[t][j] = mj;
                            }
                            wave_lds_sync();
                        }
                    }
                    __syncthreads();
                }
                // every wave: the slot from the masks (us-th expert of the
                // union; its pairs after those of the lower experts; its tokens)
                // (uniform values in vector registers: the scalar registers
                // are short here; e, beg and cnt move to them at the end)
                auto mask_at = [&](int t, int j) { return rmask[t][j]; };
                unsigned long long un[RPER];
#pragma unroll
                for (int j = 0; j < RPER; j++) un[j] = 0ull;
                for (int t = 0; t < a.T; t++) {
#pragma unroll
                    for (int j = 0; j < RPER; j++) un[j] |= mask_at(t, j);
                }
                int need = u - a.n_sh, ex = -1;
#pragma unroll
                for (int j = 0; j < RPER; j++) {
                    const int c = __popcll(un[j]);
                    if (ex < 0 && need < c) {
                        unsigned long long mm = un[j];
                        for (int q = 0; q < need; q++) mm &= mm - 1ull;
                        ex = WAVE * j + __ffsll((long long)mm) - 1;
                    } else if (ex < 0) {
                        need -= c;
                    }
                }
                if (__builtin_amdgcn_readfirstlane(ex) < 0) return; // an unused slot, uniform
                const int jw = ex >> 6;
                const unsigned long long lo = (1ull << (ex & 63)) - 1ull;
                int bg = 0;
                unsigned tm = 0u;
                for (int t = 0; t < a.T; t++) {
#pragma unroll
                    for (int j = 0; j < RPER; j++) {
                        if (j > jw) break;
                        const unsigned long long mm = mask_at(t, j);
                        bg += __popcll(j < jw ? mm : mm & lo);
                        if (j == jw) tm |= (unsigned)((mm >> (ex & 63)) & 1ull) << t;
                    }
                }
                e = __builtin_amdgcn_readfirstlane(ex);
                beg = __builtin_amdgcn_readfirstlane(bg);
                cnt = __builtin_amdgcn_readfirstlane(__popc(tm));
                if (lane < GU_ROUTE_TMAX) {
                    unsigned r = tm;
                    for (int q = 0; q < lane; q++) r &= r - 1u;
                    s_tok[wave][lane] = r ? __ffs(r) - 1 : 0;
                }
                wave_lds_sync();
            }
        }
    }
    Chain<TY, K> wc[NSET];
#pragma unroll
    for (int q = 0; q < NSET; q++) {
        const int row = row0 + q * RPW;
        wc[q].load(M, (size_t)e * rows + (row < rows ? row : 0), pi, l);
    }
    int32_t *dump = DUMP ? (m ? a.dump_b : a.dump_a) : nullptr;
    for (int i0 = 0; i0 < cnt; i0 += XC) {
        const int nt = min(XC, cnt - i0);
        if (i0 > 0) issue_chunk(i0, nt);
        // The chunk's rows are in once at most the loads issued after them
        // are outstanding (loads complete in order): for the first chunk the
        // weights' (so that the chains start while the later weights still
        // arrive), for the others none.  The waits are explicit: the DMAs
        // are inline asm, which the compiler's own waits (those of
        // __syncthreads included) do not count.
        __builtin_amdgcn_sched_barrier(0); // (the weights' loads stay above the wait)
        if (i0 == 0) wait_vm<NSET * Chain<TY, K>::NLOAD_MIN>();
        else wait_vm<0>();
        rm_barrier();
        if constexpr (QX) {
            // one thread per 32-element block of the chunk
            const int b = threadIdx.x;
            if (b < nt * (K / 32)) {
                const int jr = b / (K / 32), bb = b % (K / 32);
                quant_block_lds(reinterpret_cast<const float4 *>(&fstage[0]) + jr * (K / 4) + bb * 8, K, bb,
                                reinterpret_cast<int *>(&stage[jr * ROW16]),
                                reinterpret_cast<float *>(&stage[jr * ROW16 + K / 16]));
            }
            __syncthreads();
        }
        if constexpr (BF) {
            // BF16: f32 FMA chains over the staged f32 rows
            for (int j = 0; j < nt; j++) {
                const size_t orow = (size_t)(beg + i0 + j);
                const float *xr = reinterpret_cast<const float *>(&fstage[0]) + j * K;
#pragma unroll
                for (int q = 0; q < NSET; q++) {
                    const int row = row0 + q * RPW;
                    const bool row_ok = row < rows;
                    float acc = 0.0f;
#pragma unroll
                    for (int s = 0; s < K / 16; s++) acc = fmaf(wc[q].wval(s), xr[16 * s + ln], acc);
                    float t = row_tree16(acc); // valid in the group's first lane
                    if (GATEUP) {
                        const float up = from_lane_plus16(t); // (read by the gate groups' first lanes)
                        if (m == 0 && ln == 0 && row_ok) a.out[orow * rows + row] = silu_mul(t, up);
                    } else {
                        if (ln == 0 && row_ok) a.out[orow * rows + row] = t;
                    }
                }
            }
        } else {
        for (int j = 0; j < nt; j++) {
            const int i = i0 + j;
            // ROUTE: the pair's staged row is its token's
            const int sj = ROUTE && !shared ? s_tok[wave][j] : j;
            const size_t xrow = GATEUP ? (size_t)(shared ? tok0 + i : ROUTE ? sj : a.dp.pair_tok[beg + i]) : (size_t)(beg + i);
            const size_t orow = (size_t)(beg + i);
            int xw[S];
            float xd[S];
            const int4 *srow = stage + sj * ROW16;
#pragma unroll
            for (int q = 0; q < S / 4; q++) {
                const int4 v = srow[q * 16 + pi * 8 + l];
                xw[4 * q] = v.x;
                xw[4 * q + 1] = v.y;
                xw[4 * q + 2] = v.z;
                xw[4 * q + 3] = v.w;
                const float4 f = *reinterpret_cast<const float4 *>(&srow[K / 16 + pi * (S / 4) + q]);
                xd[4 * q] = f.x;
                xd[4 * q + 1] = f.y;
                xd[4 * q + 2] = f.z;
                xd[4 * q + 3] = f.w;
            }
#pragma unroll
            for (int q = 0; q < NSET; q++) {
                const int row = row0 + q * RPW;
                const bool row_ok = row < rows;
                float acc = 0.0f;
#pragma unroll
                for (int s = 0; s < S; s++) {
                    const int p = wc[q].partial(s, xw[s]);
                    acc = fmaf((float)p, wc[q].wscale(s) * xd[s], acc);
                    if (DUMP) {
                        // the block's int32 is the sum of its 8 lanes' partials
                        int bs = p;
                        bs += __shfl_xor(bs, 1);
                        bs += __shfl_xor(bs, 2);
                        bs += __shfl_xor(bs, 4);
                        if (dump && l == 0 && row_ok) dump[(orow * rows + row) * (K / 32) + 2 * s + pi] = bs;
                    }
                }
                float t = row_tree16(acc); // valid in the group's first lane
                if (TY == T_Q4K) t = t - q4k_mins_group<K>(M, (size_t)e * rows + (row_ok ? row : 0), a.xs, xrow, ln);
                if (GATEUP) {
                    const float up = from_lane_plus16(t); // (read by the gate groups' first lanes)
                    if (m == 0 && ln == 0 && row_ok) a.out[orow * rows + row] = silu_mul(t, up);
                } else {
                    if (ln == 0 && row_ok) a.out[orow * rows + row] = t;
                }
            }
        }
        }
        __syncthreads();
    }
}

// Q8Act of whole rows [rows][K] (the SwiGLU intermediate), one thread per block.
__global__ __launch_bounds__(256) void k_quant_rows(const float *__restrict__ x, int n_blocks, int K,
                                                    int8_t *__restrict__ qs, float *__restrict__ d,
                                                    float *__restrict__ s)
{
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n_blocks) return;
    float v[32];
    load32(x + 32 * (size_t)i, v);
    quant_block(v, K, i / (K / 32), i % (K / 32), qs, d, s);
}

// The combine as its own launch: grid (E / 256, T).
__global__ __launch_bounds__(256) void k_combine(CombineArgs a)
{
    const int t = blockIdx.y;
    const int c = blockIdx.x * blockDim.x + threadIdx.x;
    if (c >= a.E) return;
    float o = 0.0f;
    for (int j = 0; j < a.k; j++) {
        const int p = a.dp.tok_pairs[(size_t)t * a.k + j];
        o = fmaf(a.dp.pair_w[p], a.y[(size_t)p * a.E + c], o);
    }
    if (a.has_shared) o = fmaf(sigmoid(a.glogit[t]), a.y[(size_t)(a.P + t) * a.E + c], o);
    float *po = a.out + (size_t)t * a.E + c;
    *po = a.add ? *po + o : o;
}

// The same combine, four columns per thread and the k routes known at
// compile time, so that every load of a thread (the token's pair records,
// its k + 1 y rows, the residual) is issued before the first FMA: grid
// (E / 1024, T).  Each column runs the same FMA sequence as above.
template <int KK> __global__ __launch_bounds__(256) void k_combine4(CombineArgs a)
{
    const int t = blockIdx.y;
    const int c = 4 * (blockIdx.x * blockDim.x + threadIdx.x);
    if (c >= a.E) return;
    int p[KK];
    float w[KK];
    float4 y[KK];
#pragma unroll
    for (int j = 0; j < KK; j++) p[j] = a.dp.tok_pairs[(size_t)t * KK + j];
#pragma unroll
    for (int j = 0; j < KK; j++) {
        w[j] = a.dp.pair_w[p[j]];
        y[j] = *reinterpret_cast<const float4 *>(a.y + (size_t)p[j] * a.E + c);
    }
    float4 ys = make_float4(0.0f, 0.0f, 0.0f, 0.0f), r = ys;
    float g = 0.0f;
    if (a.has_shared) {
        ys = *reinterpret_cast<const float4 *>(a.y + (size_t)(a.P + t) * a.E + c);
        g = sigmoid(a.glogit[t]);
    }
    float4 *po = reinterpret_cast<float4 *>(a.out + (size_t)t * a.E + c);
    if (a.add) r = *po;
    float4 o = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
#pragma unroll
    for (int j = 0; j < KK; j++) {
        o.x = fmaf(w[j], y[j].x, o.x);
        o.y = fmaf(w[j], y[j].y, o.y);
        o.z = fmaf(w[j], y[j].z, o.z);
        o.w = fmaf(w[j], y[j].w, o.w);
    }
    if (a.has_shared) {
        o.x = fmaf(g, ys.x, o.x);
        o.y = fmaf(g, ys.y, o.y);
        o.z = fmaf(g, ys.z, o.z);
        o.w = fmaf(g, ys.w, o.w);
    }
    *po = a.add ? make_float4(r.x + o.x, r.y + o.y, r.z + o.z, r.w + o.w) : o;
}

// ---------------------------------------------------------------------------
// Down and combine in one launch, for decode sizes (every expert's pairs in
// one slot).  A workgroup owns RB output rows and computes them for every
// routed expert and the shared expert, so that it holds all of a token's y
// values for those rows and can combine them itself, in the reference's
// order (model.rs:884-896): o = 0, o = fma(w, y, o) over the token's
// experts in ascending id, then o = fma(sigmoid(g), y_shared, o).
//
// The workgroup first quantises the whole SwiGLU intermediate into LDS
// (Q8Act, as the standalone quantiser, R = P + T rows), then its 16-lane
// groups walk the (slot, row) units of its rows, each with the 16 chains of
// biv's x86 dot, D units of weight rows in flight per group.
constexpr int DC_RB = 8;    // output rows per workgroup
#ifndef BIV_DC_WAVES
#define BIV_DC_WAVES 16
#endif
#ifndef BIV_DC_DEPTH
#define BIV_DC_DEPTH 2
#endif
constexpr int DC_WAVES = BIV_DC_WAVES; // waves per workgroup
// weight rows in flight per group (at K = 512; fewer for longer rows)
template <int K> constexpr int dc_depth() { return K <= 512 ? BIV_DC_DEPTH : K <= 1024 ? (BIV_DC_DEPTH + 1) / 2 : 1; }

struct DcArgs {
    DevMat a, sa;        // routed down stack, the shared expert's down (sa.q == nullptr without one)
    const float *xf;     // the f32 intermediate [P + T][K]
    Dispatch dp;
    const float *glogit; // [T]
    float *out;          // [T][rows]
    int32_t *dump;       // optional [P + T][rows][K/32] block int32 dots
    int T, P, k, add;
    int u_max;           // slot records the sort wrote (dp.slot_cap)
};

template <int TY, int K, bool DUMP>
__global__ __launch_bounds__(DC_WAVES *WAVE) void k_down_combine(DcArgs a)
{
    constexpr int S = K / 64;
    constexpr int ROW16 = K / 16 + K / 128; // 16-byte pieces of a staged Q8 row
    constexpr int NG = DC_WAVES * 4;        // 16-lane groups
    constexpr int NTH = DC_WAVES * WAVE;
    extern __shared__ int4 dyn[];
    const int tid = threadIdx.x, lane = tid & 63;
    const int grp = tid >> 4, ln = lane & 15, pi = ln >> 3, l = ln & 7;
    const int T = a.T, P = a.P, k = a.k;
    const bool has_shared = a.sa.q != nullptr;
    const int R = has_shared ? P + T : P;
    const int rows = a.a.rows;
    const int row0 = blockIdx.x * DC_RB;
    int4 *stage = dyn;                                                // [R][ROW16]
    float *ylds = reinterpret_cast<float *>(dyn + (size_t)R * ROW16); // [R][DC_RB]
    int4 *slots = reinterpret_cast<int4 *>(ylds + (size_t)R * DC_RB); // [u_max + 1] {expert, beg, cnt, -}
    __shared__ int n_used;
    // slot heads (records with cnt 0 follow the used ones), the shared
    // expert as the last slot
    if (tid == 0) n_used = a.u_max;
    __syncthreads();
    for (int i = tid; i < a.u_max; i += NTH) {
        const int4 h = *reinterpret_cast<const int4 *>(&a.dp.slots[i]);
        slots[i] = h;
        if (h.z == 0) atomicMin(&n_used, i);
    }
    __syncthreads();
    const int U = n_used;
    if (has_shared && tid == 0) slots[U] = make_int4(-1, P, T, 0);
    __syncthreads();
    const int nsl = U + (has_shared ? 1 : 0);
    const int nunits = nsl * DC_RB;
    const int per = (nunits + NG - 1) / NG; // units per group, uniform
    // the matrix and row of unit v (a valid row past the last unit)
    auto unit_row = [&](int v, int &slot, int &r) {
        const int vv = v < nunits ? v : 0;
        slot = vv / DC_RB;
        r = row0 + vv % DC_RB;
    };
    auto load_unit = [&](Chain<TY, K> &c, int v) {
        int slot, r;
        unit_row(v, slot, r);
        const int4 h = slots[slot];
        const bool sh = h.x < 0;
        c.load(sh ? a.sa : a.a, (size_t)(sh ? 0 : h.x) * rows + r, pi, l);
    };
    // the thread's first block of the intermediate goes out first, then the
    // first weight rows: loads complete in order, so the block's
    // quantisation runs while the weights are still arriving
    const int nblk = R * (K / 32);
    float v0[32];
    if (tid < nblk) load32(a.xf + (size_t)(tid / (K / 32)) * K + 32 * (tid % (K / 32)), v0);
    constexpr int DC_D = dc_depth<K>();
    Chain<TY, K> wc[DC_D];
#pragma unroll
    for (int d = 0; d < DC_D; d++) load_unit(wc[d], grp + d * NG);
    // the combine's operands, fetched now so that none is a dependent load
    // at the end: the tokens' dispatch positions (their weights once the
    // staging is done), the shared-expert logits, the residual, exp's table
    __shared__ uint64_t tab[32];
    __shared__ int cpos[16 * 16];
    __shared__ float cwt[16 * 16], csig[16];
    const int nc = T * k; // <= 256: T <= 16, k <= 16
    const int cp = tid < nc ? a.dp.tok_pairs[tid] : 0;
    const float cg = has_shared && tid < T ? a.glogit[tid] : 0.0f;
    const int ct = tid / DC_RB, cr = tid - ct * DC_RB;
    const bool cmine = tid < T * DC_RB;
    float *const cpo = a.out + (size_t)ct * rows + row0 + cr;
    const float cres = a.add && cmine ? *cpo : 0.0f;
    const uint64_t tv = tid < 32 ? exp_tab_g[tid] : 0ull; // into LDS at the end (a store now would wait for it)
    // the intermediate, quantised into LDS: one 32-element block per thread and turn
    if (tid < nblk)
        quant_block_at(v0, K, tid % (K / 32), reinterpret_cast<int *>(&stage[(tid / (K / 32)) * ROW16]),
                       reinterpret_cast<float *>(&stage[(tid / (K / 32)) * ROW16 + K / 16]), nullptr);
    for (int b = tid + NTH; b < nblk; b += NTH) {
        const int r = b / (K / 32), bb = b - r * (K / 32);
        float v[32];
        load32(a.xf + (size_t)r * K + 32 * bb, v);
        quant_block_at(v, K, bb, reinterpret_cast<int *>(&stage[r * ROW16]),
                       reinterpret_cast<float *>(&stage[r * ROW16 + K / 16]), nullptr);
    }
    // the quantised rows are in LDS once this thread's writes are done: a
    // bare barrier after them, which leaves the weights in flight alone
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    rm_barrier();
    const float cw = tid < nc ? a.dp.pair_w[cp] : 0.0f; // consumed after the rows
    for (int i0 = 0; i0 < per; i0 += DC_D) {
#pragma unroll
        for (int d = 0; d < DC_D; d++) {
            const int v = grp + (i0 + d) * NG;
            if (v < nunits) {
                int slot, r;
                unit_row(v, slot, r);
                const int4 h = slots[slot];
                for (int j = 0; j < h.z; j++) {
                    const int orow = h.y + j;
                    float acc = 0.0f;
#pragma unroll
                    for (int q = 0; q < S / 4; q++) {
                        const int4 xv = stage[orow * ROW16 + q * 16 + pi * 8 + l];
                        const float4 xd = *reinterpret_cast<const float4 *>(&stage[orow * ROW16 + K / 16 + pi * (S / 4) + q]);
                        const int xw[4] = {xv.x, xv.y, xv.z, xv.w};
                        const float xs[4] = {xd.x, xd.y, xd.z, xd.w};
#pragma unroll
                        for (int c = 0; c < 4; c++) {
                            const int s = 4 * q + c;
                            const int p = wc[d].partial(s, xw[c]);
                            acc = fmaf((float)p, wc[d].wscale(s) * xs[c], acc);
                            if (DUMP) {
                                int bs = p;
                                bs += __shfl_xor(bs, 1);
                                bs += __shfl_xor(bs, 2);
                                bs += __shfl_xor(bs, 4);
                                if (l == 0) a.dump[((size_t)orow * rows + r) * (K / 32) + 2 * s + pi] = bs;
                            }
                        }
                    }
                    float t = row_tree16(acc); // valid in the group's first lane
                    if (ln == 0) ylds[orow * DC_RB + (r - row0)] = t;
                }
            }
            load_unit(wc[d], v + DC_D * NG);
        }
    }
    if (tid < nc) {
        cpos[tid] = cp;
        cwt[tid] = cw;
    }
    if (tid < 32) tab[tid] = tv; // wave 0, which alone reads it
    wave_lds_sync();
    if (has_shared && tid < T) csig[tid] = 1.0f / (1.0f + exp_lds(-cg, tab)); // ops::sigmoid
    __syncthreads();
    // the combine of this workgroup's rows: fma(w, y, o) over the token's
    // experts in ascending id, then the gated shared row (axpy, model.rs:880-895)
    if (cmine) {
        float o = 0.0f;
        for (int j = 0; j < k; j++) {
            const int p = cpos[ct * k + j];
            o = fmaf(cwt[ct * k + j], ylds[p * DC_RB + cr], o);
        }
        if (has_shared) o = fmaf(csig[ct], ylds[(P + ct) * DC_RB + cr], o);
        *cpo = a.add ? cres + o : o;
    }
}

template <int TY, int KK, bool GATEUP, bool DUMP, bool QX>
hipError_t launch_case(const MvArgs &a, int rows, int slots, hipStream_t st)
{
    if constexpr (QX && (TY == T_Q4K || TY == T_BF16)) {
        return hipErrorInvalidValue; // Q4_K takes the separately quantised rows (with block sums), BF16 the f32 rows
    } else if constexpr (DUMP && TY == T_BF16) {
        return launch_case<TY, KK, GATEUP, false, QX>(a, rows, slots, st); // no integer dots to tap
    } else {
        // row sets per wave: the shorter the rows, the more of them in flight
        constexpr int NSET = KK >= 2048 ? MV_NSET_LONG : MV_NSET_SHORT;
        const int rows_per_wg = MV_WAVES * (GATEUP ? 2 : 4) * NSET;
        dim3 grid((rows + rows_per_wg - 1) / rows_per_wg, slots);
        // occupancy asked of the register allocator (Q8_0 only: the K-quant
        // chains need more registers than 4 waves per SIMD leave)
        constexpr int WPE = TY != T_Q8_0 || DUMP ? 1 : KK >= 2048 && !QX ? 5 : 4;
        if (GATEUP && !DUMP && !QX && a.logits)
            k_chain_mv<TY, KK, GATEUP, false, NSET, false, WPE, GATEUP && !DUMP && !QX>
                <<<dim3(grid.x, grid.y + 1), MV_WAVES * WAVE, 0, st>>>(a); // + the routing workgroup's row
        else k_chain_mv<TY, KK, GATEUP, DUMP, NSET, QX, WPE><<<grid, MV_WAVES * WAVE, 0, st>>>(a);
        return hipGetLastError();
    }
}

// One launch over the routed slots (routed = 1) and/or the shared expert.
template <bool GATEUP, bool DUMP, bool QX>
hipError_t launch_mv_t(MvArgs a, int routed, int shared, hipStream_t st)
{
    const DevMat &M = routed ? a.a : a.sa;
    if (!routed) {
        a.u_max = 0;
        a.logits = nullptr; // the routed launch routes
    }
    a.sh_chunk = XT;
    a.n_sh = shared ? (a.T + XT - 1) / XT : 0;
    const int slots = a.u_max + a.n_sh;
    if (slots == 0) return hipSuccess;
#define BIV_MV_CASE(TY, KK)                                                                                     \
    if (M.ty == TY && M.cols == KK) return launch_case<TY, KK, GATEUP, DUMP, QX>(a, M.rows, slots, st);
    BIV_MV_CASE(T_Q8_0, 2048)
    BIV_MV_CASE(T_Q8_0, 1024)
    BIV_MV_CASE(T_Q8_0, 512)
    BIV_MV_CASE(T_Q4K, 2048)
    BIV_MV_CASE(T_Q4K, 1024)
    BIV_MV_CASE(T_Q4K, 512)
    BIV_MV_CASE(T_Q6K, 2048)
    BIV_MV_CASE(T_Q6K, 1024)
    BIV_MV_CASE(T_Q6K, 512)
    BIV_MV_CASE(T_BF16, 2048)
    BIV_MV_CASE(T_BF16, 1024)
    BIV_MV_CASE(T_BF16, 512)
#undef BIV_MV_CASE
    return hipErrorInvalidValue;
}

template <bool GATEUP, bool QX>
hipError_t launch_mv_q(const MvArgs &a, int routed, int shared, hipStream_t st)
{
    const bool dump = a.dump_a || a.dump_b;
    return dump ? launch_mv_t<GATEUP, true, QX>(a, routed, shared, st) : launch_mv_t<GATEUP, false, QX>(a, routed, shared, st);
}

template <bool GATEUP>
hipError_t launch_mv(const MvArgs &a, hipStream_t st)
{
    auto go = [&](int routed, int shared) {
        return !GATEUP && a.qx ? launch_mv_q<GATEUP, !GATEUP>(a, routed, shared, st)
                               : launch_mv_q<GATEUP, false>(a, routed, shared, st);
    };
    const bool has_shared = a.sa.q != nullptr;
    // routing inside gate/up: one token, k <= 8 distinct experts in k slots
    // (sort_pairs_small takes the pairs four at a time)
    // routing inside gate/up: up to GU_ROUTE_TMAX tokens (a wave each, all
    // staged at once; f32-input BF16 rows for one token only), k <= 8, one
    // slot per used expert
    if (a.logits && (!GATEUP || a.T > GU_ROUTE_TMAX || (a.T > 1 && a.a.ty == T_BF16) || a.k > TOPK_FAST ||
                     a.n_expert < a.k || a.n_expert > MAX_EXPERTS || a.u_max != max_slots(a.n_expert, a.P, 64)))
        return hipErrorInvalidValue;
    // routed and shared in one launch when they share types and shape
    const bool together = has_shared && a.sa.ty == a.a.ty && a.sa.cols == a.a.cols && a.sa.rows == a.a.rows &&
                          (!GATEUP || a.sb.ty == a.b.ty);
    if (together) return go(1, 1);
    hipError_t err = go(1, 0);
    if (err != hipSuccess || !has_shared) return err;
    return go(0, 1);
}

} // namespace

hipError_t launch_rms_norm(const float *x, float *y, const float *w, int rows, int n, float eps, hipStream_t st)
{
    if (rows <= 0) return hipSuccess;
    if (n == 2048) k_rms_norm<64><<<(rows + 7) / 8, 256, 0, st>>>(x, y, w, rows, n, eps);
    else k_rms_norm<0><<<(rows + 7) / 8, 256, 0, st>>>(x, y, w, rows, n, eps);
    return hipGetLastError();
}

// threads of a router workgroup for a single token (two rows each)
#ifndef BIV_ROUTER_T1_NTH
#define BIV_ROUTER_T1_NTH 64
#endif
int prep_min_t() { return RT_MIN_T; }

hipError_t launch_router(const RouterArgs &a0, hipStream_t st)
{
    RouterArgs a = a0;
    if (a.T >= RT_MIN_T && a.E % 128 == 0 && a.router_rm && (!a.gate_inp || a.gate_rm)) {
        // the pre-pass (norm into hn, gate logit, Q8 of h), then the logits of
        // the (normalised) rows in tiles of 16 x 32 (row x token), 32 x 32 or
        // 32 x 64: the largest that still gives the chip a few hundred workgroups
        const int nb = (a.T + PREP_TOK - 1) / PREP_TOK;
        if (a.E == 2048) k_prep<64><<<nb, 64 * PREP_TOK, 0, st>>>(a);
        else if (a.E == 1024) k_prep<32><<<nb, 64 * PREP_TOK, 0, st>>>(a);
        else if (a.E == 512) k_prep<16><<<nb, 64 * PREP_TOK, 0, st>>>(a);
        else return hipErrorInvalidValue;
        if (a.norm_w) a.h = a.hn;
#define BIV_RM_LAUNCH(SH, MI)                                                                              \
    do {                                                                                                   \
        const int n_tr = (a.n_expert + SH - 1) / SH, n_tt = (a.T + rm_tokens<SH, MI>() - 1) / rm_tokens<SH, MI>(); \
        k_router_mfma<SH, MI><<<n_tr * n_tt, RM_NTH, 0, st>>>(a, n_tr, n_tt);                             \
    } while (0)
        if (a.T >= BIV_RM_L_T) BIV_RM_LAUNCH(32, 4);
        else if (a.T >= BIV_RM_M_T) BIV_RM_LAUNCH(32, 2);
        else BIV_RM_LAUNCH(16, 2);
#undef BIV_RM_LAUNCH
        return hipGetLastError();
    }
    const int rows = a.n_expert + 1;
    // quantisation workgroups beside the row groups: about one block per thread
    const int qblocks = a.xq || a.norm_w ? a.T * (a.E / 32) : 0;
    // 8 rows per workgroup; tokens split over grid.y in chunks of TC (32 KB of
    // LDS, 64 KB past 2 TC tokens); batches of 2..64 tokens in chunks of TC / 4
    // (up to 16 tokens) or TC / 2: more workgroups, shorter chains each
#define BIV_ROUTER_CASE(NS)                                                                                     \
    if (a.E == 32 * NS) {                                                                                       \
        constexpr int TC = 8192 / (32 * NS);                                                                    \
        if (a.T > 1 && a.T <= 64) {                                                                             \
            /* small batches: one or two tokens per workgroup, more workgroups */                               \
            constexpr int TS1 = TC / 4 > 0 ? TC / 4 : 1, TS2 = TC / 2 > 0 ? TC / 2 : 1;                         \
            const int ts = a.T <= 16 ? TS1 : TS2, gy = (a.T + ts - 1) / ts;                                     \
            const dim3 grid((rows + 7) / 8 + (qblocks + 256 * gy - 1) / (256 * gy), gy);                        \
            if (ts == TS1) k_router<NS, TS1><<<grid, 256, 0, st>>>(a);                                          \
            else k_router<NS, TS2><<<grid, 256, 0, st>>>(a);                                                    \
        } else if (a.T == 1 && BIV_ROUTER_T1_NTH != 256) {                                                      \
            constexpr int N1 = BIV_ROUTER_T1_NTH;                                                               \
            k_router<NS, TC, N1><<<dim3((rows + N1 / 32 - 1) / (N1 / 32) + (qblocks + N1 - 1) / N1, 1), N1, 0, st>>>(a); \
        } else if (a.T <= 2 * TC) {                                                                             \
            const int gy = (a.T + TC - 1) / TC;                                                                 \
            k_router<NS, TC><<<dim3((rows + 7) / 8 + (qblocks + 256 * gy - 1) / (256 * gy), gy), 256, 0, st>>>(a); \
        } else {                                                                                                \
            const int gy = (a.T + 2 * TC - 1) / (2 * TC);                                                       \
            k_router<NS, 2 * TC><<<dim3((rows + 7) / 8 + (qblocks + 256 * gy - 1) / (256 * gy), gy), 256, 0, st>>>(a); \
        }                                                                                                       \
        return hipGetLastError();                                                                               \
    }
    BIV_ROUTER_CASE(64)
    BIV_ROUTER_CASE(32)
    BIV_ROUTER_CASE(16)
#undef BIV_ROUTER_CASE
    return hipErrorInvalidValue;
}

hipError_t launch_route_sort(const float *logits, int n_expert, int k, int T, int chunk, const Dispatch &dp,
                             int *work, hipStream_t st)
{
    // a single workgroup routes and sorts in LDS while every token has its wavefront
    const int groups = T <= RS_WAVES ? 1 : (T + RS_WAVES - 1) / RS_WAVES;
    const int threads = groups == 1 ? WAVE * T : RS_THREADS; // a wavefront per token
    k_route_sort<<<groups, threads, 0, st>>>(logits, n_expert, k, T, chunk, dp, work);
    if (groups > 1 && groups <= DP_FUSE_NB) {
        k_dispatch_place<true><<<groups, MAX_EXPERTS, 0, st>>>(n_expert, k, T, groups, chunk, dp, work);
    } else if (groups > 1) {
        k_dispatch_scan<<<1, MAX_EXPERTS * DS_SPLIT, 0, st>>>(n_expert, groups, chunk, dp, work);
        k_dispatch_place<false><<<groups, MAX_EXPERTS, 0, st>>>(n_expert, k, T, groups, chunk, dp, work);
    }
    return hipGetLastError();
}

hipError_t launch_quant_rows(const float *x, int n_blocks, int K, int8_t *qs, float *d, float *s, hipStream_t st)
{
    if (n_blocks <= 0) return hipSuccess;
    k_quant_rows<<<(n_blocks + 255) / 256, 256, 0, st>>>(x, n_blocks, K, qs, d, s);
    return hipGetLastError();
}

hipError_t launch_combine(const float *y, const Dispatch &dp, const float *glogit, int has_shared, int T, int P, int k,
                          int E, float *out, int add, hipStream_t st)
{
    CombineArgs c{y, dp, glogit, out, T, P, k, E, has_shared, add};
    if (k == 8 && E % 4 == 0 && (reinterpret_cast<uintptr_t>(out) & 15) == 0) {
        k_combine4<8><<<dim3((E + 1023) / 1024, T), 256, 0, st>>>(c);
        return hipGetLastError();
    }
    dim3 grid((E + 255) / 256, T);
    k_combine<<<grid, 256, 0, st>>>(c);
    return hipGetLastError();
}

size_t down_combine_lds(int R, int K, int u_max)
{
    return (size_t)R * (K / 16 + K / 128) * 16 + (size_t)R * DC_RB * 4 + (size_t)(u_max + 1) * 16;
}

hipError_t launch_down_combine(const DownCombineArgs &x, hipStream_t st)
{
    DcArgs a{x.a, x.sa, x.xf, x.dp, x.glogit, x.out, x.dump, x.T, x.P, x.k, x.add, x.dp.slot_cap};
    const int K = a.a.cols, rows = a.a.rows;
    if (rows % DC_RB || (a.sa.q && (a.sa.ty != a.a.ty || a.sa.cols != K || a.sa.rows != rows)))
        return hipErrorInvalidValue;
    const int R = a.sa.q ? a.P + a.T : a.P;
    const size_t lds = down_combine_lds(R, K, a.u_max);
    const bool dump = a.dump != nullptr;
#define BIV_DC_CASE(TY, KK)                                                                                     \
    if (a.a.ty == TY && K == KK) {                                                                              \
        auto fn = dump ? k_down_combine<TY, KK, true> : k_down_combine<TY, KK, false>;                          \
        if (lds > 65536) {                                                                                      \
            hipError_t e = hipFuncSetAttribute((const void *)fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds); \
            if (e != hipSuccess) return e;                                                                      \
        }                                                                                                       \
        fn<<<rows / DC_RB, DC_WAVES * WAVE, lds, st>>>(a);                                                      \
        return hipGetLastError();                                                                               \
    }
    BIV_DC_CASE(T_Q8_0, 512)
    BIV_DC_CASE(T_Q8_0, 1024)
    BIV_DC_CASE(T_Q8_0, 2048)
    BIV_DC_CASE(T_Q6K, 512)
    BIV_DC_CASE(T_Q6K, 1024)
    BIV_DC_CASE(T_Q6K, 2048)
#undef BIV_DC_CASE
    return hipErrorInvalidValue;
}

#ifndef BIV_LONG_WV_GU
#define BIV_LONG_WV_GU 4
#endif
#ifndef BIV_LONG_WV_DN
#define BIV_LONG_WV_DN 4
#endif

template <int TY, bool GATEUP, int XTT>
hipError_t launch_long_t(const LongArgs &a, bool full, size_t full_lds, hipStream_t st)
{
    // waves per workgroup; rows per workgroup: 2 (gate/up) or 4 (down) per wave
    constexpr int WV = GATEUP ? BIV_LONG_WV_GU : BIV_LONG_WV_DN;
    constexpr int per_wg = WV * (GATEUP ? 2 : 4);
    dim3 grid((a.a.rows + per_wg - 1) / per_wg, (a.T + XTT - 1) / XTT);
    if (full) {
        auto fn = k_chain_mv_long_full<TY, GATEUP, XTT, WV>;
        if (full_lds > 65536) {
            hipError_t e = hipFuncSetAttribute((const void *)fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)full_lds);
            if (e != hipSuccess) return e;
        }
        fn<<<grid, WV * WAVE, full_lds, st>>>(a);
    } else {
        k_chain_mv_long<TY, GATEUP, XTT, WV><<<grid, WV * WAVE, 0, st>>>(a);
    }
    return hipGetLastError();
}

template <int TY, bool GATEUP>
hipError_t launch_long_x(const LongArgs &a, hipStream_t st)
{
    // tokens per workgroup: as few accumulators as the batch needs
    const int xt = a.T <= 1 ? 1 : a.T <= 2 ? 2 : a.T <= 4 ? 4 : a.T == 5 ? 5 : LXT;
    // every chunk of a workgroup's rows in LDS when that fits (the weights
    // then stream LPD chunks ahead), else two chunks at a time
    const size_t piece_row = TY == T_BF16 ? LK / 4 : LK / 16 + LK / 128;
    const size_t full_lds = (size_t)(a.K / LK) * xt * piece_row * 16;
    const bool full = full_lds <= LONG_FULL_LDS;
    switch (xt) {
    case 1: return launch_long_t<TY, GATEUP, 1>(a, full, full_lds, st);
    case 2: return launch_long_t<TY, GATEUP, 2>(a, full, full_lds, st);
    case 4: return launch_long_t<TY, GATEUP, 4>(a, full, full_lds, st);
    case 5: return launch_long_t<TY, GATEUP, 5>(a, full, full_lds, st);
    default: return launch_long_t<TY, GATEUP, LXT>(a, full, full_lds, st);
    }
}

hipError_t launch_long_mv(const LongArgs &a, int gateup, hipStream_t st)
{
    if (a.T <= 0) return hipSuccess;
    if (a.K % LK || a.a.cols != a.K || (gateup && (a.b.ty != a.a.ty || a.b.cols != a.K || a.b.rows != a.a.rows)))
        return hipErrorInvalidValue;
#define BIV_LONG_CASE(TY)                                                                                       \
    if (a.a.ty == TY) return gateup ? launch_long_x<TY, true>(a, st) : launch_long_x<TY, false>(a, st);
    BIV_LONG_CASE(T_Q8_0)
    BIV_LONG_CASE(T_Q4K)
    BIV_LONG_CASE(T_Q6K)
    BIV_LONG_CASE(T_BF16)
#undef BIV_LONG_CASE
    return hipErrorInvalidValue;
}

hipError_t launch_gateup(const MvArgs &a, hipStream_t st) { return launch_mv<true>(a, st); }

hipError_t launch_down(const MvArgs &a, hipStream_t st) { return launch_mv<false>(a, st); }

} // namespace biv
