// gfx950 kernels of the qwen35moe MoE block: activation quantiser, router,
// route, dispatch sort, grouped expert matvecs and the fixed-order combine.
//
// Numerics follow biv's CPU path (engine/src/quant.rs, ops.rs, model.rs):
// activations are quantised to int8 blocks of 32 with an f32 scale exactly as
// Q8Act::quantize_into does, every weight block meets its activation block as
// one int32 dot, and that int32 is scaled in f32.  Nothing here uses a
// floating-point atomic, so a forward is bit-identical from run to run.
#include "common.hpp"

#include <hip/hip_fp16.h>

namespace biv {

namespace {

constexpr int WAVE = 64;

__device__ inline float f16_at(const uint8_t *p)
{
    return __half2float(*reinterpret_cast<const __half *>(p));
}

__device__ inline int dot4(int a, int b, int c) { return __builtin_amdgcn_sdot4(a, b, c, false); }

// e^x rounded once from double: the nearest float, which is what glibc's
// expf (the f32::exp of the reference on Linux) returns
__device__ inline float exp_f32(float x) { return (float)exp((double)x); }

// byte i (0..15) of a 16-byte vector, without indexing a private array
__device__ inline int byte_at(const int4 &v, int i)
{
    const int w = i < 4 ? v.x : i < 8 ? v.y : i < 12 ? v.z : v.w;
    return ((unsigned)w >> (8 * (i & 3))) & 0xFF;
}

// ---------------------------------------------------------------------------
// Q8Act::quantize_into (quant.rs:368-394), one thread per 32-element block:
// amax, d = amax / 127, id = 1/d (0 when d is 0), q = round-half-away(v * id),
// s = d * sum(q).  IEEE division and no contraction keep it bit-exact.
__global__ __launch_bounds__(256) void k_quant_rows(const float *__restrict__ x, int n_blocks,
                                                    int8_t *__restrict__ qs, float *__restrict__ d,
                                                    float *__restrict__ s)
{
    int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n_blocks) return;
    const float4 *xb = reinterpret_cast<const float4 *>(x + 32 * (size_t)i);
    float v[32];
#pragma unroll
    for (int j = 0; j < 8; j++) {
        float4 f = xb[j];
        v[4 * j] = f.x;
        v[4 * j + 1] = f.y;
        v[4 * j + 2] = f.z;
        v[4 * j + 3] = f.w;
    }
    float amax = 0.0f;
#pragma unroll
    for (int j = 0; j < 32; j++) amax = fmaxf(amax, fabsf(v[j]));
    float db = amax / 127.0f;
    float id = db != 0.0f ? 1.0f / db : 0.0f;
    int sum = 0;
    int packed[8];
#pragma unroll
    for (int j = 0; j < 8; j++) {
        unsigned w = 0;
#pragma unroll
        for (int b = 0; b < 4; b++) {
            int r = (int)roundf(v[4 * j + b] * id);
            sum += r;
            w |= (unsigned)(r & 0xFF) << (8 * b);
        }
        packed[j] = (int)w;
    }
    int4 *qo = reinterpret_cast<int4 *>(qs + 32 * (size_t)i);
    qo[0] = make_int4(packed[0], packed[1], packed[2], packed[3]);
    qo[1] = make_int4(packed[4], packed[5], packed[6], packed[7]);
    d[i] = db;
    s[i] = db * (float)sum;
}

// ---------------------------------------------------------------------------
// Router logits in the accumulation order of biv's AVX2 dot_f32
// (quant.rs:1177-1207): 32 running FMA sums, sum L over elements L, L+32, ...,
// combined by the tree of `hsum((a0+a1)+(a2+a3))` (quant.rs:1149-1153).
// 32 lanes per weight row, lane L owns running sum L, so a row's logits are
// those the reference computes, bit for bit.  Row n_expert is gate_inp (the
// shared expert's gate, model.rs:892).
template <int TC>
__global__ __launch_bounds__(256) void k_router(const float *__restrict__ router, const float *__restrict__ gate_inp,
                                                int n_expert, int E, const float *__restrict__ h, int T,
                                                float *__restrict__ logits, float *__restrict__ glogit)
{
    const int L = threadIdx.x & 31;
    const int row = blockIdx.x * (blockDim.x / 32) + (threadIdx.x >> 5);
    const int t0 = blockIdx.y * TC;
    const bool valid = row < n_expert || (row == n_expert && gate_inp != nullptr);
    const float *w = row < n_expert ? router + (size_t)row * E : gate_inp;
    float acc[TC];
#pragma unroll
    for (int t = 0; t < TC; t++) acc[t] = 0.0f;
    if (valid) {
#pragma unroll 8
        for (int m = 0; m < E / 32; m++) {
            float wv = w[L + 32 * m];
#pragma unroll
            for (int t = 0; t < TC; t++)
                if (t0 + t < T) acc[t] = fmaf(wv, h[(size_t)(t0 + t) * E + L + 32 * m], acc[t]);
        }
    }
#pragma unroll
    for (int t = 0; t < TC; t++) {
        float v = acc[t];
        v = v + __shfl_xor(v, 8);  // acc0+acc1 (lanes 0-7), acc2+acc3 (16-23)
        v = v + __shfl_xor(v, 16); // (acc0+acc1)+(acc2+acc3)
        v = v + __shfl_xor(v, 4);  // low half + high half of the 8 lanes
        v = v + __shfl_xor(v, 2);  // movehl
        v = v + __shfl_xor(v, 1);  // movehdup
        if (valid && L == 0 && t0 + t < T) {
            if (row < n_expert) logits[(size_t)(t0 + t) * n_expert + row] = v;
            else glogit[t0 + t] = v;
        }
    }
}

// ---------------------------------------------------------------------------
// route (model.rs:256-268): softmax over the token's logits (ops.rs:192-201),
// the k highest probabilities with the lower expert first among equals, and
// weights p / max(sum of the k in rank order, 1/16384).  One wavefront per
// token, up to 8 logits per lane.
__device__ inline bool better(float pa, int ia, float pb, int ib) { return pa > pb || (pa == pb && ia < ib); }

__global__ __launch_bounds__(256) void k_route(const float *__restrict__ logits, int n_expert, int k, int T,
                                               int *__restrict__ ids, float *__restrict__ wts)
{
    const int lane = threadIdx.x & 63;
    const int t = blockIdx.x * (blockDim.x / WAVE) + (threadIdx.x >> 6);
    if (t >= T) return;
    constexpr int PER = 8;
    float v[PER];
    float mx = -INFINITY;
#pragma unroll
    for (int j = 0; j < PER; j++) {
        int i = lane + WAVE * j;
        v[j] = i < n_expert ? logits[(size_t)t * n_expert + i] : -INFINITY;
        mx = fmaxf(mx, v[j]);
    }
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) mx = fmaxf(mx, __shfl_xor(mx, m));
    float sum = 0.0f;
#pragma unroll
    for (int j = 0; j < PER; j++) {
        int i = lane + WAVE * j;
        v[j] = i < n_expert ? exp_f32(v[j] - mx) : 0.0f;
        sum += v[j];
    }
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) sum += __shfl_xor(sum, m);
    float inv = 1.0f / sum;
    float p[PER];
    unsigned taken = 0;
#pragma unroll
    for (int j = 0; j < PER; j++) p[j] = v[j] * inv;
    float sel_p = 0.0f, s = 0.0f;
    int sel_i = 0;
    for (int r = 0; r < k; r++) {
        float bp = -1.0f;
        int bi = 0x7fffffff;
#pragma unroll
        for (int j = 0; j < PER; j++) {
            int i = lane + WAVE * j;
            if (i < n_expert && !(taken >> j & 1) && better(p[j], i, bp, bi)) {
                bp = p[j];
                bi = i;
            }
        }
#pragma unroll
        for (int m = 32; m >= 1; m >>= 1) {
            float op = __shfl_xor(bp, m);
            int oi = __shfl_xor(bi, m);
            if (better(op, oi, bp, bi)) {
                bp = op;
                bi = oi;
            }
        }
        // NaN probabilities (non-finite h) match no candidate: take the lowest
        // free expert so that ids stay in range
        if (bi >= n_expert) {
            int j = 0;
            for (; j < n_expert; j++) {
                const int owner_taken = __shfl((int)taken, j & 63);
                if (!((owner_taken >> (j >> 6)) & 1)) break;
            }
            bi = j < n_expert ? j : 0;
            bp = 0.0f;
        }
        if ((bi & 63) == lane) taken |= 1u << (bi >> 6);
        if (r == lane) {
            sel_p = bp;
            sel_i = bi;
        }
        s += bp; // the sum in rank order, as the reference's iterator sum
    }
    s = fmaxf(s, 1.0f / 16384.0f);
    if (lane < k) {
        ids[(size_t)t * k + lane] = sel_i;
        wts[(size_t)t * k + lane] = sel_p / s;
    }
}

// ---------------------------------------------------------------------------
// Dispatch: a counting sort of the T*k pairs by expert, tokens ascending
// within an expert (the `routed` lists of model.rs:866-873; Metal's moe_sort,
// kernels.metal:1675-1739).  Counts are integer atomics in LDS, whose result
// does not depend on their order; a pair's place among its expert's pairs is
// the number of earlier tokens with that expert, read from a token bitmap, so
// the order is deterministic.  One workgroup of 1024 threads.
constexpr int SORT_THREADS = 1024;
constexpr int MAX_EXPERTS = 256;

__global__ __launch_bounds__(SORT_THREADS) void k_sort(const int *__restrict__ ids, const float *__restrict__ wts,
                                                       int n_expert, int k, int T, Dispatch dp)
{
    __shared__ int cnt[MAX_EXPERTS];
    __shared__ int scan[MAX_EXPERTS];
    __shared__ int run[MAX_EXPERTS];
    __shared__ unsigned bm[MAX_EXPERTS][SORT_THREADS / 32];
    const int tid = threadIdx.x;
    const int P = T * k;
    for (int e = tid; e < MAX_EXPERTS; e += SORT_THREADS) {
        cnt[e] = 0;
        run[e] = 0;
    }
    for (int i = tid; i < MAX_EXPERTS * (SORT_THREADS / 32); i += SORT_THREADS) (&bm[0][0])[i] = 0u;
    __syncthreads();
    for (int i = tid; i < P; i += SORT_THREADS) atomicAdd(&cnt[ids[i]], 1); // ids < n_expert (k_route)
    __syncthreads();
    // inclusive scan of (active << 20 | count): expert offsets and active slots at once
    if (tid < MAX_EXPERTS) scan[tid] = tid < n_expert ? ((cnt[tid] > 0) << 20) | cnt[tid] : 0;
    __syncthreads();
    for (int off = 1; off < MAX_EXPERTS; off <<= 1) {
        int add = (tid < MAX_EXPERTS && tid >= off) ? scan[tid - off] : 0;
        __syncthreads();
        if (tid < MAX_EXPERTS) scan[tid] += add;
        __syncthreads();
    }
    if (tid < n_expert) {
        int c = cnt[tid];
        int incl = scan[tid];
        int beg = (incl & 0xFFFFF) - c;
        if (c > 0) {
            int u = (incl >> 20) - 1;
            dp.act_expert[u] = tid;
            dp.act_beg[u] = beg;
            dp.act_cnt[u] = c;
        }
        cnt[tid] = beg; // from here on: the expert's first position
    }
    if (tid == 0) *dp.n_active = scan[MAX_EXPERTS - 1] >> 20;
    __syncthreads();
    for (int c0 = 0; c0 < T; c0 += SORT_THREADS) {
        const int t = c0 + tid;
        const int word = tid >> 5;
        const unsigned bit = 1u << (tid & 31);
        if (t < T)
            for (int j = 0; j < k; j++) atomicOr(&bm[ids[(size_t)t * k + j]][word], bit);
        __syncthreads();
        if (t < T) {
            int pos[16];
            for (int j = 0; j < k; j++) {
                int e = ids[(size_t)t * k + j];
                int r = run[e] + __popc(bm[e][word] & (bit - 1));
                for (int w = 0; w < word; w++) r += __popc(bm[e][w]);
                int p = cnt[e] + r;
                dp.pair_tok[p] = t;
                dp.pair_exp[p] = e;
                dp.pair_w[p] = wts[(size_t)t * k + j];
                pos[j] = p;
            }
            // positions ascend with the expert id: insertion sort of k values
            for (int a = 1; a < k; a++) {
                int v = pos[a], b = a - 1;
                while (b >= 0 && pos[b] > v) {
                    pos[b + 1] = pos[b];
                    b--;
                }
                pos[b + 1] = v;
            }
            for (int j = 0; j < k; j++) dp.tok_pairs[(size_t)t * k + j] = pos[j];
        }
        __syncthreads();
        if (tid < MAX_EXPERTS) {
            int add = 0;
            for (int w = 0; w < SORT_THREADS / 32; w++) {
                add += __popc(bm[tid][w]);
                bm[tid][w] = 0u;
            }
            run[tid] += add;
        }
        __syncthreads();
    }
}

// ---------------------------------------------------------------------------
// Block dots: one 32-element weight block against one Q8 activation block.
// `idot` is the block's int32 (the integer of quant.rs:599-607 / 609-627 /
// 651-686), the return value its f32 contribution.

struct XBlock {
    int v[8];
    float d, s;
};

__device__ inline void load_x(const int8_t *xq, const float *xd, const float *xs, size_t xrow, int K, int b,
                              XBlock &x)
{
    const int4 *p = reinterpret_cast<const int4 *>(xq + xrow * K + 32 * b);
    int4 a = p[0], c = p[1];
    x.v[0] = a.x; x.v[1] = a.y; x.v[2] = a.z; x.v[3] = a.w;
    x.v[4] = c.x; x.v[5] = c.y; x.v[6] = c.z; x.v[7] = c.w;
    x.d = xd[xrow * (K / 32) + b];
    x.s = xs[xrow * (K / 32) + b];
}

// The weight block, loaded once for every token of the expert.
template <int TY> struct WBlock;

template <> struct WBlock<T_Q8_0> {
    int q[8];
    float d;
    __device__ inline void load(const DevMat &M, size_t mrow, int b)
    {
        const int4 *p = reinterpret_cast<const int4 *>(M.q + mrow * M.cols + 32 * b);
        int4 a = p[0], c = p[1];
        q[0] = a.x; q[1] = a.y; q[2] = a.z; q[3] = a.w;
        q[4] = c.x; q[5] = c.y; q[6] = c.z; q[7] = c.w;
        d = f16_at(M.s + 2 * (mrow * (M.cols / 32) + b));
    }
    __device__ inline float dot(const XBlock &x, int &idot) const
    {
        int acc = 0;
#pragma unroll
        for (int i = 0; i < 8; i++) acc = dot4(q[i], x.v[i], acc);
        idot = acc;
        return (float)acc * (d * x.d);
    }
    // The eight 4-byte partial sums the reference's 8 i32 lanes hold, and the
    // block's f32 scale f16(d) * x.d (quant.rs:1373-1378).
    __device__ inline void partials(const XBlock &x, int v[8], float &c, float &mt, float &dm) const
    {
#pragma unroll
        for (int i = 0; i < 8; i++) v[i] = dot4(q[i], x.v[i], 0);
        c = d * x.d;
        mt = 0.0f;
        dm = 0.0f;
    }
};

// q4_K: sub-block sb of a 256-element super-block; 6-bit scale and min from
// the packed bytes (scale_min_k4, quant.rs:143-153).
template <> struct WBlock<T_Q4K> {
    int q[8];
    float dsc, dmn;
    __device__ inline void load(const DevMat &M, size_t mrow, int b)
    {
        const int sbk = b >> 3, sb = b & 7;
        const int4 *p = reinterpret_cast<const int4 *>(M.q + mrow * (M.cols / 2) + 128 * sbk + 32 * (sb >> 1));
        int4 a = p[0], c = p[1];
        int raw[8] = {a.x, a.y, a.z, a.w, c.x, c.y, c.z, c.w};
        const int sh = 4 * (sb & 1);
#pragma unroll
        for (int i = 0; i < 8; i++) q[i] = (int)(((unsigned)raw[i] >> sh) & 0x0F0F0F0Fu);
        const uint8_t *hd = M.s + 16 * (mrow * (M.cols / 256) + sbk);
        const int4 hv = *reinterpret_cast<const int4 *>(hd);
        float d = __half2float(__ushort_as_half((unsigned short)(hv.x & 0xFFFF)));
        float dmin = __half2float(__ushort_as_half((unsigned short)((unsigned)hv.x >> 16)));
        // the 12 scale bytes start at byte 4 of the header
        auto sc = [&](int i) { return byte_at(hv, 4 + i); };
        int s, m;
        if (sb < 4) {
            s = sc(sb) & 63;
            m = sc(sb + 4) & 63;
        } else {
            s = (sc(sb + 4) & 0xF) | ((sc(sb - 4) >> 6) << 4);
            m = (sc(sb + 4) >> 4) | ((sc(sb) >> 6) << 4);
        }
        dsc = d * (float)s;
        dmn = dmin * (float)m;
        dmin_ = dmin;
        m_ = m;
    }
    float dmin_;
    int m_;
    __device__ inline float dot(const XBlock &x, int &idot) const
    {
        int acc = 0;
#pragma unroll
        for (int i = 0; i < 8; i++) acc = dot4(q[i], x.v[i], acc);
        idot = acc;
        return (float)acc * (dsc * x.d) - dmn * x.s;
    }
    // lanes of dot_u8_i8(nibbles, x), scale d*sc*x.d, and the min term m*x.s
    // with the super-block's dmin (quant.rs:1394-1420)
    __device__ inline void partials(const XBlock &x, int v[8], float &c, float &mt, float &dm) const
    {
#pragma unroll
        for (int i = 0; i < 8; i++) v[i] = dot4(q[i], x.v[i], 0);
        c = dsc * x.d;
        mt = (float)m_ * x.s;
        dm = dmin_;
    }
};

// q6_K: 32-element block bb of a super-block is half n = bb/4, quarter k =
// bb%4: nibbles of ql[32(k&1)..] (low for k<2, high otherwise), bits 2k..2k+1
// of qh, sub-scales sc[8n + 2k] (elements 0..15) and sc[8n + 2k + 1] (16..31).
template <> struct WBlock<T_Q6K> {
    int q[8];
    int sc0, sc1;
    float d;
    __device__ inline void load(const DevMat &M, size_t mrow, int b)
    {
        const int sbk = b >> 3, bb = b & 7, n = bb >> 2, k = bb & 3;
        const uint8_t *base = M.q + 192 * (mrow * (M.cols / 256) + sbk);
        const int4 *pl = reinterpret_cast<const int4 *>(base + 64 * n + 32 * (k & 1));
        const int4 *ph = reinterpret_cast<const int4 *>(base + 128 + 32 * n);
        int4 l0 = pl[0], l1 = pl[1], h0 = ph[0], h1 = ph[1];
        int lo[8] = {l0.x, l0.y, l0.z, l0.w, l1.x, l1.y, l1.z, l1.w};
        int hi[8] = {h0.x, h0.y, h0.z, h0.w, h1.x, h1.y, h1.z, h1.w};
        const int ls = 4 * (k >> 1), hs = 2 * k;
#pragma unroll
        for (int i = 0; i < 8; i++)
            q[i] = (int)((((unsigned)lo[i] >> ls) & 0x0F0F0F0Fu) | ((((unsigned)hi[i] >> hs) & 0x03030303u) << 4));
        const int8_t *scp = reinterpret_cast<const int8_t *>(M.s + 16 * (mrow * (M.cols / 256) + sbk));
        sc0 = scp[8 * n + 2 * k];
        sc1 = scp[8 * n + 2 * k + 1];
        d = f16_at(M.d + 2 * (mrow * (M.cols / 256) + sbk));
    }
    __device__ inline float dot(const XBlock &x, int &idot) const
    {
        // values are 0..63 here; the -32 offset is 32 * (sum of x), as in
        // the reference's maddubs(32, x) term (quant.rs:1514-1517)
        int a0 = 0, a1 = 0, s0 = 0, s1 = 0;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            a0 = dot4(q[i], x.v[i], a0);
            s0 = dot4(0x01010101, x.v[i], s0);
            a1 = dot4(q[4 + i], x.v[4 + i], a1);
            s1 = dot4(0x01010101, x.v[4 + i], s1);
        }
        int isum = sc0 * (a0 - 32 * s0) + sc1 * (a1 - 32 * s1);
        idot = isum;
        return (float)isum * (d * x.d);
    }
    // lanes of madd(maddubs(q, x) - maddubs(32, x), sc): lanes 0-3 carry
    // elements 0..15 under sc0, lanes 4-7 elements 16..31 under sc1
    // (quant.rs:1510-1527)
    __device__ inline void partials(const XBlock &x, int v[8], float &c, float &mt, float &dm) const
    {
#pragma unroll
        for (int i = 0; i < 8; i++)
            v[i] = (i < 4 ? sc0 : sc1) * (dot4(q[i], x.v[i], 0) - 32 * dot4(0x01010101, x.v[i], 0));
        c = d * x.d;
        mt = 0.0f;
        dm = 0.0f;
    }
};

__device__ inline float sigmoid(float x) { return 1.0f / (1.0f + exp_f32(-x)); }

__device__ inline float silu_mul(float g, float u)
{
    // ops::silu(g) * u (ops.rs:159-167, model.rs:1121-1124)
    return (g * sigmoid(g)) * u;
}

// ---------------------------------------------------------------------------
// Grouped expert matvec.  blockIdx.y is an active-expert slot (or, at u_max,
// the shared expert); a group of G = K/32 lanes owns one weight row, one lane
// per 32-element block.  The block is loaded once and met by every token of
// the expert, TCH tokens at a time.  Group sums use a fixed butterfly, so the
// result does not depend on timing.
constexpr int MV_WAVES = 4;
constexpr int TCH = 4;

template <int TY, int G, bool GATEUP, bool DUMP>
__global__ __launch_bounds__(MV_WAVES *WAVE) void k_expert_mv(MvArgs a)
{
    constexpr int RPW = WAVE / G; // rows per wave
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int b = lane % G; // this lane's block
    const int u = blockIdx.y;
    const bool shared = u == a.u_max;
    int e = 0, beg, cnt;
    if (shared) {
        beg = a.P;
        cnt = a.T;
    } else {
        if (u >= *a.dp.n_active) return;
        e = a.dp.act_expert[u];
        beg = a.dp.act_beg[u];
        cnt = a.dp.act_cnt[u];
    }
    const DevMat &A = shared ? a.sa : a.a;
    const DevMat &B = shared ? a.sb : a.b;
    const int rows = A.rows, K = A.cols;
    const int row = (blockIdx.x * MV_WAVES + wave) * RPW + lane / G;
    if (row >= rows) return; // whole groups leave together: shuffles stay inside a group
    const size_t mrow = (size_t)e * rows + row;
    WBlock<TY> wa, wb;
    wa.load(A, mrow, b);
    if (GATEUP) wb.load(B, mrow, b);
    for (int i0 = 0; i0 < cnt; i0 += TCH) {
        float sa[TCH], sb[TCH];
#pragma unroll
        for (int j = 0; j < TCH; j++) {
            sa[j] = 0.0f;
            sb[j] = 0.0f;
            const int i = i0 + j;
            if (i >= cnt) continue;
            const size_t xrow = a.x_by_token ? (size_t)(shared ? i : a.dp.pair_tok[beg + i]) : (size_t)(beg + i);
            XBlock x;
            load_x(a.xq, a.xd, a.xs, xrow, K, b, x);
            int ia, ib = 0;
            sa[j] = wa.dot(x, ia);
            if (GATEUP) sb[j] = wb.dot(x, ib);
            if (DUMP) {
                const size_t at = ((size_t)(beg + i) * rows + row) * G + b;
                if (a.dump_a) a.dump_a[at] = ia;
                if (GATEUP && a.dump_b) a.dump_b[at] = ib;
            }
        }
#pragma unroll
        for (int m = G / 2; m >= 1; m >>= 1) {
#pragma unroll
            for (int j = 0; j < TCH; j++) {
                sa[j] += __shfl_xor(sa[j], m);
                if (GATEUP) sb[j] += __shfl_xor(sb[j], m);
            }
        }
        if (b == 0) {
#pragma unroll
            for (int j = 0; j < TCH; j++) {
                const int i = i0 + j;
                if (i >= cnt) break;
                a.out[(size_t)(beg + i) * rows + row] = GATEUP ? silu_mul(sa[j], sb[j]) : sa[j];
            }
        }
    }
}

// ---------------------------------------------------------------------------
// Gate/up in the reference's f32 order.  The SwiGLU intermediate is quantised
// again before the down projection, so any difference in the rounding of
// gate or up can move an int8 of the intermediate by one.  These sums are
// therefore formed exactly as biv's x86 kernels form them (quant.rs:1368-1533):
// every block gives eight 4-byte i32 partials (the 8 lanes of a ymm
// register), converted to f32 and FMA'd with the block's scale into one of two
// accumulators by block parity; then acc0 + acc1 and the hsum tree
// (quant.rs:1149-1153); for Q4_K the mins are summed apart and subtracted
// last.  The result is the reference's f32, bit for bit.
//
// A wave first stores the partials of 4 (matrix, row, token) combinations in
// LDS ("fills"), then 16 lanes per combination run the 16 FMA chains.
constexpr int GU_TCH = 2; // tokens per chunk
constexpr int SLOT = 11;  // floats per block in LDS: 8 partials, scale, min term, dmin

template <int TY, int G, bool DUMP>
__global__ __launch_bounds__(MV_WAVES *WAVE) void k_gateup_exact(MvArgs a)
{
    constexpr int RPW = WAVE / G;          // rows per wave
    constexpr int FILLS = 4 / RPW;         // fills per chain pass
    constexpr int COMBOS = 2 * RPW * GU_TCH; // per token chunk: (gate, up) x rows x tokens
    constexpr int PASSES = COMBOS / 4;
    __shared__ float sp[MV_WAVES][4][G][SLOT];
    __shared__ float sr[MV_WAVES][COMBOS];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int b = lane % G, rg = lane / G;
    const int u = blockIdx.y;
    const bool shared = u == a.u_max;
    int e = 0, beg, cnt;
    if (shared) {
        beg = a.P;
        cnt = a.T;
    } else {
        if (u >= *a.dp.n_active) return; // uniform over the workgroup
        e = a.dp.act_expert[u];
        beg = a.dp.act_beg[u];
        cnt = a.dp.act_cnt[u];
    }
    const DevMat &A = shared ? a.sa : a.a;
    const DevMat &B = shared ? a.sb : a.b;
    const int rows = A.rows, K = A.cols;
    const int row0 = (blockIdx.x * MV_WAVES + wave) * RPW;
    const int row = row0 + rg;
    const bool row_ok = row < rows;
    const size_t mrow = (size_t)e * rows + (row_ok ? row : 0);
    WBlock<TY> wm[2];
    wm[0].load(A, mrow, b);
    wm[1].load(B, mrow, b);
    // chain lane roles: combination cb, parity pi, ymm lane l
    const int cb = lane >> 4, pi = (lane >> 3) & 1, l = lane & 7;
    for (int i0 = 0; i0 < cnt; i0 += GU_TCH) {
        for (int pass = 0; pass < PASSES; pass++) {
#pragma unroll
            for (int f = 0; f < FILLS; f++) {
                const int slot = f * RPW + rg;          // 0..3 within the pass
                const int idx = (pass * 4 + f * RPW) / RPW; // (matrix, token) index
                const int m = idx & 1, j = idx >> 1;
                const int i = i0 + j;
                float *dst = sp[wave][slot][b];
                if (i < cnt && row_ok) {
                    const size_t xrow = shared ? (size_t)i : (size_t)a.dp.pair_tok[beg + i];
                    XBlock x;
                    load_x(a.xq, a.xd, a.xs, xrow, K, b, x);
                    int v[8];
                    float c, mt, dm;
                    if (m == 0) wm[0].partials(x, v, c, mt, dm);
                    else wm[1].partials(x, v, c, mt, dm);
#pragma unroll
                    for (int q = 0; q < 8; q++) dst[q] = (float)v[q];
                    dst[8] = c;
                    dst[9] = mt;
                    dst[10] = dm;
                    if (DUMP) {
                        int32_t *dump = m == 0 ? a.dump_a : a.dump_b;
                        if (dump) {
                            int sum = 0;
#pragma unroll
                            for (int q = 0; q < 8; q++) sum += v[q];
                            dump[((size_t)(beg + i) * rows + row) * G + b] = sum;
                        }
                    }
                } else {
#pragma unroll
                    for (int q = 0; q < SLOT; q++) dst[q] = 0.0f;
                }
            }
            __syncthreads();
            // 16 chains per combination: acc over blocks pi, pi+2, ... in order
            const float(*blk)[SLOT] = sp[wave][cb];
            float acc = 0.0f;
#pragma unroll 8
            for (int s2 = 0; s2 < G / 2; s2++) {
                const int bb = 2 * s2 + pi;
                acc = fmaf(blk[bb][l], blk[bb][8], acc);
            }
            float t = acc + __shfl_xor(acc, 8); // acc0 + acc1
            t = t + __shfl_xor(t, 4);           // 128-bit halves
            t = t + __shfl_xor(t, 2);           // movehl
            t = t + __shfl_xor(t, 1);           // movehdup
            if (TY == T_Q4K && (lane & 15) == 0) {
                // mins += dmin * (m1 * s[2j] + m2 * s[2j+1]), in block order
                float mins = 0.0f;
                for (int s2 = 0; s2 < G / 2; s2++)
                    mins = mins + blk[2 * s2][10] * (blk[2 * s2][9] + blk[2 * s2 + 1][9]);
                t = t - mins;
            }
            if ((lane & 15) == 0) sr[wave][pass * 4 + cb] = t;
            __syncthreads();
        }
        // combination index c = (j * 2 + m) * RPW + rg
        if (b == 0 && row_ok) {
#pragma unroll
            for (int j = 0; j < GU_TCH; j++) {
                const int i = i0 + j;
                if (i >= cnt) break;
                const float g = sr[wave][(j * 2 + 0) * RPW + rg];
                const float up = sr[wave][(j * 2 + 1) * RPW + rg];
                a.out[(size_t)(beg + i) * rows + row] = silu_mul(g, up);
            }
        }
        __syncthreads();
    }
}

// ---------------------------------------------------------------------------
// Combine (model.rs:884-896): out[t] = 0; for each of t's experts in
// ascending id, out = fma(w, y, out) (quant::axpy, quant.rs:1209-1226); then
// out = fma(sigmoid(g), y_shared, out).  Then out is written or added.
__global__ __launch_bounds__(256) void k_combine(const float *__restrict__ y, Dispatch dp,
                                                 const float *__restrict__ glogit, int has_shared, int T, int P,
                                                 int k, int E, float *__restrict__ out, int add)
{
    const int t = blockIdx.y;
    const int c = blockIdx.x * blockDim.x + threadIdx.x;
    if (c >= E) return;
    float o = 0.0f;
    for (int j = 0; j < k; j++) {
        int p = dp.tok_pairs[(size_t)t * k + j];
        o = fmaf(dp.pair_w[p], y[(size_t)p * E + c], o);
    }
    if (has_shared) {
        float g = glogit[t];
        float sg = sigmoid(g);
        o = fmaf(sg, y[(size_t)(P + t) * E + c], o);
    }
    float *po = out + (size_t)t * E + c;
    *po = add ? *po + o : o;
}

// One launch over the routed slots (routed = 1) and/or the shared expert.
template <bool GATEUP, bool DUMP>
hipError_t launch_mv_t(MvArgs a, int routed, int shared, hipStream_t st)
{
    const DevMat &M = routed ? a.a : a.sa;
    const int G = M.cols / 32;
    if (!routed) a.u_max = 0; // the only slot is the shared expert's
    const int slots = (routed ? a.u_max : 0) + (shared ? 1 : 0);
    if (slots == 0) return hipSuccess;
    const int rows_per_wg = MV_WAVES * (WAVE / G);
    dim3 grid((M.rows + rows_per_wg - 1) / rows_per_wg, slots);
    dim3 block(MV_WAVES * WAVE);
#define BIV_MV_CASE(TY, GG)                                                                                     \
    if (M.ty == TY && G == GG) {                                                                                \
        k_expert_mv<TY, GG, GATEUP, DUMP><<<grid, block, 0, st>>>(a);                                           \
        return hipGetLastError();                                                                               \
    }
    BIV_MV_CASE(T_Q8_0, 64)
    BIV_MV_CASE(T_Q8_0, 32)
    BIV_MV_CASE(T_Q8_0, 16)
    BIV_MV_CASE(T_Q4K, 64)
    BIV_MV_CASE(T_Q4K, 32)
    BIV_MV_CASE(T_Q4K, 16)
    BIV_MV_CASE(T_Q6K, 64)
    BIV_MV_CASE(T_Q6K, 32)
    BIV_MV_CASE(T_Q6K, 16)
#undef BIV_MV_CASE
    return hipErrorInvalidValue;
}

// One launch of the exact gate/up kernel over routed slots and/or the shared expert.
template <bool DUMP>
hipError_t launch_gu_t(MvArgs a, int routed, int shared, hipStream_t st)
{
    const DevMat &M = routed ? a.a : a.sa;
    const int G = M.cols / 32;
    if (!routed) a.u_max = 0;
    const int slots = (routed ? a.u_max : 0) + (shared ? 1 : 0);
    if (slots == 0) return hipSuccess;
    const int rows_per_wg = MV_WAVES * (WAVE / G);
    dim3 grid((M.rows + rows_per_wg - 1) / rows_per_wg, slots);
    dim3 block(MV_WAVES * WAVE);
#define BIV_GU_CASE(TY, GG)                                                                                     \
    if (M.ty == TY && G == GG) {                                                                                \
        k_gateup_exact<TY, GG, DUMP><<<grid, block, 0, st>>>(a);                                                \
        return hipGetLastError();                                                                               \
    }
    BIV_GU_CASE(T_Q8_0, 64)
    BIV_GU_CASE(T_Q8_0, 32)
    BIV_GU_CASE(T_Q8_0, 16)
    BIV_GU_CASE(T_Q4K, 64)
    BIV_GU_CASE(T_Q4K, 32)
    BIV_GU_CASE(T_Q4K, 16)
    BIV_GU_CASE(T_Q6K, 64)
    BIV_GU_CASE(T_Q6K, 32)
    BIV_GU_CASE(T_Q6K, 16)
#undef BIV_GU_CASE
    return hipErrorInvalidValue;
}

template <bool GATEUP>
hipError_t launch_mv(const MvArgs &a, hipStream_t st)
{
    const bool dump = a.dump_a || a.dump_b;
    const bool has_shared = a.sa.q != nullptr;
    // routed and shared in one launch when they share type and shape
    const bool together = has_shared && a.sa.ty == a.a.ty && a.sa.cols == a.a.cols && a.sa.rows == a.a.rows;
    hipError_t err;
    if (together)
        return dump ? launch_mv_t<GATEUP, true>(a, 1, 1, st) : launch_mv_t<GATEUP, false>(a, 1, 1, st);
    err = dump ? launch_mv_t<GATEUP, true>(a, 1, 0, st) : launch_mv_t<GATEUP, false>(a, 1, 0, st);
    if (err != hipSuccess || !has_shared) return err;
    return dump ? launch_mv_t<GATEUP, true>(a, 0, 1, st) : launch_mv_t<GATEUP, false>(a, 0, 1, st);
}

} // namespace

hipError_t launch_quant_rows(const float *x, int n_blocks, int8_t *qs, float *d, float *s, hipStream_t st)
{
    if (n_blocks <= 0) return hipSuccess;
    k_quant_rows<<<(n_blocks + 255) / 256, 256, 0, st>>>(x, n_blocks, qs, d, s);
    return hipGetLastError();
}

hipError_t launch_router(const float *router, const float *gate_inp, int n_expert, int E, const float *h, int T,
                         float *logits, float *glogit, hipStream_t st)
{
    const int rows = n_expert + 1;
    if (T <= 1) {
        dim3 grid((rows + 1) / 2, T);
        k_router<1><<<grid, 64, 0, st>>>(router, gate_inp, n_expert, E, h, T, logits, glogit);
    } else if (T <= 8) {
        dim3 grid((rows + 3) / 4, 1);
        k_router<8><<<grid, 128, 0, st>>>(router, gate_inp, n_expert, E, h, T, logits, glogit);
    } else {
        dim3 grid((rows + 7) / 8, (T + 15) / 16);
        k_router<16><<<grid, 256, 0, st>>>(router, gate_inp, n_expert, E, h, T, logits, glogit);
    }
    return hipGetLastError();
}

hipError_t launch_route(const float *logits, int n_expert, int k, int T, int *ids, float *wts, hipStream_t st)
{
    k_route<<<(T + 3) / 4, 256, 0, st>>>(logits, n_expert, k, T, ids, wts);
    return hipGetLastError();
}

hipError_t launch_sort(const int *ids, const float *wts, int n_expert, int k, int T, const Dispatch &dp,
                       hipStream_t st)
{
    k_sort<<<1, SORT_THREADS, 0, st>>>(ids, wts, n_expert, k, T, dp);
    return hipGetLastError();
}

hipError_t launch_gateup(const MvArgs &a, hipStream_t st)
{
    const bool dump = a.dump_a || a.dump_b;
    const bool has_shared = a.sa.q != nullptr;
    const bool together = has_shared && a.sa.ty == a.a.ty && a.sa.cols == a.a.cols && a.sa.rows == a.a.rows;
    if (together) return dump ? launch_gu_t<true>(a, 1, 1, st) : launch_gu_t<false>(a, 1, 1, st);
    hipError_t err = dump ? launch_gu_t<true>(a, 1, 0, st) : launch_gu_t<false>(a, 1, 0, st);
    if (err != hipSuccess || !has_shared) return err;
    return dump ? launch_gu_t<true>(a, 0, 1, st) : launch_gu_t<false>(a, 0, 1, st);
}

hipError_t launch_down(const MvArgs &a, hipStream_t st) { return launch_mv<false>(a, st); }

hipError_t launch_combine(const float *y, const Dispatch &dp, const float *glogit, int has_shared, int T, int P,
                          int k, int E, float *out, int add, hipStream_t st)
{
    dim3 grid((E + 255) / 256, T);
    k_combine<<<grid, 256, 0, st>>>(y, dp, glogit, has_shared, T, P, k, E, out, add);
    return hipGetLastError();
}

} // namespace biv
