// BF16 experts at prefill sizes on the matrix cores (gfx950 MFMA).
//
// biv's dot_bf16 (engine/src/quant.rs:1228-1256) multiplies bf16 weights by
// f32 activations in f32 FMA chains.  Here the activations are split into
// two bf16 halves, x = hi + lo + r with |r| <= 2^-17 |x| (hi = x rounded to
// bf16, lo = x - hi rounded to bf16), and each product w * hi and w * lo is
// exact in f32; v_mfma_f32_32x32x16_bf16 sums them in f32.  Only the order of
// the sums differs from the reference (bit-identical results come from the
// chain kernels in kernels.hip, which run decode sizes).
//
// Operand order: a 16-byte chunk c of a row holds the 8 elements
// 128 (c / 16) + 16 m + (c % 16), m = 0..7: the BF16 weight layout of
// layout.hpp (bf16_elem), so a lane's MFMA operand is one 16-byte load of the
// weights and one of each activation half.
#include "common.hpp"
#include "expf_ref.h"

namespace biv {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int WAVE = 64;

__device__ inline uint32_t bf16_bits(float x)
{
    // round to nearest, ties to even (finite x); NaN stays NaN
    const uint32_t u = __float_as_uint(x);
    if (x != x) return 0x7FC0u;
    return (u + 0x7FFFu + ((u >> 16) & 1u)) >> 16;
}

__device__ inline bf16x8 as_bf16x8(const uint4 &v) { return __builtin_bit_cast(bf16x8, v); }

// hi / lo bf16 halves of rows x [rows][K] in the chunk order above:
// xh[r][c] and xl[r][c] are 16-byte chunks.  One thread per chunk.
__global__ __launch_bounds__(256) void k_split_bf16(const float *__restrict__ x, int rows, int K,
                                                    uint4 *__restrict__ xh, uint4 *__restrict__ xl)
{
    const size_t idx = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    const int nc = K / 8;
    if (idx >= (size_t)rows * nc) return;
    const size_t r = idx / nc;
    const int c = (int)(idx % nc), g = c / 16, L = c % 16;
    uint32_t h[8], lo[8];
#pragma unroll
    for (int m = 0; m < 8; m++) {
        const float v = x[r * K + 128 * g + 16 * m + L];
        h[m] = bf16_bits(v);
        lo[m] = bf16_bits(v - __uint_as_float(h[m] << 16));
    }
    xh[idx] = make_uint4(h[0] | h[1] << 16, h[2] | h[3] << 16, h[4] | h[5] << 16, h[6] | h[7] << 16);
    xl[idx] = make_uint4(lo[0] | lo[1] << 16, lo[2] | lo[3] << 16, lo[4] | lo[5] << 16, lo[6] | lo[7] << 16);
}

__device__ const uint64_t exp_tab[32] = BIV_EXPF_TAB_INIT;

// silu(g) * u (ops.rs:159-167) with the exp table in shared memory
__device__ inline float silu_mul_t(float g, float u, const uint64_t *tab)
{
    double r;
    uint64_t ki;
    const uint32_t i = biv_expf_reduce(-g, &r, &ki);
    const float ex = biv_expf_finish(-g, r, ki, tab[i]);
    return (g * (1.0f / (1.0f + ex))) * u;
}

// Grouped GEMM over the slots of the dispatch (the shared expert's first):
// a workgroup takes a whole slot (up to TOK_TILE pairs) and ROW_TILE output
// rows; wave (wt, wr) of the 4 x 2 grid takes 64 pairs x 64 rows of each of
// gate and up (gate/up) or 64 pairs x 128 rows (down), as 32 x 32 blocks, and
// skips the blocks of pairs past the slot's count.
// gate/up: each block has a gate and an up accumulator and the SwiGLU is
// formed in the epilogue.
//
// The row tiles of a slot go to one XCD (workgroup ids b, b + 8, ... are
// dispatched to one XCD): the slot's activation rows come from HBM once per
// slot and from that XCD's L2 after, and every expert's weights are read
// once per slot.
//
// K advances in stages of 32 (4 chunks, 64 bytes of a row).  A stage's tiles
// go straight from global memory into LDS (global_load_lds) into a ring of
// three buffers: the loads of the next two stages are in flight while the
// waves run this stage's MFMAs from LDS.  LDS layouts: A [half][pair][4], B
// [row][4], chunk c of row r in slot 4 r + (c ^ ((r >> 2) & 3)): the 64 lanes
// of a load write 64 consecutive slots, 4 lanes reading one row's 64
// contiguous bytes, and the swizzle keeps a fragment read (consecutive rows,
// one chunk) free of bank conflicts.
constexpr int NWT = 4;              // waves along the pairs
constexpr int NWR = 2;              // waves along the rows
constexpr int TOK_TILE = 64 * NWT;  // pairs of a workgroup
constexpr int NTH = 64 * NWT * NWR; // threads of a workgroup
constexpr int SK = 4;               // chunks per stage
constexpr int N_XCD = 8;
static_assert(TOK_TILE == MFMA_TOK_TILE, "slot size");

template <int K, bool GATEUP>
__global__ __launch_bounds__(NTH) __attribute__((amdgpu_waves_per_eu(2, 8))) void k_mfma_bf16(MfArgs a)
{
    constexpr int NC = K / 8;          // chunks per row
    constexpr int NS = NC / SK;        // stages
    constexpr int NB = GATEUP ? 2 : 1; // weight matrices
    constexpr int RB = 4 / NB;         // 32-row blocks of a wave, per matrix
    constexpr int ROW_TILE = 32 * RB * NWR; // output rows of a workgroup
    constexpr int BR = ROW_TILE * NB;  // weight rows of a tile
    constexpr int A_SLOTS = 2 * SK * TOK_TILE, B_SLOTS = SK * BR;
    static_assert(A_SLOTS % NTH == 0 && B_SLOTS % NTH == 0, "tile shapes");
    __shared__ uint4 sA0[A_SLOTS], sA1[A_SLOTS], sA2[A_SLOTS], sB0[B_SLOTS], sB1[B_SLOTS], sB2[B_SLOTS];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int li = lane & 31, kg = lane >> 5;
    // the two waves of a SIMD (waves w and w + 4) take pairs 64 apart x 2
    const int wt = wave >> 1, wr = wave & 1;
    // workgroup -> (slot, row tile): ids b with one b % 8 are one XCD's
    const int G = N_XCD * a.n_rt, b = blockIdx.x;
    const int u = (b / G) * N_XCD + b % N_XCD, rt = (b % G) / N_XCD;
    if (u >= a.u_max + a.n_sh) return;
    const bool shared = u < a.n_sh;
    int e = 0, beg, cnt, tok0 = 0;
    if (shared) {
        tok0 = u * a.sh_chunk;
        beg = a.P + tok0;
        cnt = min(a.sh_chunk, a.T - tok0);
    } else {
        const Slot sl = a.dp.slots[u - a.n_sh];
        if (sl.cnt == 0) return; // uniform over the workgroup
        e = sl.expert;
        beg = sl.beg;
        cnt = sl.cnt;
    }
    const DevMat &Ma = shared ? a.sa : a.a;
    const int rows = Ma.rows;
    const int r0 = rt * ROW_TILE;
    // this wave's 32-pair blocks that hold pairs of the slot
    const bool live0 = wt * 64 < cnt, live1 = wt * 64 + 32 < cnt;
    // this thread's load slots: slot tid + NTH q is row (tid + NTH q) / 4,
    // position tid % 4 (the chunk it loads is swizzled by the row); pairs
    // past the count load the slot's last pair (unused)
    constexpr int RQ = NTH / SK; // rows a pass of the threads covers
    const int p = tid % SK;
    const uint4 *srcA[2 * TOK_TILE / RQ];
    int swA[2 * TOK_TILE / RQ];
#pragma unroll
    for (int q = 0; q < 2 * TOK_TILE / RQ; q++) { // A rows: (half, pair)
        const int tr = (tid + NTH * q) / SK, hl = tr / TOK_TILE, tt = tr % TOK_TILE;
        const int ti = min(tt, cnt - 1);
        const size_t ar = GATEUP ? (size_t)(shared ? tok0 + ti : a.dp.pair_tok[beg + ti]) : (size_t)(beg + ti);
        srcA[q] = (hl ? a.xl : a.xh) + ar * NC;
        swA[q] = p ^ ((tt >> 2) & 3);
    }
    const uint4 *srcB[BR / RQ];
    int swB[BR / RQ];
#pragma unroll
    for (int q = 0; q < BR / RQ; q++) { // B rows: gate rows, then up rows
        const int br = (tid + NTH * q) / SK;
        const uint8_t *base = (GATEUP && br >= ROW_TILE) ? (shared ? a.sb.q : a.b.q) : Ma.q;
        srcB[q] = reinterpret_cast<const uint4 *>(base + ((size_t)e * rows + r0 + br % ROW_TILE) * K * 2);
        swB[q] = p ^ ((br >> 2) & 3);
    }
    auto lds_load = [](const uint4 *src, uint4 *dst_wave) {
        __builtin_amdgcn_global_load_lds(src, (__attribute__((address_space(3))) void *)dst_wave, 16, 0, 0);
    };
    auto issue = [&](int s, uint4 *sA, uint4 *sB) {
#pragma unroll
        for (int q = 0; q < A_SLOTS / NTH; q++) lds_load(srcA[q] + s * SK + swA[q], sA + NTH * q + 64 * wave);
#pragma unroll
        for (int q = 0; q < B_SLOTS / NTH; q++) lds_load(srcB[q] + s * SK + swB[q], sB + NTH * q + 64 * wave);
    };
    auto slot_of = [](int r, int c) { return SK * r + (c ^ ((r >> 2) & 3)); };
    f32x16 acc[2][RB][NB];
#pragma unroll
    for (int tb = 0; tb < 2; tb++)
#pragma unroll
        for (int rb = 0; rb < RB; rb++)
#pragma unroll
            for (int q = 0; q < NB; q++)
#pragma unroll
                for (int j = 0; j < 16; j++) acc[tb][rb][q][j] = 0.0f;
    auto compute = [&](const uint4 *sA, const uint4 *sB) {
#pragma unroll
        for (int ks = 0; ks < SK / 2; ks++) {
            const int c = 2 * ks + kg;
            uint4 xa[2][2], wb[RB][NB];
#pragma unroll
            for (int tb = 0; tb < 2; tb++)
#pragma unroll
                for (int hl = 0; hl < 2; hl++)
                    if (tb ? live1 : live0) xa[tb][hl] = sA[slot_of(hl * TOK_TILE + wt * 64 + tb * 32 + li, c)];
#pragma unroll
            for (int rb = 0; rb < RB; rb++)
#pragma unroll
                for (int q = 0; q < NB; q++) wb[rb][q] = sB[slot_of(q * ROW_TILE + wr * 32 * RB + rb * 32 + li, c)];
            // the halves outermost: consecutive MFMAs feed different
            // accumulators (an MFMA on the accumulator just written waits)
#pragma unroll
            for (int hl = 0; hl < 2; hl++)
#pragma unroll
                for (int tb = 0; tb < 2; tb++)
                    if (tb ? live1 : live0)
#pragma unroll
                    for (int rb = 0; rb < RB; rb++)
#pragma unroll
                        for (int q = 0; q < NB; q++)
                            acc[tb][rb][q] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(
                                as_bf16x8(xa[tb][hl]), as_bf16x8(wb[rb][q]), acc[tb][rb][q], 0, 0, 0);
        }
    };
    // three buffers, loads two stages ahead: stage s is in buffer s % 3
    constexpr int NLD = A_SLOTS / NTH + B_SLOTS / NTH; // loads of a stage, per thread
    // s_waitcnt immediates: vmcnt <= NLD (or 0) and lgkmcnt 0 (this wave's
    // LDS reads of the buffer the next loads overwrite are done)
    constexpr int WAIT_ONE_STAGE = (NLD & 15) | ((NLD >> 4) << 14) | (7 << 4);
    constexpr int WAIT_NONE_LEFT = 7 << 4;
    auto step = [&](int s, const uint4 *__restrict__ cA, const uint4 *__restrict__ cB, uint4 *__restrict__ nA,
                    uint4 *__restrict__ nB) {
        // this thread's loads of stage s are in (stage s + 1's may be in
        // flight); after the barrier every thread's are, and every wave is
        // done with stage s - 1, whose buffer stage s + 2 takes
        if (s + 1 < NS) __builtin_amdgcn_s_waitcnt(WAIT_ONE_STAGE);
        else __builtin_amdgcn_s_waitcnt(WAIT_NONE_LEFT);
        // a raw s_barrier (the compiler's barrier would wait for every load)
        // between compiler fences, so no LDS access moves across it
        asm volatile("" ::: "memory");
        __builtin_amdgcn_s_barrier();
        asm volatile("" ::: "memory");
        if (s + 2 < NS) issue(s + 2, nA, nB);
        compute(cA, cB);
    };
    issue(0, sA0, sB0);
    if (NS > 1) issue(1, sA1, sB1);
    int s = 0;
    for (; s + 3 <= NS; s += 3) {
        step(s, sA0, sB0, sA2, sB2);
        step(s + 1, sA1, sB1, sA0, sB0);
        step(s + 2, sA2, sB2, sA1, sB1);
    }
    if (s < NS) step(s, sA0, sB0, sA2, sB2);
    if (s + 1 < NS) step(s + 1, sA1, sB1, sA0, sB0);
    // the exp table in LDS for the SwiGLU (the tiles are no longer read)
    uint64_t *tab = reinterpret_cast<uint64_t *>(sA0);
    if (GATEUP) {
        __syncthreads();
        if (tid < 32) tab[tid] = exp_tab[tid];
        __syncthreads();
    }
    // D of a 32 x 32 block: lane (li, kg), register j: row (pair) (j / 4) * 8
    // + 4 kg + j % 4, column (weight row) li
#pragma unroll
    for (int tb = 0; tb < 2; tb++)
#pragma unroll
        for (int rb = 0; rb < RB; rb++)
#pragma unroll
            for (int j = 0; j < 16; j++) {
                const int ti = wt * 64 + tb * 32 + (j / 4) * 8 + 4 * kg + (j % 4);
                const int row = r0 + wr * 32 * RB + rb * 32 + li;
                if (ti < cnt) {
                    const float v = GATEUP ? silu_mul_t(acc[tb][rb][0][j], acc[tb][rb][NB - 1][j], tab)
                                           : acc[tb][rb][0][j];
                    a.out[(size_t)(beg + ti) * rows + row] = v;
                }
            }
}

} // namespace

hipError_t launch_split_bf16(const float *x, int rows, int K, void *xh, void *xl, hipStream_t st)
{
    const size_t n = (size_t)rows * (K / 8);
    if (n == 0) return hipSuccess;
    k_split_bf16<<<(unsigned)((n + 255) / 256), 256, 0, st>>>(x, rows, K, static_cast<uint4 *>(xh),
                                                                static_cast<uint4 *>(xl));
    return hipGetLastError();
}

template <bool GATEUP> hipError_t launch_mfma_t(MfArgs a, int routed, int shared, hipStream_t st)
{
    const DevMat &M = routed ? a.a : a.sa;
    if (!routed) a.u_max = 0;
    a.n_sh = shared ? (a.T + a.sh_chunk - 1) / a.sh_chunk : 0;
    const int slots = a.u_max + a.n_sh;
    if (slots == 0) return hipSuccess;
    const int row_tile = 32 * NWR * (GATEUP ? 2 : 4);
    if (M.rows % row_tile) return hipErrorInvalidValue;
    if (a.chunk > TOK_TILE || a.sh_chunk > TOK_TILE) return hipErrorInvalidValue;
    a.n_rt = M.rows / row_tile;
    const dim3 grid((unsigned)((slots + N_XCD - 1) / N_XCD * N_XCD * a.n_rt));
#define BIV_MF_CASE(KK)                                                                                         \
    if (M.cols == KK) {                                                                                         \
        k_mfma_bf16<KK, GATEUP><<<grid, NTH, 0, st>>>(a);                                                       \
        return hipGetLastError();                                                                               \
    }
    BIV_MF_CASE(2048)
    BIV_MF_CASE(1024)
    BIV_MF_CASE(512)
#undef BIV_MF_CASE
    return hipErrorInvalidValue;
}

template <bool GATEUP> hipError_t launch_mfma(const MfArgs &a, hipStream_t st)
{
    // every matrix BF16 (the caller checks); routed and shared in one launch
    // when they share a shape
    const bool has_shared = a.sa.q != nullptr;
    if (has_shared && a.sa.cols == a.a.cols && a.sa.rows == a.a.rows) return launch_mfma_t<GATEUP>(a, 1, 1, st);
    hipError_t err = launch_mfma_t<GATEUP>(a, 1, 0, st);
    if (err != hipSuccess || !has_shared) return err;
    return launch_mfma_t<GATEUP>(a, 0, 1, st);
}

hipError_t launch_mfma_gateup(const MfArgs &a, hipStream_t st) { return launch_mfma<true>(a, st); }
hipError_t launch_mfma_down(const MfArgs &a, hipStream_t st) { return launch_mfma<false>(a, st); }

} // namespace biv
