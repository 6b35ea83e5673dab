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
#include <type_traits>

#include "common.hpp"
#include "expf_ref.h"
#include "layout.hpp"

namespace biv {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int WAVE = 64;
constexpr int N_XCD = 8;

// (slot, row tile) of workgroup b of a grouped launch.  The units (the
// shared expert's slots, then the routed slots in use, row tiles fastest)
// go to the 8 XCDs in runs of RUN slots, run g to XCD g % 8 (workgroup
// ids go round-robin over the XCDs): an expert's consecutive slots, and
// every row tile of a slot, then share one XCD's L2, so that the expert's
// rows come from HBM about once, while runs from all over the dispatch
// order keep the XCDs' loads alike.  (Slots of the BF16 kernel hold up to
// 256 pairs, one expert each as a rule: runs of 1.)  The routed slots in
// use are counted in every used slot record.  False: no unit for this
// workgroup.
constexpr int SLOT_RUN = 4, SLOT_RUN_BF16 = 1;
template <int RUN, class Args> __device__ inline bool slot_unit(const Args &a, int b, int &u, int &rt)
{
    const int used = a.u_max > 0 ? min(a.dp.slots[0].used, a.u_max) : 0;
    const int n = (a.n_sh + used) * a.n_rt, run = RUN * a.n_rt;
    const int x = b % N_XCD, i = b / N_XCD;
    const int unit = (x + N_XCD * (i / run)) * run + i % run;
    if (unit >= n) return false;
    u = unit / a.n_rt;
    rt = unit % a.n_rt;
    return true;
}
// workgroups of a grouped launch over `slots` slots (an upper bound) of
// n_rt row tiles: every XCD's share of the runs
template <int RUN> inline unsigned slot_grid(int slots, int n_rt)
{
    const int runs = (slots + RUN - 1) / RUN;
    return (unsigned)(N_XCD * ((runs + N_XCD - 1) / N_XCD) * RUN * n_rt);
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
        bf16_split(v, &h[m], &lo[m]);
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
// The row tiles of a slot go to one XCD (slot_unit): the slot's activation
// rows come from HBM once per slot and from that XCD's L2 after, and every
// expert's weights are read once per slot.
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
    // separate arrays: the compiler then tells the buffers a DMA writes apart
    // (one array would make it wait for every DMA before each LDS read)
    __shared__ uint4 sA0[A_SLOTS], sA1[A_SLOTS], sA2[A_SLOTS], sB0[B_SLOTS], sB1[B_SLOTS], sB2[B_SLOTS];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int li = lane & 31, kg = lane >> 5;
    // the two waves of a SIMD (waves w and w + 4) take pairs 64 apart x 2
    const int wt = wave >> 1, wr = wave & 1;
    // workgroup -> (slot, row tile): ids b with one b % 8 are one XCD's
    int u, rt;
    if (!slot_unit<SLOT_RUN_BF16>(a, blockIdx.x, u, rt)) return;
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
    // A load q of a thread covers pairs 128 (q & 1) .. + 127 of half q >> 1
    // (for every wave alike): a slot of at most 128 pairs (HALF) leaves out
    // the odd ones, which would only load its last pair again.  (Leaving out
    // each wave's loads that hold no pair of the slot, down to all of them,
    // measured no faster.)
    static_assert(A_SLOTS / NTH == 4 && NTH / SK == 128, "A loads by pair halves");
    auto issue = [&](int s, uint4 *sA, uint4 *sB, auto half_c) {
        constexpr bool HALF = decltype(half_c)::value;
#pragma unroll
        for (int q = 0; q < A_SLOTS / NTH; q++)
            if (!HALF || !(q & 1)) lds_load(srcA[q] + s * SK + swA[q], sA + NTH * q + 64 * wave);
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
                            acc[tb][rb][q] = GATEUP ? __builtin_amdgcn_mfma_f32_32x32x16_bf16(
                                                          as_bf16x8(wb[rb][q]), as_bf16x8(xa[tb][hl]), acc[tb][rb][q], 0, 0, 0)
                                                    : __builtin_amdgcn_mfma_f32_32x32x16_bf16(
                                                          as_bf16x8(xa[tb][hl]), as_bf16x8(wb[rb][q]), acc[tb][rb][q], 0, 0, 0);
        }
    };
    // three buffers, loads two stages ahead: stage s is in buffer s % 3
    auto run = [&](auto half_c) {
        constexpr bool HALF = decltype(half_c)::value;
        // loads of a stage, per thread
        constexpr int NLD = (HALF ? A_SLOTS / NTH / 2 : A_SLOTS / NTH) + B_SLOTS / NTH;
        // s_waitcnt immediates: vmcnt <= NLD (or 0) and lgkmcnt 0 (this
        // wave's LDS reads of the buffer the next loads overwrite are done)
        constexpr int WAIT_ONE_STAGE = (NLD & 15) | ((NLD >> 4) << 14) | (7 << 4);
        constexpr int WAIT_NONE_LEFT = 7 << 4;
        auto step = [&](int s, const uint4 *__restrict__ cA, const uint4 *__restrict__ cB, uint4 *__restrict__ nA,
                        uint4 *__restrict__ nB) {
            // this thread's loads of stage s are in (stage s + 1's may be in
            // flight); after the barrier every thread's are, and every wave
            // is done with stage s - 1, whose buffer stage s + 2 takes
            if (s + 1 < NS) __builtin_amdgcn_s_waitcnt(WAIT_ONE_STAGE);
            else __builtin_amdgcn_s_waitcnt(WAIT_NONE_LEFT);
            // a raw s_barrier (the compiler's barrier would wait for every
            // load) between compiler fences, so no LDS access moves across it
            asm volatile("" ::: "memory");
            __builtin_amdgcn_s_barrier();
            asm volatile("" ::: "memory");
            if (s + 2 < NS) issue(s + 2, nA, nB, half_c);
            compute(cA, cB);
        };
        issue(0, sA0, sB0, half_c);
        if (NS > 1) issue(1, sA1, sB1, half_c);
        int s = 0;
        for (; s + 3 <= NS; s += 3) {
            step(s, sA0, sB0, sA2, sB2);
            step(s + 1, sA1, sB1, sA0, sB0);
            step(s + 2, sA2, sB2, sA1, sB1);
        }
        if (s < NS) step(s, sA0, sB0, sA2, sB2);
        if (s + 1 < NS) step(s + 1, sA1, sB1, sA0, sB0);
    };
    // uniform over the workgroup (compute reads only the pairs below cnt)
    if (cnt <= TOK_TILE / 2) run(std::true_type());
    else run(std::false_type());
    // the exp table in LDS for the SwiGLU
    __shared__ uint64_t tab[GATEUP ? 32 : 1];
    if (GATEUP) {
        if (tid < 32) tab[tid] = exp_tab[tid];
        __syncthreads(); // (also: every wave is done with the ring)
    }
    // D of a 32 x 32 block.  gate/up (weights as A, the pairs as B): lane
    // (li, kg), registers 4 q .. 4 q + 3: weight rows 8 q + 4 kg .. 8 q + 4 kg
    // + 3 of the block, pair li: four consecutive outputs, one 16-byte store.
    // down (the pairs as A): register j is pair 8 (j / 4) + 4 kg + j % 4,
    // weight row li: a half wave stores 32 consecutive outputs (down's large
    // output keeps whole 128-byte segments that way; 16-byte stores across 32
    // rows measured slower)
    if constexpr (GATEUP) if (a.xo_h) {
        // the intermediate's bf16 hi / lo halves in the chunk order, as
        // k_split_bf16 forms them: the tile's SwiGLU values [pair][row]
        // through LDS (the ring's buffers, PA pairs' rows in each A buffer
        // and PB in each B buffer, EP floats apart), then 16-byte chunks:
        // this row tile is elements 128 rt .. 128 rt + 127 of each row, so
        // chunk 16 rt + L holds its rows 16 m + L
        constexpr int EP = 136, PA = A_SLOTS * 4 / EP, PB = B_SLOTS * 4 / EP;
        static_assert(ROW_TILE == 128, "one 128-element span per row tile");
        static_assert(3 * (PA + PB) >= TOK_TILE, "the tile fits in the ring");
        auto trow = [&](int p) -> float * {
            if (p < 3 * PA) {
                const int i = p / PA;
                return reinterpret_cast<float *>(i == 0 ? sA0 : i == 1 ? sA1 : sA2) + (p - PA * i) * EP;
            }
            const int i = (p - 3 * PA) / PB;
            return reinterpret_cast<float *>(i == 0 ? sB0 : i == 1 ? sB1 : sB2) + (p - 3 * PA - PB * i) * EP;
        };
#pragma unroll
        for (int tb = 0; tb < 2; tb++)
            if (tb ? live1 : live0)
#pragma unroll
                for (int rb = 0; rb < RB; rb++)
#pragma unroll
                    for (int q = 0; q < 4; q++) {
                        float4 v;
                        v.x = silu_mul_t(acc[tb][rb][0][4 * q], acc[tb][rb][NB - 1][4 * q], tab);
                        v.y = silu_mul_t(acc[tb][rb][0][4 * q + 1], acc[tb][rb][NB - 1][4 * q + 1], tab);
                        v.z = silu_mul_t(acc[tb][rb][0][4 * q + 2], acc[tb][rb][NB - 1][4 * q + 2], tab);
                        v.w = silu_mul_t(acc[tb][rb][0][4 * q + 3], acc[tb][rb][NB - 1][4 * q + 3], tab);
                        *reinterpret_cast<float4 *>(trow(wt * 64 + tb * 32 + li) + wr * 32 * RB + rb * 32 + 8 * q +
                                                    4 * kg) = v;
                    }
        __syncthreads();
        const int nc = rows / 8;
        for (int x = tid; x < cnt * 16; x += NTH) {
            const int p = x >> 4, L = x & 15;
            uint32_t h[8], lo[8];
#pragma unroll
            for (int m = 0; m < 8; m++) {
                const float v = trow(p)[16 * m + L];
                bf16_split(v, &h[m], &lo[m]);
            }
            const size_t c = (size_t)(beg + p) * nc + 16 * rt + L;
            a.xo_h[c] = make_uint4(h[0] | h[1] << 16, h[2] | h[3] << 16, h[4] | h[5] << 16, h[6] | h[7] << 16);
            a.xo_l[c] = make_uint4(lo[0] | lo[1] << 16, lo[2] | lo[3] << 16, lo[4] | lo[5] << 16, lo[6] | lo[7] << 16);
        }
        return;
    }
    if constexpr (GATEUP) {
#pragma unroll
        for (int tb = 0; tb < 2; tb++) {
            const int ti = wt * 64 + tb * 32 + li;
            if (ti < cnt)
#pragma unroll
                for (int rb = 0; rb < RB; rb++)
#pragma unroll
                    for (int q = 0; q < 4; q++) {
                        const int row = r0 + wr * 32 * RB + rb * 32 + 8 * q + 4 * kg;
                        float4 v;
                        v.x = silu_mul_t(acc[tb][rb][0][4 * q], acc[tb][rb][NB - 1][4 * q], tab);
                        v.y = silu_mul_t(acc[tb][rb][0][4 * q + 1], acc[tb][rb][NB - 1][4 * q + 1], tab);
                        v.z = silu_mul_t(acc[tb][rb][0][4 * q + 2], acc[tb][rb][NB - 1][4 * q + 2], tab);
                        v.w = silu_mul_t(acc[tb][rb][0][4 * q + 3], acc[tb][rb][NB - 1][4 * q + 3], tab);
                        *reinterpret_cast<float4 *>(a.out + (size_t)(beg + ti) * rows + row) = v;
                    }
        }
    } else {
        // pair ti's row starts (beg + ti) * rows floats in: one 64-bit base
        // per pair block and 32-bit offsets (j / 4) * 8 rows + (j % 4) rows,
        // not a 64-bit multiply per store
        const int r1 = rows, r8 = 8 * rows;
#pragma unroll
        for (int tb = 0; tb < 2; tb++) {
            const int t0 = wt * 64 + tb * 32 + 4 * kg;
            float *ob = a.out + (size_t)(beg + t0) * rows + r0 + wr * 32 * RB + li;
#pragma unroll
            for (int rb = 0; rb < RB; rb++)
#pragma unroll
                for (int j = 0; j < 16; j++) {
                    const int dt = (j / 4) * 8 + (j % 4);
                    if (t0 + dt < cnt) ob[(j / 4) * r8 + (j % 4) * r1 + rb * 32] = acc[tb][rb][0][j];
                }
        }
    }
}


// ---------------------------------------------------------------------------
// Q8_0 down matrices at prefill sizes on the int8 matrix cores.
//
// biv's dot_q8_0 (quant.rs:599-607, x86 1368-1382) sums, per row and input
// row, f16(d_w) * d_x * idot over the 32-element blocks, idot the exact int32
// dot of the block's int8 quants.  v_mfma_i32_16x16x32_i8 computes exactly
// those int32 block dots for 16 rows x 16 pairs at once (one block per
// instruction, so the dots stay apart); the scaling and the sum over blocks
// run in f32 on the vector ALU, in an order of their own.  Only the down
// matrices run here: their outputs go straight to the combine, so the other
// order moves them by rounding only.  gate/up outputs are quantised again
// (the down input), where a rounding difference can move a quant by one
// step; gate/up therefore keeps the x86 order (the chain kernels).
//
// Operands: a block's 32 quants as lanes (x, kq) see them, kq = 0..3 taking
// bytes 8 kq .. 8 kq + 7, for weights and activations alike.  In the chain
// layout (layout.hpp) the 16-byte unit 16 g + 8 pi + w of a row holds word w
// of the blocks 8 g + pi + 2 j, j = 0..3, so lane kq loads units 2 kq and
// 2 kq + 1 of each parity (32 contiguous bytes) and finds its 8 bytes of
// block j in word j of the two.
//
// A workgroup takes a slot (up to QT pairs, staged in LDS: quants and block
// scales) and QW waves of QR rows each; a wave streams its rows' blocks from
// HBM half a group (4 blocks of each row) ahead.  D of an MFMA: lane (n, kq)
// holds row n, pairs 4 kq .. 4 kq + 3 of the 16-pair tile.
constexpr int QW = 8;            // waves of a workgroup
constexpr int QT = MFMA_Q8_TILE; // pairs of a slot
constexpr int NTT = QT / 16;     // 16-pair tiles of a slot
constexpr int QNTH = QW * 64;
constexpr int QRT = 2;           // 16-row tiles of a wave
constexpr int Q_ROWS_WG = QW * 16 * QRT;

typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

// Four small integers as four exact f16 (two dwords).  Each byte u (0..255)
// becomes the f16 with bits 0x64uu, i.e. 1024 + u, and BIAS is taken off
// (exact: every value is an integer below 2048).  Signed int8 quants come
// in as q ^ 0x80 = q + 128 with BIAS 1152; nibbles 0..15 with BIAS 1024.
template <int BIAS> __device__ __forceinline__ uint2 bytes_to_f16x4(uint32_t u)
{
    const uint32_t r0 = __builtin_amdgcn_perm(0x64646464u, u, 0x04010400u);
    const uint32_t r1 = __builtin_amdgcn_perm(0x64646464u, u, 0x04030402u);
    const f16x2 bias = {(_Float16)BIAS, (_Float16)BIAS};
    const f16x2 h0 = __builtin_bit_cast(f16x2, r0) - bias, h1 = __builtin_bit_cast(f16x2, r1) - bias;
    return make_uint2(__builtin_bit_cast(uint32_t, h0), __builtin_bit_cast(uint32_t, h1));
}
__device__ __forceinline__ uint2 i8x4_to_f16x4(uint32_t q) { return bytes_to_f16x4<1152>(q ^ 0x80808080u); }

__device__ inline float f16_to_f32(uint32_t h) { return (float)__builtin_bit_cast(_Float16, (uint16_t)h); }

// byte i (0..15) of a 16-byte vector
__device__ inline int byte_at4(const int4 &v, int i)
{
    const int w = i < 4 ? v.x : i < 8 ? v.y : i < 12 ? v.z : v.w;
    return ((unsigned)w >> (8 * (i & 3))) & 0xFF;
}

template <int K, bool DUMP>
__global__ __launch_bounds__(QNTH) void k_q8_down_mfma(MvArgs a)
{
    constexpr int RT = QRT;
    constexpr int NG = K / 256; // groups of 8 blocks
    constexpr int NB = K / 32;
    constexpr int XSTR = K / 16 + 1; // staged quant row: 16-byte units (+1 against bank conflicts)
    constexpr int DSTR = QT + 4;     // staged scales [block][pair], floats
    __shared__ uint4 xq_s[QT * XSTR];
    __shared__ float xd_s[NB * DSTR];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int n = lane & 15, kq = lane >> 4;
    int u, rt;
    if (!slot_unit<SLOT_RUN>(a, blockIdx.x, u, rt)) return;
    const bool shared = u < a.n_sh;
    int e = 0, beg, cnt;
    if (shared) {
        const int tok0 = u * a.sh_chunk;
        beg = a.P + tok0;
        cnt = min(a.sh_chunk, a.T - tok0);
    } else {
        const Slot sl = a.dp.slots[u - a.n_sh];
        if (sl.cnt == 0) return; // uniform over the workgroup
        e = sl.expert;
        beg = sl.beg;
        cnt = sl.cnt;
    }
    const DevMat &M = shared ? a.sa : a.a;
    const int rows = M.rows;
    // the weight rows of this lane: row n of each 16-row tile
    const int rw0 = rt * Q_ROWS_WG + wave * 16 * RT;
    const uint4 *wq[RT];
    const uint2 *wsc[RT];
#pragma unroll
    for (int r = 0; r < RT; r++) {
        const size_t row = (size_t)e * rows + rw0 + 16 * r + n;
        wq[r] = reinterpret_cast<const uint4 *>(M.q + row * K) + 2 * kq;
        wsc[r] = reinterpret_cast<const uint2 *>(M.s + row * NB * 2);
    }
    // half-group h = (g, pi)'s weights: per tile two units of quants and 4
    // f16 scales (blocks 8 g + pi + 2 j)
    struct Half {
        uint4 q[RT][2];
        uint2 s[RT];
    };
    auto load = [&](int h, Half &w) {
        const int g = h >> 1, pi = h & 1;
#pragma unroll
        for (int r = 0; r < RT; r++) {
            w.q[r][0] = wq[r][16 * g + 8 * pi];
            w.q[r][1] = wq[r][16 * g + 8 * pi + 1];
            w.s[r] = wsc[r][(pi * (K / 64) + 4 * g) / 4];
        }
    };
    Half w0, w1;
    load(0, w0); // the first weights go out before the staging waits
    // stage the slot's input rows: quants (chain layout, row stride XSTR
    // units) and block scales transposed to [block][pair]; pairs past the
    // count repeat the last one (their results are not stored)
    {
        constexpr int UPR = K / 16; // units per row
        static_assert((QT * UPR) % QNTH == 0, "staging shape");
#pragma unroll
        for (int it = 0; it < QT * UPR / QNTH; it++) {
            const int idx = tid + QNTH * it, i = idx / UPR, c = idx % UPR;
            const size_t ar = beg + min(i, cnt - 1);
            xq_s[i * XSTR + c] = reinterpret_cast<const uint4 *>(a.xq + ar * K)[c];
        }
        for (int idx = tid; idx < QT * NB; idx += QNTH) {
            const int i = idx / NB, bs = idx % NB;
            const size_t ar = beg + min(i, cnt - 1);
            const int b = 2 * (bs % (K / 64)) + bs / (K / 64); // lay::q8_scale's inverse
            xd_s[b * DSTR + i] = a.xd[ar * NB + bs];
        }
    }
    __syncthreads();
    float acc[NTT][RT][4];
#pragma unroll
    for (int t = 0; t < NTT; t++)
#pragma unroll
        for (int r = 0; r < RT; r++)
#pragma unroll
            for (int j = 0; j < 4; j++) acc[t][r][j] = 0.0f;
    auto compute = [&](int h, const Half &w) {
        const int g = h >> 1, pi = h & 1;
#pragma unroll
        for (int t = 0; t < NTT; t++) {
            if (16 * t >= cnt) break; // uniform: no pairs in this tile
            // this lane's activation units of the half-group
            const uint4 *xr = xq_s + (16 * t + n) * XSTR + 16 * g + 8 * pi + 2 * kq;
            const uint4 x0 = xr[0], x1 = xr[1];
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const int b = 8 * g + pi + 2 * j;
                const float4 dx = *reinterpret_cast<const float4 *>(xd_s + b * DSTR + 16 * t + 4 * kq);
                const long xo = (long)((uint64_t)x0[j] | (uint64_t)x1[j] << 32);
#pragma unroll
                for (int r = 0; r < RT; r++) {
                    const uint32_t h2 = j < 2 ? w.s[r].x : w.s[r].y;
                    const float dw = f16_to_f32((j & 1) ? h2 >> 16 : h2 & 0xFFFF);
                    const long wo = (long)((uint64_t)w.q[r][0][j] | (uint64_t)w.q[r][1][j] << 32);
                    const i32x4 z = {0, 0, 0, 0};
                    const i32x4 d = __builtin_amdgcn_mfma_i32_16x16x32_i8(xo, wo, z, 0, 0, 0);
                    acc[t][r][0] = __builtin_fmaf((float)d[0], dx.x * dw, acc[t][r][0]);
                    acc[t][r][1] = __builtin_fmaf((float)d[1], dx.y * dw, acc[t][r][1]);
                    acc[t][r][2] = __builtin_fmaf((float)d[2], dx.z * dw, acc[t][r][2]);
                    acc[t][r][3] = __builtin_fmaf((float)d[3], dx.w * dw, acc[t][r][3]);
                    if (DUMP && a.dump_a) { // the block dots, for the taps
#pragma unroll
                        for (int jj = 0; jj < 4; jj++) {
                            const int i = 16 * t + 4 * kq + jj;
                            if (i < cnt) a.dump_a[((size_t)(beg + i) * rows + rw0 + 16 * r + n) * NB + b] = d[jj];
                        }
                    }
                }
                // keep each block's MFMA results short-lived (registers for
                // more waves rather than for MFMAs in flight)
                __builtin_amdgcn_sched_barrier(0);
            }
        }
    };
    // two half-groups per turn, loads one ahead
    for (int h = 0; h < 2 * NG; h += 2) {
        load(h + 1, w1);
        compute(h, w0);
        if (h + 2 < 2 * NG) load(h + 2, w0);
        compute(h + 1, w1);
    }
    // pair 16 t + 4 kq + j of the slot, row rw0 + 16 r + n
#pragma unroll
    for (int t = 0; t < NTT; t++)
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const int i = 16 * t + 4 * kq + j;
            if (i < cnt) {
#pragma unroll
                for (int r = 0; r < RT; r++) a.out[(size_t)(beg + i) * rows + rw0 + 16 * r + n] = acc[t][r][j];
            }
        }
}


// ---------------------------------------------------------------------------
// Q8_0 and Q4_K gate/up at prefill sizes, bit for bit in the x86 order, with
// the integer work on the matrix cores.
//
// biv's x86 dot_q8_0 and dot_q4k (quant.rs:1368-1423) keep 16 f32 chains per
// row: chain (pi, l) takes the 32-element blocks b = pi, pi + 2, ... and for
// each the int32 of the block's word l (bytes 4l..4l+3: a 4-element dot),
// fma(float(word dot), w_scale(b) * d_x(b), acc); then the chains are summed
// in a fixed tree, and Q4_K subtracts its mins term last (the chain kernels
// in kernels.hip do exactly this on the vector ALU).  Here
// v_mfma_f32_32x32x16_f16 produces the word dots, already as f32, 1024 per
// instruction: K = 16 is half a block (words 4 hh .. 4 hh + 3); the A
// operand holds 8 input rows, each four times, A row 4 t + w keeping only
// word 4 hh + w of input row t (the other 12 of its 16 values are zero); the
// B operand holds 32 weight rows (16 rows of gate, then the same 16 of up).
// Both hold the quants (Q4_K: nibbles 0..15) as f16, exact for integers
// this small; every product is exact and every partial sum an integer below
// 2^17, so D row 4 t + w, column n is the word dot of input row t and weight
// row n, exactly, and equal to the reference's float(int32 word dot).  The
// vector ALU does what remains, in the reference's order: fma into the
// chain, the tree, the mins, the SwiGLU.
//
// D of the MFMA: lane (n, kg) (n = lane % 32, kg = lane / 32) holds column n
// and rows 8 q + 4 kg + r (q, r = 0..3), i.e. words 4 hh + r of input rows
// 2 q + kg: so a lane ends up holding all 16 chains of 4 input rows of its
// 8-row tile with weight row n, and the tree runs within the lane.
//
// A workgroup takes a slot (up to QT = 16 pairs, staged in LDS as f16 words:
// two 8-row tiles) and 4 waves of 16 output rows; a wave streams its 32
// weight rows one step ahead and keeps the chains of the slot's pairs in
// registers (2 tiles x 4 rows x 16 chains).  The weight operands are
// converted to f16 once per half block and meet both tiles.
constexpr int GW = 4;               // waves of a workgroup
constexpr int GNTH = GW * 64;
constexpr int G_ROWS_WG = GW * 16;  // output rows of a workgroup
constexpr int GNT = QT / 8;         // 8-row tiles of a slot
#ifndef GU_AJ
#define GU_AJ 2 // blocks per masked A read group
#endif

// Weight operands of the exact kernel.  A step covers the blocks 8 g + pi +
// 2 j (j = 0..3) of one parity (Q8_0: a half-group) or both parities (Q4_K:
// super-block g, whose nibble bytes serve both).  Lane kg of a column takes
// words 2 kg, 2 kg + 1 (half 0) and 4 + 2 kg, 5 + 2 kg (half 1) of each
// block.  operand(w, pi, j, hh) is its 8 quants of half hh of block
// 8 g + pi + 2 j as exact f16; scale(w, pi, j) the block's f32 weight scale
// as the reference forms it.
template <int TY, int K> struct GuW;

// Q8_0 (chain layout: unit 16 g + 8 pi + w holds word w of the blocks
// 8 g + pi + 2 j); scale f16(d) (quant.rs:1368-1382)
template <int K> struct GuW<T_Q8_0, K> {
    static constexpr int STEPS = K / 128; // half-groups
    static constexpr bool BOTH = false;  // a step is one parity
    struct Step {
        uint4 q[4]; // units 2 kg, 2 kg + 1, 4 + 2 kg, 5 + 2 kg of the half-group
        uint2 s;
    };
    const uint4 *wq;
    const uint2 *wsc;
    __device__ GuW(const uint8_t *q, const uint8_t *s, size_t row, int kg)
        : wq(reinterpret_cast<const uint4 *>(q + row * K) + 2 * kg),
          wsc(reinterpret_cast<const uint2 *>(s + row * (K / 32) * 2)) {}
    __device__ void load(int h, Step &w) const
    {
        const int g = h >> 1, pi = h & 1;
        const uint4 *p = wq + 16 * g + 8 * pi;
        w.q[0] = p[0];
        w.q[1] = p[1];
        w.q[2] = p[4];
        w.q[3] = p[5];
        w.s = wsc[(pi * (K / 64) + 4 * g) / 4];
    }
    __device__ static f16x8 operand(const Step &w, int pi, int j, int hh)
    {
        const uint2 lo = i8x4_to_f16x4(w.q[2 * hh][j]), hi = i8x4_to_f16x4(w.q[2 * hh + 1][j]);
        return __builtin_bit_cast(f16x8, make_uint4(lo.x, lo.y, hi.x, hi.y));
    }
    __device__ static float scale(const Step &w, int pi, int j)
    {
        const uint32_t h2 = j < 2 ? w.s.x : w.s.y;
        return f16_to_f32((j & 1) ? h2 >> 16 : h2 & 0xFFFF);
    }
};

// Q4_K (chain layout: unit 8 g + w holds word w of the four sub-block pairs
// of super-block g, low nibbles the even sub-block, high the odd); scale
// d * sc of the sub-block, the mins apart (quant.rs:1384-1423)
template <int K> struct GuW<T_Q4K, K> {
    static constexpr int STEPS = K / 256; // super-blocks
    static constexpr bool BOTH = true;
    struct Step {
        uint4 q[4];
        int4 hd; // d, dmin, the 12 scale bytes
    };
    const uint4 *wq;
    const int4 *whd;
    __device__ GuW(const uint8_t *q, const uint8_t *s, size_t row, int kg)
        : wq(reinterpret_cast<const uint4 *>(q + row * (K / 2)) + 2 * kg),
          whd(reinterpret_cast<const int4 *>(s + row * (K / 256) * 16)) {}
    __device__ void load(int g, Step &w) const
    {
        const uint4 *p = wq + 8 * g;
        w.q[0] = p[0];
        w.q[1] = p[1];
        w.q[2] = p[4];
        w.q[3] = p[5];
        w.hd = whd[g];
    }
    __device__ static f16x8 operand(const Step &w, int pi, int j, int hh)
    {
        const uint2 lo = bytes_to_f16x4<1024>((w.q[2 * hh][j] >> (4 * pi)) & 0x0F0F0F0Fu);
        const uint2 hi = bytes_to_f16x4<1024>((w.q[2 * hh + 1][j] >> (4 * pi)) & 0x0F0F0F0Fu);
        return __builtin_bit_cast(f16x8, make_uint4(lo.x, lo.y, hi.x, hi.y));
    }
    __device__ static float scale(const Step &w, int pi, int j)
    {
        const int sb = 2 * j + pi;
        const int sc = sb < 4 ? byte_at4(w.hd, 4 + sb) & 63
                              : (byte_at4(w.hd, 4 + sb + 4) & 0xF) | ((byte_at4(w.hd, 4 + sb - 4) >> 6) << 4);
        const float d = f16_to_f32((uint32_t)w.hd.x & 0xFFFF);
        return d * (float)sc;
    }
};

// two workgroups per CU (LDS: 70 KB each at K = 2048), two waves per SIMD
template <int TY, int K, bool DUMP>
__global__ __launch_bounds__(GNTH) __attribute__((amdgpu_waves_per_eu(DUMP ? 1 : 2))) void k_gu_exact(MvArgs a)
{
    using W = GuW<TY, K>;
    constexpr int NB = K / 32;
    constexpr bool Q4K = TY == T_Q4K;
    // The input rows' words as exact f16: word l of block b of input row i
    // (four values, 8 bytes) at xop_s[i * XRS + 8 b + l].  Rows are 32 bytes
    // more than their words apart: the 16 lanes of a masked read (rows 0..7,
    // two words) then fall in distinct banks.
    constexpr int XRS = NB * 8 + 4;
    // Block scales of the input rows, [q8_scale order][tile][kg][q] for row
    // 8 tile + 2 q + kg: a lane's four rows in one 16-byte read.
    constexpr int DSTR = QT + 4;
    constexpr int SSTR = NB + 4; // Q4_K block sums [row][q8_scale order]
    __shared__ uint2 xop_s[QT * XRS];
    __shared__ float xd_s[NB * DSTR];
    __shared__ float xs_s[Q4K ? QT * SSTR : 1];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int li = lane & 31, kg = lane >> 5;
    int u, rt;
    if (!slot_unit<SLOT_RUN>(a, blockIdx.x, u, rt)) return;
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
    const DevMat &M = shared ? a.sa : a.a;
    const DevMat &B = shared ? a.sb : a.b;
    const int rows = M.rows;
    // this lane's weight row: column li of the MFMA tile, gate rows then up
    const int orow = rt * G_ROWS_WG + wave * 16 + (li & 15);
    const size_t wr = (size_t)e * rows + orow;
    const W wsrc(li < 16 ? M.q : B.q, li < 16 ? M.s : B.s, wr, kg);
    typename W::Step w0;
    wsrc.load(0, w0); // the first weights go out before the staging waits
    // stage the slot's input rows: f16 words (from the chain layout: unit
    // 16 g + 8 pi + l holds word l of blocks 8 g + pi + 2 j), block scales
    // (and Q4_K's block sums); rows past the count repeat the last one (their
    // results are not stored)
    {
        constexpr int UPR = K / 16; // units per row
        for (int idx = tid; idx < QT * UPR; idx += GNTH) {
            const int i = idx / UPR, c = idx % UPR;
            const int ti = min(i, cnt - 1);
            const size_t ar = shared ? (size_t)(tok0 + ti) : (size_t)a.dp.pair_tok[beg + ti];
            const uint4 v = reinterpret_cast<const uint4 *>(a.xq + ar * K)[c];
            const int g = c >> 4, pi = (c >> 3) & 1, l = c & 7;
#pragma unroll
            for (int j = 0; j < 4; j++) xop_s[i * XRS + (8 * g + pi + 2 * j) * 8 + l] = i8x4_to_f16x4(v[j]);
        }
        for (int idx = tid; idx < QT * NB; idx += GNTH) {
            const int i = idx / NB, bs = idx % NB;
            const int ti = min(i, cnt - 1);
            const size_t ar = shared ? (size_t)(tok0 + ti) : (size_t)a.dp.pair_tok[beg + ti];
            xd_s[bs * DSTR + (i >> 3) * 8 + (i & 1) * 4 + ((i & 7) >> 1)] = a.xd[ar * NB + bs];
            if (Q4K) xs_s[i * SSTR + bs] = a.xs[ar * NB + bs];
        }
    }
    __syncthreads();
    // Q4_K's mins, per (input row, weight row): the sum over super-blocks
    // and sub-block pairs, in that order, of dmin * (m_a * s_a + m_b * s_b)
    // (the chain kernels' q4k_mins), s the input row's block sums; super-
    // blocks outermost so that each header is decoded once for all rows.
    // Formed before the chains, while their registers are free.
    float mins[GNT][4];
#pragma unroll
    for (int t = 0; t < GNT; t++)
#pragma unroll
        for (int q = 0; q < 4; q++) mins[t][q] = 0.0f;
    if constexpr (Q4K) {
        const int4 *hd = reinterpret_cast<const int4 *>((li < 16 ? M.s : B.s) + wr * (K / 256) * 16);
#pragma unroll 1
        for (int sbk = 0; sbk < K / 256; sbk++) {
            const int4 h = hd[sbk];
            const float dmin = f16_to_f32((uint32_t)h.x >> 16);
            float mf[8];
#pragma unroll
            for (int sb = 0; sb < 8; sb++)
                mf[sb] = (float)(sb < 4 ? byte_at4(h, 4 + sb + 4) & 63
                                        : (byte_at4(h, 4 + sb + 4) >> 4) | ((byte_at4(h, 4 + sb) >> 6) << 4));
#pragma unroll
            for (int t = 0; t < GNT; t++)
#pragma unroll
                for (int q = 0; q < 4; q++) {
                    const float *sr = xs_s + (8 * t + 2 * q + kg) * SSTR;
#pragma unroll
                    for (int j = 0; j < 4; j++) {
                        const int s2 = 4 * sbk + j;
                        mins[t][q] = mins[t][q] + dmin * (mf[2 * j] * sr[lay::q8_scale(K, 2 * s2)] +
                                                          mf[2 * j + 1] * sr[lay::q8_scale(K, 2 * s2 + 1)]);
                    }
                }
        }
    }
    // The A operand: A row li = 4 t + w keeps word 4 hh + w of input row t,
    // which lane kg = w / 2 holds in its low half (w even) or high half (w
    // odd); every other half of every lane is zero.  The registers start at
    // zero and the lanes load only their own half (reads under an exec mask,
    // ANDed with the current exec), so the zeros stay and no lane reads LDS
    // for them.
    const int at = li >> 2, aw = li & 3;
    const bool mine = (aw >> 1) == kg;
    const uint64_t mlo = __ballot(mine && !(aw & 1)), mhi = __ballot(mine && (aw & 1));
    const uint32_t xa0 = (uint32_t)reinterpret_cast<uintptr_t>(xop_s + at * XRS + aw);
    constexpr int TO = 8 * XRS * 8; // bytes from tile to tile
    static_assert(TO * (GNT - 1) + 160 < 65536, "ds_read offsets are 16-bit");
    static_assert(GNT == 2, "two tiles");
    // The chains and everything after, for NT 8-row tiles: a slot of at most
    // 8 pairs takes one tile (no MFMAs or FMAs for rows that do not exist).
    auto run = [&](auto nt_c) {
        constexpr int NT = decltype(nt_c)::value;
        constexpr int NM = 2 * NT; // MFMAs per block: (half, tile), half-major
        uint64_t alo[GU_AJ * NM], ahi[GU_AJ * NM]; // [block of the read group][half][tile]
#pragma unroll
        for (int i = 0; i < GU_AJ * NM; i++) alo[i] = ahi[i] = 0ull;
        // chains acc[tile][q][pi][l] of input row 8 tile + 2 q + kg, weight row li
        float acc[NT][4][2][8];
#pragma unroll
        for (int t = 0; t < NT; t++)
#pragma unroll
            for (int q = 0; q < 4; q++)
#pragma unroll
                for (int pi = 0; pi < 2; pi++)
#pragma unroll
                    for (int l = 0; l < 8; l++) acc[t][q][pi][l] = 0.0f;
        // the blocks 8 g + pi + 2 j, j = 0..3, of parity pi (a compile-time
        // constant: it picks the chain accumulators)
        auto compute = [&](int g, auto pi_c, const typename W::Step &w) {
            constexpr int pi = decltype(pi_c)::value;
            f16x8 wo_next;      // block j + 1's first operand, formed during block j
            float sb_next[4];   // (Q8_0, two tiles) block j + 1's tile-0 scales, likewise
            float4 dx_next;
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const int b = 8 * g + pi + 2 * j;
                // A: both halves of each tile of GU_AJ blocks (this one and
                // the next ones of the parity, 128 bytes apart), low words
                // under one mask, high under the other, exec restored, then a
                // wait for them (in the same statement: the compiler takes an
                // asm's outputs as ready when it ends, and may copy them
                // right after)
                if (j % GU_AJ == 0) {
                    const uint32_t xa = xa0 + b * 64;
                    uint64_t ex;
                    if constexpr (NT == 2 && GU_AJ == 2) {
                        asm volatile("s_mov_b64 %0, exec\n\ts_and_b64 exec, %17, %0\n\t"
                                     "ds_read_b64 %1, %19\n\t"
                                     "ds_read_b64 %2, %19 offset:%20\n\t"
                                     "ds_read_b64 %3, %19 offset:32\n\t"
                                     "ds_read_b64 %4, %19 offset:%21\n\t"
                                     "ds_read_b64 %5, %19 offset:128\n\t"
                                     "ds_read_b64 %6, %19 offset:%22\n\t"
                                     "ds_read_b64 %7, %19 offset:160\n\t"
                                     "ds_read_b64 %8, %19 offset:%23\n\t"
                                     "s_and_b64 exec, %18, %0\n\t"
                                     "ds_read_b64 %9, %19\n\t"
                                     "ds_read_b64 %10, %19 offset:%20\n\t"
                                     "ds_read_b64 %11, %19 offset:32\n\t"
                                     "ds_read_b64 %12, %19 offset:%21\n\t"
                                     "ds_read_b64 %13, %19 offset:128\n\t"
                                     "ds_read_b64 %14, %19 offset:%22\n\t"
                                     "ds_read_b64 %15, %19 offset:160\n\t"
                                     "ds_read_b64 %16, %19 offset:%23\n\t"
                                     "s_mov_b64 exec, %0\n\ts_waitcnt lgkmcnt(0)"
                                     : "=&s"(ex), "+v"(alo[0]), "+v"(alo[1]), "+v"(alo[2]), "+v"(alo[3]),
                                       "+v"(alo[4]), "+v"(alo[5]), "+v"(alo[6]), "+v"(alo[7]), "+v"(ahi[0]),
                                       "+v"(ahi[1]), "+v"(ahi[2]), "+v"(ahi[3]), "+v"(ahi[4]), "+v"(ahi[5]),
                                       "+v"(ahi[6]), "+v"(ahi[7])
                                     : "s"(mlo), "s"(mhi), "v"(xa), "i"(TO), "i"(TO + 32), "i"(TO + 128),
                                       "i"(TO + 160)
                                     : "memory", "scc");
                    } else if constexpr (NT == 2) {
                        asm volatile("s_mov_b64 %0, exec\n\ts_and_b64 exec, %9, %0\n\t"
                                     "ds_read_b64 %1, %11\n\t"
                                     "ds_read_b64 %2, %11 offset:%12\n\t"
                                     "ds_read_b64 %3, %11 offset:32\n\t"
                                     "ds_read_b64 %4, %11 offset:%13\n\t"
                                     "s_and_b64 exec, %10, %0\n\t"
                                     "ds_read_b64 %5, %11\n\t"
                                     "ds_read_b64 %6, %11 offset:%12\n\t"
                                     "ds_read_b64 %7, %11 offset:32\n\t"
                                     "ds_read_b64 %8, %11 offset:%13\n\t"
                                     "s_mov_b64 exec, %0\n\ts_waitcnt lgkmcnt(0)"
                                     : "=&s"(ex), "+v"(alo[0]), "+v"(alo[1]), "+v"(alo[2]), "+v"(alo[3]),
                                       "+v"(ahi[0]), "+v"(ahi[1]), "+v"(ahi[2]), "+v"(ahi[3])
                                     : "s"(mlo), "s"(mhi), "v"(xa), "i"(TO), "i"(TO + 32)
                                     : "memory", "scc");
                    } else if constexpr (GU_AJ == 2) {
                        asm volatile("s_mov_b64 %0, exec\n\ts_and_b64 exec, %9, %0\n\t"
                                     "ds_read_b64 %1, %11\n\t"
                                     "ds_read_b64 %2, %11 offset:32\n\t"
                                     "ds_read_b64 %3, %11 offset:128\n\t"
                                     "ds_read_b64 %4, %11 offset:160\n\t"
                                     "s_and_b64 exec, %10, %0\n\t"
                                     "ds_read_b64 %5, %11\n\t"
                                     "ds_read_b64 %6, %11 offset:32\n\t"
                                     "ds_read_b64 %7, %11 offset:128\n\t"
                                     "ds_read_b64 %8, %11 offset:160\n\t"
                                     "s_mov_b64 exec, %0\n\ts_waitcnt lgkmcnt(0)"
                                     : "=&s"(ex), "+v"(alo[0]), "+v"(alo[1]), "+v"(alo[2]), "+v"(alo[3]),
                                       "+v"(ahi[0]), "+v"(ahi[1]), "+v"(ahi[2]), "+v"(ahi[3])
                                     : "s"(mlo), "s"(mhi), "v"(xa)
                                     : "memory", "scc");
                    } else {
                        asm volatile("s_mov_b64 %0, exec\n\ts_and_b64 exec, %5, %0\n\t"
                                     "ds_read_b64 %1, %7\n\t"
                                     "ds_read_b64 %2, %7 offset:32\n\t"
                                     "s_and_b64 exec, %6, %0\n\t"
                                     "ds_read_b64 %3, %7\n\t"
                                     "ds_read_b64 %4, %7 offset:32\n\t"
                                     "s_mov_b64 exec, %0\n\ts_waitcnt lgkmcnt(0)"
                                     : "=&s"(ex), "+v"(alo[0]), "+v"(alo[1]), "+v"(ahi[0]), "+v"(ahi[1])
                                     : "s"(mlo), "s"(mhi), "v"(xa)
                                     : "memory", "scc");
                    }
                }
                // w_scale * d_x of each of the lane's input rows, as the reference
                const float dw = W::scale(w, pi, j);
                const int sidx = lay::q8_scale(K, b);
                float sb[NT][4];
                auto scales = [&](int t) {
                    const float4 dx = *reinterpret_cast<const float4 *>(xd_s + sidx * DSTR + t * 8 + kg * 4);
                    sb[t][0] = dw * dx.x;
                    sb[t][1] = dw * dx.y;
                    sb[t][2] = dw * dx.z;
                    sb[t][3] = dw * dx.w;
                };
                // (the second tile's after the first MFMA; with two tiles,
                // Q8_0 forms the next block's tile-0 scales during this one)
                constexpr bool SB_AHEAD = !Q4K && NT == 2;
                if (SB_AHEAD && j > 0) {
#pragma unroll
                    for (int q = 0; q < 4; q++) sb[0][q] = sb_next[q];
                } else {
                    scales(0);
                }
                const int jo = (j % GU_AJ) * NM; // this block's A operands
                auto mfma = [&](int m, const f16x8 &wo) {
                    const f32x16 z = {};
                    return __builtin_amdgcn_mfma_f32_32x32x16_f16(
                        __builtin_bit_cast(f16x8, make_ulonglong2(alo[jo + m], ahi[jo + m])), wo, z, 0, 0, 0);
                };
                int bsum[NT][4];
                auto chains = [&](int m, const f32x16 &d) {
                    const int hh = m / NT, t = m % NT;
#pragma unroll
                    for (int q = 0; q < 4; q++)
#pragma unroll
                        for (int r = 0; r < 4; r++)
                            acc[t][q][pi][4 * hh + r] = __builtin_fmaf(d[4 * q + r], sb[t][q], acc[t][q][pi][4 * hh + r]);
                    if (DUMP) {
#pragma unroll
                        for (int q = 0; q < 4; q++) {
                            const int s4 = (int)d[4 * q] + (int)d[4 * q + 1] + (int)d[4 * q + 2] + (int)d[4 * q + 3];
                            bsum[t][q] = hh ? bsum[t][q] + s4 : s4;
                        }
                    }
                };
                // one MFMA result live at a time (issuing the next MFMA before
                // the FMAs of the last measured slower); independent work goes
                // between an MFMA and the FMAs that wait for its result: after
                // the block's first MFMA the second half's weight operand and
                // the second tile's scales, after its last the next block's
                // first operand (Q8_0 at T = 512 256-259 -> 251-254 us, Q4_K
                // at T = 2048 832-837 -> 821 us)
                {
                    const f16x8 wo0 = j > 0 ? wo_next : W::operand(w, pi, j, 0);
                    const f32x16 d0 = mfma(0, wo0);
                    const f16x8 wo1 = W::operand(w, pi, j, 1);
                    if constexpr (NT == 2) scales(1);
                    chains(0, d0);
                    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
                    for (int t = 1; t < NT; t++) {
                        const f32x16 d = mfma(t, wo0);
                        if (SB_AHEAD && j < 3)
                            dx_next = *reinterpret_cast<const float4 *>(xd_s + lay::q8_scale(K, b + 2) * DSTR + kg * 4);
                        chains(t, d);
                        __builtin_amdgcn_sched_barrier(0);
                    }
#pragma unroll
                    for (int t = 0; t < NT; t++) {
                        const f32x16 d = mfma(NT + t, wo1);
                        if (SB_AHEAD && t == 0 && j < 3) {
                            const float dwn = W::scale(w, pi, j + 1);
                            sb_next[0] = dwn * dx_next.x;
                            sb_next[1] = dwn * dx_next.y;
                            sb_next[2] = dwn * dx_next.z;
                            sb_next[3] = dwn * dx_next.w;
                        }
                        if (t == NT - 1 && j < 3) wo_next = W::operand(w, pi, j + 1, 0);
                        chains(NT + t, d);
                        __builtin_amdgcn_sched_barrier(0);
                    }
                }
                __builtin_amdgcn_sched_barrier(0);
                if (DUMP) {
                    int32_t *dump = li < 16 ? a.dump_a : a.dump_b;
#pragma unroll
                    for (int t = 0; t < NT; t++)
#pragma unroll
                        for (int q = 0; q < 4; q++) {
                            const int i = 8 * t + 2 * q + kg;
                            if (dump && i < cnt) dump[((size_t)(beg + i) * rows + orow) * NB + b] = bsum[t][q];
                        }
                }
            }
        };
        static_assert(W::STEPS % 2 == 0, "steps");
        // step h of parity PAR (compile-time: a runtime parity would be a
        // branch in the loop body, past which the compiler sinks the chains'
        // FMAs, keeping every MFMA result of a step live at once)
        auto stepc = [&](int h, auto par_c, const typename W::Step &w) {
            if constexpr (W::BOTH) {
                compute(h, std::integral_constant<int, 0>(), w);
                compute(h, std::integral_constant<int, 1>(), w);
            } else {
                compute(h >> 1, par_c, w);
            }
        };
        // two steps in flight per wave, loads one ahead (a deeper ring, three
        // steps for Q8_0, measured slower); the last turn reloads its own step
        // rather than branch
        typename W::Step w1;
        // the step count as a value the compiler cannot see through (a.T is
        // never negative): narrow rows give a loop of one or two turns,
        // which it would otherwise lay out flat, with the turns' loads and
        // chains overlapped past the registers
        const int nsteps = W::STEPS + (a.T < 0 ? 2 : 0);
#pragma unroll 1
        for (int h = 0; h < nsteps; h += 2) {
            wsrc.load(h + 1, w1);
            stepc(h, std::integral_constant<int, 0>(), w0);
            wsrc.load(min(h + 2, W::STEPS - 2), w0);
            stepc(h + 1, std::integral_constant<int, 1>(), w1);
        }
        // the reference's tree, within the lane: u_l = chain (0, l) + chain
        // (1, l); v_l = u_l + u_(l+4); (v0 + v2) + (v1 + v3); Q4_K then
        // subtracts its mins; then silu(gate) * up, up from column li + 16
#pragma unroll
        for (int t = 0; t < NT; t++)
#pragma unroll
            for (int q = 0; q < 4; q++) {
                float v[4];
#pragma unroll
                for (int l = 0; l < 4; l++) {
                    const float u0 = acc[t][q][0][l] + acc[t][q][1][l];
                    const float u1 = acc[t][q][0][l + 4] + acc[t][q][1][l + 4];
                    v[l] = u0 + u1;
                }
                float s = (v[0] + v[2]) + (v[1] + v[3]);
                if constexpr (Q4K) s = s - mins[t][q];
                const float up = __shfl_xor(s, 16);
                const int i = 8 * t + 2 * q + kg;
                if (li < 16 && i < cnt) a.out[(size_t)(beg + i) * rows + orow] = silu_mul_t(s, up, exp_tab);
            }
    };
    if (cnt > 8) run(std::integral_constant<int, 2>());
    else run(std::integral_constant<int, 1>());
}


// ---------------------------------------------------------------------------
// Q6_K down matrices at prefill sizes on the int8 matrix cores.
//
// biv's dot_q6k (quant.rs:651-686, x86 1475-1533) weighs each 16-element
// half of a 32-element block by its own int8 sub-scale: isum = sc_0 *
// dot16_0 + sc_1 * dot16_1 (exact int32), then d * d_x * isum.  Here
// v_mfma_i32_16x16x32_i8 takes A = one block of 8 input rows, each twice:
// A row 2 t + hh keeps only half hh of input row t (lanes kq = 2 hh, 2 hh + 1
// hold that half's bytes); B = the block of 16 weight rows as q - 32.  D row
// 2 t + hh, column n is dot16_hh of input row t and weight row n, exactly,
// and lane (n, kq) holds both halves of input rows 2 kq and 2 kq + 1: isum
// in integers, then the f32 scaling; the sum over blocks runs in an order of
// its own (down's outputs only meet the combine): d_x * isum summed over a
// super-block's eight blocks, times its d once.
//
// Weights (chain layout, layout.hpp): per 512 elements (four halves qq of a
// row) the ql units 16 (qq / 4) + 8 pi + w hold ql word w of quarters pi and
// pi + 2 of each half, the qh units 8 (qq / 4) + w qh word w; lane kq loads
// words 2 kq and 2 kq + 1, i.e. bytes 8 kq .. 8 kq + 7 of every block.
template <int K, bool DUMP>
__global__ __launch_bounds__(QNTH) void k_q6k_down_mfma(MvArgs a)
{
    constexpr int RT = QRT;
    constexpr int NB = K / 32;
    constexpr int NQ = K / 512;      // groups of four halves
    constexpr int XSTR = K / 16 + 1; // staged quant row: 16-byte units (+1 against bank conflicts)
    constexpr int DSTR = QT + 4;     // staged scales [block][pair], floats
    static_assert(K % 512 == 0 && QT % 8 == 0, "shapes");
    __shared__ uint4 xq_s[(QT + 1) * XSTR]; // the slot's rows, then a row of zeros
    __shared__ float xd_s[NB * DSTR];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int n = lane & 15, kq = lane >> 4;
    int u, rt;
    if (!slot_unit<SLOT_RUN>(a, blockIdx.x, u, rt)) return;
    const bool shared = u < a.n_sh;
    int e = 0, beg, cnt;
    if (shared) {
        const int tok0 = u * a.sh_chunk;
        beg = a.P + tok0;
        cnt = min(a.sh_chunk, a.T - tok0);
    } else {
        const Slot sl = a.dp.slots[u - a.n_sh];
        if (sl.cnt == 0) return; // uniform over the workgroup
        e = sl.expert;
        beg = sl.beg;
        cnt = sl.cnt;
    }
    const DevMat &M = shared ? a.sa : a.a;
    const int rows = M.rows;
    const int rw0 = rt * Q_ROWS_WG + wave * 16 * RT;
    // this lane's weight words of group gq, per row tile
    uint4 ql[RT][2][2], qh[RT][2];
    int4 scv[RT][2];
    float dsb[RT][2];
    auto load_group = [&](int gq) {
#pragma unroll
        for (int r = 0; r < RT; r++) {
            const size_t row = (size_t)e * rows + rw0 + 16 * r + n;
            const uint8_t *base = M.q + row * (K / 256) * 192;
            const uint4 *pl = reinterpret_cast<const uint4 *>(base);
            const uint4 *ph = reinterpret_cast<const uint4 *>(base + (K / 256) * 128);
#pragma unroll
            for (int pi = 0; pi < 2; pi++)
#pragma unroll
                for (int w = 0; w < 2; w++) ql[r][pi][w] = pl[16 * gq + 8 * pi + 2 * kq + w];
#pragma unroll
            for (int w = 0; w < 2; w++) qh[r][w] = ph[8 * gq + 2 * kq + w];
            // sub-scales of the group's 16 blocks: [pi][hsel] runs of K / 64
            const int8_t *sc = reinterpret_cast<const int8_t *>(M.s + row * (K / 16));
#pragma unroll
            for (int c = 0; c < 2; c++) {
                // scv[r][c]: bytes [pi = c][hsel = 0 / 1][s = 8 gq .. + 7] as two int2 halves
                const uint2 s0 = *reinterpret_cast<const uint2 *>(sc + (2 * c + 0) * (K / 64) + 8 * gq);
                const uint2 s1 = *reinterpret_cast<const uint2 *>(sc + (2 * c + 1) * (K / 64) + 8 * gq);
                scv[r][c] = make_int4((int)s0.x, (int)s0.y, (int)s1.x, (int)s1.y);
            }
            const uint16_t *dp = reinterpret_cast<const uint16_t *>(M.d + row * (K / 256) * 2);
            dsb[r][0] = f16_to_f32(dp[2 * gq]);
            dsb[r][1] = f16_to_f32(dp[2 * gq + 1]);
        }
    };
    // the first group's weights go out before the staging waits
    load_group(0);
    // stage the slot's input rows (as the Q8_0 down kernel)
    {
        constexpr int UPR = K / 16;
        for (int idx = tid; idx < QT * UPR; idx += QNTH) {
            const int i = idx / UPR, c = idx % UPR;
            const size_t ar = beg + min(i, cnt - 1);
            xq_s[i * XSTR + c] = reinterpret_cast<const uint4 *>(a.xq + ar * K)[c];
        }
        for (int c = tid; c < XSTR; c += QNTH) xq_s[QT * XSTR + c] = make_uint4(0u, 0u, 0u, 0u);
        for (int idx = tid; idx < QT * NB; idx += QNTH) {
            const int i = idx / NB, bs = idx % NB;
            const size_t ar = beg + min(i, cnt - 1);
            const int b = 2 * (bs % (K / 64)) + bs / (K / 64); // lay::q8_scale's inverse
            xd_s[b * DSTR + i] = a.xd[ar * NB + bs];
        }
    }
    __syncthreads();
    // A row 2 t + hh keeps only half hh, bytes 16 hh .. 16 hh + 15: lanes
    // kq = 2 hh and 2 hh + 1 read them, the other lanes the row of zeros
    // (no masking per block)
    const bool keep = (n & 1) == (kq >> 1);
    const int at = n >> 1; // A row's input row within the 8-row group
    const uint4 *const xrow = keep ? xq_s + at * XSTR : xq_s + QT * XSTR;
    const int xtstr = keep ? 8 * XSTR : 0; // from one 8-row group to the next
    // acc: the sum over super-blocks of d * (the super-block's sum over its
    // blocks of d_x * isum, in asb)
    float acc[QT / 8][RT][2], asb[QT / 8][RT][2];
#pragma unroll
    for (int t = 0; t < QT / 8; t++)
#pragma unroll
        for (int r = 0; r < RT; r++) acc[t][r][0] = acc[t][r][1] = 0.0f;
    for (int gq = 0; gq < NQ; gq++) {
        if (gq > 0) load_group(gq);
#pragma unroll
        for (int bl = 0; bl < 16; bl++) { // block b = 16 gq + bl: half qq = 4 gq + bl / 4, quarter k = bl % 4
            const int qq = bl >> 2, k = bl & 3, pi = k & 1, hi = k >> 1;
            const int b = 16 * gq + bl;
            const int s2 = 2 * (4 * gq + qq) + hi; // the sub-scale step of (pi, hsel)
            // B: q - 32 of words 2 kq, 2 kq + 1 of block b, per row tile
            long wo[RT];
            int sc0[RT], sc1[RT];
#pragma unroll
            for (int r = 0; r < RT; r++) {
                uint32_t wv[2];
#pragma unroll
                for (int w = 0; w < 2; w++) {
                    // each byte's high bits 2 k, 2 k + 1 of qh moved to bits 4, 5
                    const uint32_t lo = (ql[r][pi][w][qq] >> (4 * hi)) & 0x0F0F0F0Fu;
                    const uint32_t qv = qh[r][w][qq];
                    const uint32_t hs = k <= 2 ? qv << (4 - 2 * k) : qv >> (2 * k - 4);
                    const uint32_t x = (hs & 0x30303030u) | lo;
                    // bytewise q - 32: q + 96 carries out of no byte, and
                    // flipping bit 7 then subtracts 128 mod 256
                    wv[w] = (x + 0x60606060u) ^ 0x80808080u;
                }
                wo[r] = (long)((uint64_t)wv[0] | (uint64_t)wv[1] << 32);
                const int sidx = s2 - 8 * gq; // 0..7 within the group's run
                const int4 sv = scv[r][pi];
                const uint32_t w0 = sidx < 4 ? (uint32_t)sv.x : (uint32_t)sv.y;
                const uint32_t w1 = sidx < 4 ? (uint32_t)sv.z : (uint32_t)sv.w;
                sc0[r] = (int)(int8_t)((w0 >> (8 * (sidx & 3))) & 0xFF);
                sc1[r] = (int)(int8_t)((w1 >> (8 * (sidx & 3))) & 0xFF);
            }
            // the activations' block b: chain layout unit 16 g + 8 pi + w, word j
            const int g = b >> 3, xpi = b & 1, j = (b >> 1) & 3;
#pragma unroll
            for (int t = 0; t < QT / 8; t++) {
                if (8 * t >= cnt) break; // uniform
                const uint4 *xr = xrow + t * xtstr + 16 * g + 8 * xpi + 2 * kq;
                const uint32_t lo = xr[0][j], hi2 = xr[1][j];
                const long xo = (long)((uint64_t)lo | (uint64_t)hi2 << 32);
                const float2 dx = *reinterpret_cast<const float2 *>(xd_s + b * DSTR + 8 * t + 2 * kq);
#pragma unroll
                for (int r = 0; r < RT; r++) {
                    const i32x4 z = {0, 0, 0, 0};
                    const i32x4 d = __builtin_amdgcn_mfma_i32_16x16x32_i8(xo, wo[r], z, 0, 0, 0);
                    // 24-bit products (full rate; |dot16| <= 16 * 128 * 32,
                    // sub-scales int8): the same integers as 32-bit ones
                    const int is0 = __mul24(sc0[r], d[0]) + __mul24(sc1[r], d[1]);
                    const int is1 = __mul24(sc0[r], d[2]) + __mul24(sc1[r], d[3]);
                    asb[t][r][0] = (bl & 7) ? __builtin_fmaf((float)is0, dx.x, asb[t][r][0]) : (float)is0 * dx.x;
                    asb[t][r][1] = (bl & 7) ? __builtin_fmaf((float)is1, dx.y, asb[t][r][1]) : (float)is1 * dx.y;
                    if ((bl & 7) == 7) {
                        const float dd = dsb[r][qq >> 1];
                        acc[t][r][0] = __builtin_fmaf(dd, asb[t][r][0], acc[t][r][0]);
                        acc[t][r][1] = __builtin_fmaf(dd, asb[t][r][1], acc[t][r][1]);
                    }
                    if (DUMP && a.dump_a) { // the block int32s, for the taps
                        const int i0 = 8 * t + 2 * kq, row = rw0 + 16 * r + n;
                        if (i0 < cnt) a.dump_a[((size_t)(beg + i0) * rows + row) * NB + b] = is0;
                        if (i0 + 1 < cnt) a.dump_a[((size_t)(beg + i0 + 1) * rows + row) * NB + b] = is1;
                    }
                }
            }
            __builtin_amdgcn_sched_barrier(0);
        }
    }
    // input rows 8 t + 2 kq + c, row rw0 + 16 r + n
#pragma unroll
    for (int t = 0; t < QT / 8; t++)
#pragma unroll
        for (int c = 0; c < 2; c++) {
            const int i = 8 * t + 2 * kq + c;
            if (i < cnt) {
#pragma unroll
                for (int r = 0; r < RT; r++) a.out[(size_t)(beg + i) * rows + rw0 + 16 * r + n] = acc[t][r][c];
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
    const dim3 grid(slot_grid<SLOT_RUN_BF16>(slots, a.n_rt));
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


hipError_t launch_q8_down_t(MvArgs a, int routed, int shared, hipStream_t st)
{
    const DevMat &M = routed ? a.a : a.sa;
    if (!routed) a.u_max = 0;
    a.n_sh = shared ? (a.T + a.sh_chunk - 1) / a.sh_chunk : 0;
    const int slots = a.u_max + a.n_sh;
    if (slots == 0) return hipSuccess;
    if (a.sh_chunk > QT || M.rows % Q_ROWS_WG) return hipErrorInvalidValue;
    a.n_rt = M.rows / Q_ROWS_WG;
    const dim3 grid(slot_grid<SLOT_RUN>(slots, a.n_rt));
#define BIV_Q8_CASE(KK)                                                                                         \
    if (M.cols == KK) {                                                                                         \
        if (a.dump_a)                                                                                           \
            k_q8_down_mfma<KK, true><<<grid, QNTH, 0, st>>>(a);                                                 \
        else                                                                                                    \
            k_q8_down_mfma<KK, false><<<grid, QNTH, 0, st>>>(a);                                                \
        return hipGetLastError();                                                                               \
    }
    if (M.ty == T_Q8_0) {
        BIV_Q8_CASE(2048)
        BIV_Q8_CASE(1024)
        BIV_Q8_CASE(512)
    }
#undef BIV_Q8_CASE
#define BIV_Q6_CASE(KK)                                                                                         \
    if (M.cols == KK) {                                                                                         \
        if (a.dump_a)                                                                                           \
            k_q6k_down_mfma<KK, true><<<grid, QNTH, 0, st>>>(a);                                                \
        else                                                                                                    \
            k_q6k_down_mfma<KK, false><<<grid, QNTH, 0, st>>>(a);                                               \
        return hipGetLastError();                                                                               \
    }
    if (M.ty == T_Q6K) {
        BIV_Q6_CASE(2048)
        BIV_Q6_CASE(1024)
        BIV_Q6_CASE(512)
    }
#undef BIV_Q6_CASE
    return hipErrorInvalidValue;
}

hipError_t launch_q8_mfma_down(const MvArgs &a, hipStream_t st)
{
    const bool has_shared = a.sa.q != nullptr;
    if (has_shared && a.sa.ty == a.a.ty && a.sa.cols == a.a.cols && a.sa.rows == a.a.rows)
        return launch_q8_down_t(a, 1, 1, st);
    hipError_t err = launch_q8_down_t(a, 1, 0, st);
    if (err != hipSuccess || !has_shared) return err;
    return launch_q8_down_t(a, 0, 1, st);
}


hipError_t launch_gu_t(MvArgs a, int routed, int shared, hipStream_t st)
{
    const DevMat &M = routed ? a.a : a.sa;
    if (!routed) a.u_max = 0;
    a.n_sh = shared ? (a.T + a.sh_chunk - 1) / a.sh_chunk : 0;
    const int slots = a.u_max + a.n_sh;
    if (slots == 0) return hipSuccess;
    if (a.sh_chunk > QT || M.rows % G_ROWS_WG) return hipErrorInvalidValue;
    a.n_rt = M.rows / G_ROWS_WG;
    const dim3 grid(slot_grid<SLOT_RUN>(slots, a.n_rt));
    const bool dump = a.dump_a || a.dump_b;
#define BIV_GU_CASE(TY, KK)                                                                                     \
    if (M.ty == TY && M.cols == KK) {                                                                           \
        if (dump)                                                                                               \
            k_gu_exact<TY, KK, true><<<grid, GNTH, 0, st>>>(a);                                                 \
        else                                                                                                    \
            k_gu_exact<TY, KK, false><<<grid, GNTH, 0, st>>>(a);                                                \
        return hipGetLastError();                                                                               \
    }
    BIV_GU_CASE(T_Q8_0, 2048)
    BIV_GU_CASE(T_Q8_0, 1024)
    BIV_GU_CASE(T_Q8_0, 512)
    BIV_GU_CASE(T_Q4K, 2048)
    BIV_GU_CASE(T_Q4K, 1024)
    BIV_GU_CASE(T_Q4K, 512)
#undef BIV_GU_CASE
    return hipErrorInvalidValue;
}

hipError_t launch_mfma_gateup_exact(const MvArgs &a, hipStream_t st)
{
    // routed and shared in one launch when they share a type and shape
    const bool has_shared = a.sa.q != nullptr;
    if (a.a.ty != a.b.ty || (has_shared && a.sa.ty != a.sb.ty)) return hipErrorInvalidValue;
    if (has_shared && a.sa.ty == a.a.ty && a.sa.cols == a.a.cols && a.sa.rows == a.a.rows)
        return launch_gu_t(a, 1, 1, st);
    hipError_t err = launch_gu_t(a, 1, 0, st);
    if (err != hipSuccess || !has_shared) return err;
    return launch_gu_t(a, 0, 1, st);
}

} // namespace biv
