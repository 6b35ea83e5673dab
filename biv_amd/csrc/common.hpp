// Shared definitions of the gfx950 MoE backend: device matrix layouts, the
// per-forward scratch, and the kernel launchers api.cpp drives.
#pragma once
#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include "bf16_split.h"

namespace biv {

enum : int { T_F32 = 0, T_F16 = 1, T_Q8_0 = 8, T_Q4K = 12, T_Q6K = 14, T_BF16 = 30 };

// One matrix, or a stack of n matrices of rows x cols, in device memory,
// repacked at upload into planes whose rows start on 16-byte boundaries and
// whose words sit in the chain layouts of layout.hpp.  The bytes per element
// are those of the ggml type: repacking moves bytes, it adds none.
//   Q8_0: q = int8  [n][rows][cols]              the quants, lay::q8_word order
//         s = f16   [n][rows][cols/32]           block scales, lay::q8_scale order
//   Q4_K: q = uint8 [n][rows][cols/2]            the nibble bytes, lay::q4k_word order
//         s = uint8 [n][rows][cols/256][16]      d, dmin (f16) and the 12 packed scale bytes
//   Q6_K: q = uint8 [n][rows][cols/256 * 192]    ql words (lay::q6k_ql_word), then qh (lay::q6k_qh_word)
//         s = int8  [n][rows][cols/16]           sub-block scales, lay::q6k_sc order
//         d = f16   [n][rows][cols/256]          super-block scales
//   BF16: q = uint16[n][rows][cols]
//   F32:  q = float [n][rows][cols]              lay::f32_elem order
struct DevMat {
    int ty = -1;
    int cols = 0, rows = 0, n = 0;
    uint8_t *q = nullptr;
    uint8_t *s = nullptr; // F32: the rows as given (row-major), besides q's chain layout
    uint8_t *d = nullptr;
};

// A run of at most `chunk` consecutive dispatch positions of one expert.
// Consumers read the whole record with scalar loads; tok[] holds the tokens
// of its first SLOT_TOKS pairs (entries past cnt are not written).
constexpr int SLOT_TOKS = 8;
struct alignas(16) Slot {
    int expert, beg, cnt; // cnt 0: an unused slot
    int used;             // the number of slots in use (in every used record; 0 in unused ones)
    int tok[SLOT_TOKS];
};

// Routing and dispatch state of one forward of T tokens (device pointers).
// A slot is a run of at most `chunk` consecutive pairs of one expert; an
// expert with more pairs has several slots.  Slots are in ascending expert
// order.
struct Dispatch {
    struct Slot *slots; // [slot_cap]
    int slot_cap;       // slots the consumers' grids cover (max_slots); the sort writes every one
    int *pair_tok;   // [P] token of each pair in dispatch order
    int *pair_exp;   // [P] expert of each pair in dispatch order
    float *pair_w;   // [P] routing weight of each pair
    int *tok_pairs;  // [T][k] dispatch positions of token t's pairs, ascending expert id
    int *ids;        // [T][k] chosen experts in rank order
    float *wts;      // [T][k] their weights
};

// Launchers (kernels.hip).  All enqueue on `st`; none synchronises.
//
// A forward is router (with the quantisation of h); route and dispatch
// sort; gate/up; then down and combine in one launch at decode sizes, or the
// quantisation of the intermediate, down and combine apart.  Past 16 tokens
// the dispatch sort is a counting sort over blocks of 16 tokens in three
// launches (per-block counts with the routing, one scan, the placement).

struct RouterArgs {
    const float *router;   // [n_expert][E], f32 chain layout
    const float *router_rm; // the same rows row-major (the matrix-core router at prefill)
    const float *gate_inp; // [E] or nullptr
    const float *gate_rm;  // the same row as given (row-major)
    int n_expert, E, T;
    const float *h;        // [T][E]
    float *logits;         // [T][n_expert]
    float *glogit;         // [T]
    int8_t *xq;            // h quantised: [T][E] chain layout
    float *xd, *xs;        // [T][E/32]
    // With norm_w: h is the residual x and every use of it takes
    // rms_norm(x) (ops.rs:136-144) with these weights and eps, the
    // post_norm before the FFN (model.rs:786-790); hn [T][E] receives it.
    const float *norm_w;
    float eps;
    float *hn;
    // With xh (BF16 experts at T >= prep_min_t()): the bf16 hi / lo halves of
    // the (normalised) rows in the matrix-core chunk order, as
    // launch_split_bf16 writes them, formed by the pre-pass
    uint4 *xh, *xl;
};
// tokens from which launch_router runs the prefill pre-pass (and the
// matrix-core router)
int prep_min_t();

// router logits + gate_inp logit + Q8 quantisation of h
hipError_t launch_router(const RouterArgs &a, hipStream_t st);
// route every token, then sort the pairs into dispatch order (`work`:
// route_work_ints(T) ints of scratch)
hipError_t launch_route_sort(const float *logits, int n_expert, int k, int T, int chunk, const Dispatch &dp,
                             int *work, hipStream_t st);

// upper bound of the routed slots of T tokens: one partial slot per expert plus P / chunk full ones
inline int max_slots(int n_expert, int P, int chunk) { return (n_expert < P ? n_expert : P) + P / chunk; }

struct MvArgs {
    DevMat a, b;            // routed stacks (b: the up stack of a gate/up pair)
    DevMat sa, sb;          // the shared expert's matrices (n = 1), sa.q == nullptr without one
    const int8_t *xq;       // input rows: int8 [rows_in][K], chain layout
    const float *xd;        // [rows_in][K/32] block scales
    const float *xs;        // [rows_in][K/32] block d * sum(q) (Q4_K mins)
    const float *xf;        // the f32 input rows [rows_in][K]: what BF16 matrices read, and what the down
                            // kernel quantises itself when qx is set
    int qx;                 // down, quantised matrices: quantise xf in the kernel (not with Q4_K)
    Dispatch dp;
    float *out;             // [P + T][rows]
    int32_t *dump_a;        // optional [P + T][rows][K/32] block int32 dots of a
    int32_t *dump_b;        // optional, of b
    int T, P;
    int u_max;              // grid slots of the routed experts (max_slots)
    int n_sh;               // grid slots of the shared expert, which come first (set by the launcher)
    int sh_chunk;           // tokens per shared-expert slot (set by the launcher)
    int n_rt;               // row tiles of a slot (matrix-core launches; set by the launcher)
    // gate/up of one token with the routing inside (no route launch): the
    // router's logits [n_expert]; every routed workgroup routes the token,
    // the first writes the dispatch records
    const float *logits;
    int n_expert, k;
};

// gate/up: out[p][r] = silu(gate_r . x) * (up_r . x) for every pair and shared row.
hipError_t launch_gateup(const MvArgs &a, hipStream_t st);
// down: out[p][r] = down_r . x_p, with x_p = Q8Act(xf[p]) when a.qx is set
hipError_t launch_down(const MvArgs &a, hipStream_t st);
// Q8Act of n_blocks 32-element blocks of rows of K, into the chain layout
hipError_t launch_quant_rows(const float *x, int n_blocks, int K, int8_t *qs, float *d, float *s, hipStream_t st);
// out[t] (+)= sum over t's pairs, ascending expert, of w * y[pair], then
// sigmoid(glogit[t]) * y[P + t] when there is a shared expert.
hipError_t launch_combine(const float *y, const Dispatch &dp, const float *glogit, int has_shared, int T, int P, int k,
                          int E, float *out, int add, hipStream_t st);

// Down and combine in one launch at decode sizes (each expert's pairs in one
// slot, so T <= the slot size): out[t] (+)= the combine of t's experts' down
// rows, the intermediate xf quantised in the kernel.  Down matrices Q8_0 or
// Q6_K, the shared expert's of the routed type and shape.
struct DownCombineArgs {
    DevMat a, sa;
    const float *xf;     // f32 intermediate [P + T][K]
    Dispatch dp;
    const float *glogit;
    float *out;
    int32_t *dump;       // optional block-dot taps, as the down matvec's
    int T, P, k, add;
};
// LDS bytes it needs for R intermediate rows of K and u_max slot records
size_t down_combine_lds(int R, int K, int u_max);
hipError_t launch_down_combine(const DownCombineArgs &a, hipStream_t st);

// Matvecs over rows of any length K (a multiple of 512), the dense FFN's:
// gate/up writes out[t][r] = silu(gate_r . x_t) * (up_r . x_t); down writes
// out[t][r] = down_r . x_t, or adds it (add).  Quantised matrices read the
// Q8 rows xq / xd (/ xs for Q4_K's mins), BF16 the f32 rows xf.
struct LongArgs {
    DevMat a, b;         // gate and up (b), or down (a)
    const int8_t *xq;    // [T][K] chain layout
    const float *xd, *xs;
    const float *xf;     // [T][K] f32
    float *out;          // [T][rows]
    int T, K, add;
};
hipError_t launch_long_mv(const LongArgs &a, int gateup, hipStream_t st);

// BF16 experts at prefill sizes on the matrix cores (mfma.hip).  The input
// rows are first split into bf16 hi / lo halves (launch_split_bf16); gate/up
// writes the f32 SwiGLU intermediate, down the f32 y rows, as the chain
// kernels do.
// pairs a matrix-core workgroup takes: the slot size for those launches
constexpr int MFMA_TOK_TILE = 256;

struct MfArgs {
    DevMat a, b;       // routed stacks, BF16 (b: up)
    DevMat sa, sb;     // the shared expert's, BF16, sa.q == nullptr without one
    const uint4 *xh;   // input rows, hi halves: [rows_in][K / 8] 16-byte chunks
    const uint4 *xl;   // lo halves
    Dispatch dp;
    float *out;        // [P + T][rows]
    uint4 *xo_h, *xo_l; // gate/up: instead of out, the outputs' bf16 halves (as k_split_bf16 writes them)
    int T, P;
    int n_rt;          // row tiles (set by the launcher)
    int u_max;         // grid slots of the routed experts
    int chunk;         // pairs per routed slot, at most
    int sh_chunk;      // tokens per shared-expert slot
    int n_sh;          // set by the launcher
};
hipError_t launch_split_bf16(const float *x, int rows, int K, void *xh, void *xl, hipStream_t st);
hipError_t launch_mfma_gateup(const MfArgs &a, hipStream_t st);
hipError_t launch_mfma_down(const MfArgs &a, hipStream_t st);

// Quantised experts at prefill sizes on the int8 matrix cores (mfma.hip),
// with the chain kernels' contract (MvArgs: Q8 input rows a.xq / a.xd / a.xs,
// f32 out, dump taps) and slots of at most MFMA_Q8_TILE pairs.  gate/up
// (Q8_0 or Q4_K; gate and up of one type): bit for bit the x86 order, the
// MFMAs making the 4-element word dots.  down (Q8_0 or Q6_K):
// exact int32 block dots (Q6_K: 16-element halves times their sub-scales),
// f32 sums over blocks in an order of their own.
constexpr int MFMA_Q8_TILE = 16;
hipError_t launch_mfma_gateup_exact(const MvArgs &a, hipStream_t st);
hipError_t launch_q8_mfma_down(const MvArgs &a, hipStream_t st);

// y = ops::rms_norm(x) of rows x n (y may be x; n a multiple of 32)
hipError_t launch_rms_norm(const float *x, float *y, const float *w, int rows, int n, float eps, hipStream_t st);

// ints of the dispatch sort's work area for T tokens (per-block expert
// counts, then each expert's first position and first slot)
inline size_t route_work_ints(int T) { return ((size_t)(T + 15) / 16 + 2) * 256; }

} // namespace biv
