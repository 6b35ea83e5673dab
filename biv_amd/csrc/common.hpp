// Shared definitions of the gfx950 MoE backend: device matrix layouts, the
// per-forward scratch, and the kernel launchers api.cpp drives.
#pragma once
#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

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
    uint8_t *s = nullptr;
    uint8_t *d = nullptr;
};

// Routing and dispatch state of one forward of T tokens (device pointers).
struct Dispatch {
    int *n_active;   // [1]  U: experts with at least one pair
    int *act_expert; // [n_expert] expert of active slot u, ascending
    int *act_beg;    // [n_expert] first dispatch position of slot u
    int *act_cnt;    // [n_expert] pairs of slot u
    int *pair_tok;   // [P] token of each pair in dispatch order
    int *pair_exp;   // [P] expert of each pair in dispatch order
    float *pair_w;   // [P] routing weight of each pair
    int *tok_pairs;  // [T][k] dispatch positions of token t's pairs, ascending expert id
    int *ids;        // [T][k] chosen experts in rank order
    float *wts;      // [T][k] their weights
};

// Launchers (kernels.hip).  All enqueue on `st`; none synchronises.
hipError_t launch_quant_rows(const float *x, int n_blocks, int K, int8_t *qs, float *d, float *s, hipStream_t st);
hipError_t launch_router(const float *router, const float *gate_inp, int n_expert, int E, const float *h, int T,
                         float *logits, float *glogit, hipStream_t st);
hipError_t launch_route(const float *logits, int n_expert, int k, int T, int *ids, float *wts, hipStream_t st);
hipError_t launch_sort(const int *ids, const float *wts, int n_expert, int k, int T, const Dispatch &dp,
                       hipStream_t st);

struct MvArgs {
    DevMat a, b;            // routed stacks (b: the up stack of a gate/up pair)
    DevMat sa, sb;          // the shared expert's matrices (n = 1), sa.q == nullptr without one
    const int8_t *xq;       // input rows: int8 [rows_in][K]
    const float *xd;        // [rows_in][K/32] block scales
    const float *xs;        // [rows_in][K/32] block d * sum(q) (Q4_K mins)
    Dispatch dp;
    float *out;             // [P + T][rows]
    int32_t *dump_a;        // optional [P + T][rows][K/32] block int32 dots of a
    int32_t *dump_b;        // optional, of b
    int T, P, u_max;
    int x_by_token;         // 1: input row of a pair is its token's (gate/up); 0: the pair's own (down)
};

// gate/up: out[p][r] = silu(gate_r . x) * (up_r . x) for every pair and shared row.
hipError_t launch_gateup(const MvArgs &a, hipStream_t st);
// down: out[p][r] = down_r . x_p
hipError_t launch_down(const MvArgs &a, hipStream_t st);

// out[t] (+)= sum over t's pairs, ascending expert, of w * y[pair], then
// sigmoid(glogit[t]) * y[P + t] when there is a shared expert.
hipError_t launch_combine(const float *y, const Dispatch &dp, const float *glogit, int has_shared, int T, int P,
                          int k, int E, float *out, int add, hipStream_t st);

} // namespace biv
