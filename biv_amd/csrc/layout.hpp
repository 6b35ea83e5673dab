// Chain layouts: where each byte of a weight or activation row lives in
// device memory.
//
// biv's x86 kernels (engine/src/quant.rs:1043-1545) accumulate a row's dot
// product in the 8 f32 lanes of two ymm registers: block b goes to register
// b & 1, and lane l of that register sums bytes 4l..4l+3 of every block, in
// block order.  That is 16 independent FMA chains per row.  On the GPU each
// chain is one lane: lane (pi, l) of a 16-lane group walks the blocks of
// parity pi and uses word l of each.  The layouts below put the words one
// lane needs next to each other, four steps per 128-bit load, and make each
// load instruction of the 16 lanes read 256 contiguous bytes.
//
// Steps per chain: S = K / 64 (K elements per row, 32 per block, two
// parities).  Step s of chain pi is block b = 2 s + pi.
#pragma once

namespace biv {
namespace lay {

// Q8_0 weights and every Q8 activation row (the int8 quants): word l of block b.
__host__ __device__ constexpr int q8_word(int b, int l)
{
    return (((b >> 3) * 16 + (b & 1) * 8 + l) << 2) + ((b >> 1) & 3);
}

// Q8_0 block scales (f16) and Q8 activation scales / sums (f32): block b.
__host__ __device__ constexpr int q8_scale(int K, int b) { return (b & 1) * (K / 64) + (b >> 1); }

// Q4_K: sub-blocks 2s and 2s+1 share 32 bytes (low and high nibbles); word l
// of pair s.  Both parities of lane l read the same word.
__host__ __device__ constexpr int q4k_word(int s, int l) { return (((s >> 2) * 8 + l) << 2) + (s & 3); }

// Q6_K, with qq = 2 * super-block + half: the ql word of chain pi (quarters
// pi and pi + 2 of the half share it), and the qh word (all four quarters).
__host__ __device__ constexpr int q6k_ql_word(int qq, int pi, int l)
{
    return (((qq >> 2) * 16 + pi * 8 + l) << 2) + (qq & 3);
}
__host__ __device__ constexpr int q6k_qh_word(int qq, int l) { return (((qq >> 2) * 8 + l) << 2) + (qq & 3); }

// Q6_K sub-scales: the one lane (pi, l) applies at step s; hsel = l >= 4
// (lanes 4-7 hold elements 16..31 of a block).
__host__ __device__ constexpr int q6k_sc(int K, int pi, int hsel, int s) { return (pi * 2 + hsel) * (K / 64) + s; }

// F32 rows (router, gate_inp): biv's dot_f32 (quant.rs:1177-1207) has 32
// chains, chain L summing elements L, L + 32, ...; value i of chain L.
__host__ __device__ constexpr int f32_elem(int i, int L) { return (((i >> 2) * 32 + L) << 2) + (i & 3); }

// BF16 rows (biv's dot_bf16, quant.rs:1228-1256: two 8-lane accumulators
// over 16-element steps): chain L (0..15) sums elements L, L + 16, ...;
// lane L's 128-bit load g holds its steps 8g..8g+7.  Index (in 16-bit
// units) of element e of a row.
__host__ __device__ constexpr int bf16_elem(int e)
{
    return (((e >> 4) >> 3) * 16 + (e & 15)) * 8 + ((e >> 4) & 7);
}

} // namespace lay
} // namespace biv
