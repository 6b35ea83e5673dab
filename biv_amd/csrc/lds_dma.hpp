// Loads straight into LDS that the compiler does not track, and the waits
// and barriers that go with them (gfx9 encodings).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace biv {

// s_waitcnt for at most N vector memory operations outstanding (gfx9
// encoding: vmcnt in bits 3:0 and 15:14; expcnt and lgkmcnt left free)
template <int N> __device__ inline void wait_vm()
{
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

// One 16-byte-per-lane global -> LDS load (LDS address m0 + 16 lane), in
// inline asm: the compiler, which cannot tell which stage buffer an LDS DMA
// writes, would otherwise wait for every DMA in flight before each LDS read
// and undo the prefetch.  The caller waits for it with wait_vm.  (Writing m0
// needs one wait state before the DMA reads it.  The compiler does not save
// m0 around the asm; no kernel that calls this also uses
// __builtin_amdgcn_global_load_lds or anything else for which the compiler
// keeps a value in m0, which the assembly of every kernel shows.)
__device__ inline void lds_dma16_at(const void *g, unsigned lds_addr)
{
    const unsigned m0 = __builtin_amdgcn_readfirstlane(lds_addr);
    asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(g), "s"(m0) : "memory", "m0");
}
// the LDS address (byte offset) of a shared-memory pointer
__device__ inline unsigned lds_addr(const void *p)
{
    return (unsigned)(uintptr_t)(const __attribute__((address_space(3))) void *)p;
}
__device__ inline void lds_dma16(const float *g, const float4 *lds_dst) { lds_dma16_at(g, lds_addr(lds_dst)); }

// a workgroup barrier with no memory fence: the callers order their LDS
// themselves (their loads' waits), and a fence would also wait for every
// load and store in flight
__device__ inline void rm_barrier() { asm volatile("s_barrier" ::: "memory"); }

} // namespace biv
