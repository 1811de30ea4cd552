// HBM -> LDS streaming helpers shared by the pipelined kernels (GEMM,
// attention): the LDS-DMA load, an explicit vector-memory wait, and the
// barrier that does not drain the pipeline.
#pragma once

#include "dotl_common.h"

namespace dotl {

typedef __attribute__((address_space(3))) void lds_void_t;

// Compile-time loop: f(std::integral_constant<int, I>) for I in [B, E).
template <int B, int E, typename Fn>
__device__ __forceinline__ void static_for(Fn&& f) {
    if constexpr (B < E) {
        f(std::integral_constant<int, B>{});
        static_for<B + 1, E>(f);
    }
}

// s_waitcnt with only the vector-memory counter constrained (gfx9 encoding:
// vmcnt in bits 3:0 and 15:14, expcnt 6:4 and lgkmcnt 11:8 left at maximum).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
    static_assert(N >= 0 && N < 64, "vmcnt is 6 bits");
    __builtin_amdgcn_s_waitcnt((N & 0xF) | ((N >> 4) << 14) | (0x7 << 4) | (0xF << 8));
}

// Workgroup barrier for a pipeline. __syncthreads() carries a release fence,
// which would make every wave drain ALL its outstanding DMAs (vmcnt(0)) --
// including the younger tiles that are meant to stay in flight. Here the
// wave first waits (explicitly, before calling this) for the DMAs of the tile
// about to be read, and the barrier only needs this wave's LDS reads of the
// stage about to be refilled to be complete (lgkmcnt(0)). The memory clobber
// keeps the compiler from moving LDS accesses across it.
__device__ __forceinline__ void stage_barrier() {
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

// LDS byte offset of a generic pointer into LDS: the low 32 bits of a flat
// address in the LDS aperture. Taken directly rather than through an
// address-space cast, whose null check this toolchain's backend rejects
// (an SGPR aperture operand in a VALU compare) in some kernels. Wave-uniform
// by contract; readfirstlane puts it in an SGPR where the compiler cannot
// prove the uniformity itself.
__device__ __forceinline__ unsigned lds_offset(const void* lds) {
    return __builtin_amdgcn_readfirstlane(static_cast<unsigned>(reinterpret_cast<uintptr_t>(lds)));
}

// One 16-byte-per-lane LDS-DMA load: lane l's 16 bytes at g land at
// lds + 16 l (lds wave-uniform). Issued from inline assembly so the
// compiler's wait-count bookkeeping does not see it: the compiler would
// otherwise drain every outstanding DMA (vmcnt(0)) before any read of a stage
// that still has one in flight, collapsing the pipeline. The kernel's own
// wait_vmcnt calls order the reads instead. M0 (the LDS base register of the
// instruction) is saved and restored around it.
__device__ __forceinline__ void dma16(const void* g, const void* lds) {
    const unsigned base = lds_offset(lds);
    unsigned saved;
    asm volatile(
        "s_mov_b32 %0, m0\n\t"
        "s_mov_b32 m0, %1\n\t"
        "s_nop 0\n\t"
        "global_load_lds_dwordx4 %2, off\n\t"
        "s_nop 0\n\t"
        "s_mov_b32 m0, %0"
        : "=&s"(saved)
        : "s"(base), "v"(g)
        : "memory");
}

// The same load addressed as a wave-uniform 64-bit base (SGPRs) plus this
// lane's 32-bit byte offset: no per-lane 64-bit address arithmetic. The
// base is uniform by contract; readfirstlane states it where the compiler
// cannot prove it (an "s" operand it has placed in VGPRs does not assemble).
__device__ __forceinline__ void dma16_off(const void* base_any, unsigned offset, const void* lds) {
    // readfirstlane returns a signed int: each word goes through unsigned
    // before widening, or a low word >= 2^31 would sign-extend into the high
    // one.
    const uint64_t b64 = reinterpret_cast<uintptr_t>(base_any);
    const uint64_t lo = static_cast<unsigned>(
        __builtin_amdgcn_readfirstlane(static_cast<int>(static_cast<unsigned>(b64))));
    const uint64_t hi = static_cast<unsigned>(
        __builtin_amdgcn_readfirstlane(static_cast<int>(static_cast<unsigned>(b64 >> 32))));
    const void* base = reinterpret_cast<const void*>(lo | (hi << 32));
    const unsigned lbase = lds_offset(lds);
    unsigned saved;
    asm volatile(
        "s_mov_b32 %0, m0\n\t"
        "s_mov_b32 m0, %1\n\t"
        "s_nop 0\n\t"
        "global_load_lds_dwordx4 %2, %3\n\t"
        "s_nop 0\n\t"
        "s_mov_b32 m0, %0"
        : "=&s"(saved)
        : "s"(lbase), "v"(offset), "s"(base)
        : "memory");
}

}  // namespace dotl
