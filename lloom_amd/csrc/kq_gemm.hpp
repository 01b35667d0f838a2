// kq_gemm.hpp -- pieces the LDS-tiled GEMMs share: the XCD-aware tile
// order and the global_load_lds issue.
#pragma once

#include "kq_common.hpp"

namespace lloom {

typedef int v16i __attribute__((ext_vector_type(16)));

// Tile order.  Workgroups are dealt round-robin to the 8 XCDs; renumber them
// XCD-major so each XCD gets a contiguous range, then walk that range in
// groups of GM m-blocks (column-major inside a group): the ~32 workgroups an
// XCD runs at once cover a 4 x 8 block of tiles whose activation and weight
// tiles fit its 4 MB L2, instead of re-reading them for every tile.
__device__ __forceinline__ void tile_of(int nbm, int nbn, int& bm, int& bn) {
    constexpr int GM = 4;
    int pid = blockIdx.x;
    if ((gridDim.x & 7) == 0) pid = (blockIdx.x & 7) * (gridDim.x >> 3) + (blockIdx.x >> 3);
    const int per_group = GM * nbn;
    const int group = pid / per_group;
    const int first = group * GM;
    const int gsz = min(nbm - first, GM);
    const int in = pid - group * per_group;
    bm = first + in % gsz;
    bn = in / gsz;
}

// global_load_lds written as the instruction: the compiler does not see
// these LDS writes, so it adds no vmcnt(0) in front of later LDS reads it
// cannot prove disjoint from them; the kernel orders them itself (counted
// vmcnt waits, then s_barrier).  The LDS destination goes to m0 through an
// operand constraint, so the compiler itself writes m0 (and knows it is
// taken) before each load; the s_nop covers the m0-write-to-LDS-DMA hazard.
__device__ __forceinline__ uint32_t lds_addr(const void* p) {
    return (uint32_t)(uintptr_t)(__attribute__((address_space(3))) const uint8_t*)p;
}
// From a wave-uniform base (SGPRs) plus a 32-bit per-lane offset, to a
// wave-uniform LDS destination: the per-step address arithmetic is scalar.
__device__ __forceinline__ void dma16s(const void* base, uint32_t voff, uint32_t lds) {
    asm volatile("s_nop 0\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(voff), "s"(base), "{m0}"(lds) : "memory");
}
__device__ __forceinline__ void dma4s(const void* base, uint32_t voff, uint32_t lds) {
    asm volatile("s_nop 0\n\tglobal_load_lds_dword %0, %1" ::"v"(voff), "s"(base), "{m0}"(lds) : "memory");
}

// Raise a kernel's dynamic LDS limit.  Called before every launch: the call
// is host-only and cheap, it holds for the current device whichever that
// is, and no process-wide flag is shared between threads.
inline hipError_t set_lds_limit(const void* kernel, int bytes) {
    return hipFuncSetAttribute(kernel, hipFuncAttributeMaxDynamicSharedMemorySize, bytes);
}

}  // namespace lloom
