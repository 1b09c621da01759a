#pragma once

// Loads from global memory straight into LDS (gfx950 global_load_lds_dwordx4).
//
// Two compiler facts shape how kernels use them:
//  * the compiler does not count such a load as a write to the LDS array it
//    fills. A kernel whose only writes to an array are direct loads can see
//    its later reads of that array dropped as reads of unwritten memory, so
//    such kernels keep one ordinary store to the array that never runs;
//  * called inside a kernel template, the builtin made clang's host pass drop
//    the kernel's launch stub (an undefined symbol at load time), so kernels
//    call it through this plain __device__ function.
// A direct load is counted by vmcnt: `s_waitcnt vmcnt(0)` in every wave and a
// workgroup barrier must separate it from reads of what it wrote.

namespace opworks::detail {

// 16 bytes per lane: lane l of the wave writes lds_block + 16 l, whatever
// address it loads from. lds_block must be the same for every lane.
__device__ __forceinline__ void load_lds16(const void *src, void *lds_block) {
    __builtin_amdgcn_global_load_lds(src, (__attribute__((address_space(3))) void *)lds_block, 16, 0, 0);
}

// s_waitcnt operand (gfx9 encoding) for vmcnt(0) with expcnt and lgkmcnt at
// their maxima: waits until every vector memory access of the wave, direct
// loads included, has completed.
constexpr int kWaitVmcnt0Only = 0x0F70;

} // namespace opworks::detail
