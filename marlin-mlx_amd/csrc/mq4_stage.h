// LDS-DMA staging of packed weight lines, shared by the kernels that stream
// weights through LDS (mq4_rows.hip, mq4_lmring.hip).
#pragma once

#include "mq4_device.h"

namespace mq4 {
namespace stage {

// Weight lines staged by LDS DMA: one DMA instruction moves 64 lanes x 16
// bytes, eight lanes per 128-byte line (whole lines, the pattern that keeps
// the CU's load pipeline busy for the fewest cycles).  Within a line the
// eight 16-byte chunks go to the lanes rotated by (row / 2) % 8, so that the
// MFMA operand reads (16 rows x one chunk at a time) hit 16 distinct bank
// groups.  Line index G (row, or row + 16 x line-in-row) and chunk u live at
// 16-byte slot 8 G + ((u - (row >> 1)) & 7) of the staging buffer.
//
// LDS DMA is issued as inline assembly, so that the compiler does not track
// it: it would otherwise wait for every outstanding DMA of the wave before
// each LDS access.  The kernel waits for its DMA itself (wait_vmcnt), before
// the reads of the staged data and before the barriers after which other
// waves read it.  The compiler's own waits stay correct: vector memory
// operations complete in issue order, so a wait for a tracked load also
// covers untracked ones issued before it, and an untracked load issued
// after it only makes the wait stricter.  M0 holds the wave-uniform LDS
// destination; lane l writes bytes [size l, size (l + 1)) of it.
__device__ __forceinline__ uint32_t lds_addr(const void* p) {
    return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void*)p;
}
// (M0 is an operand, "{m0}", so the compiler sets it and knows it is used;
// the s_nop covers the wait state between an M0 write and the DMA.)
__device__ __forceinline__ void dma16(const void* src, const void* lds_dst) {
    asm volatile("s_nop 0\n\tglobal_load_lds_dwordx4 %0, off"
                 :: "v"(src), "{m0}"(__builtin_amdgcn_readfirstlane(lds_addr(lds_dst))) : "memory");
}
__device__ __forceinline__ void dma4(const void* src, const void* lds_dst) {
    asm volatile("s_nop 0\n\tglobal_load_lds_dword %0, off"
                 :: "v"(src), "{m0}"(__builtin_amdgcn_readfirstlane(lds_addr(lds_dst))) : "memory");
}

// The same DMA with a wave-uniform 64-bit base in scalar registers and a
// 32-bit per-lane byte offset (the saddr form): no vector address arithmetic
// per instruction.  `base` must be wave-uniform.
__device__ __forceinline__ void dma16_s(const void* base, uint32_t voff, const void* lds_dst) {
    asm volatile("s_nop 0\n\tglobal_load_lds_dwordx4 %0, %1"
                 :: "v"(voff), "s"(base), "{m0}"(__builtin_amdgcn_readfirstlane(lds_addr(lds_dst))) : "memory");
}
__device__ __forceinline__ void dma4_s(const void* base, uint32_t voff, const void* lds_dst) {
    asm volatile("s_nop 0\n\tglobal_load_lds_dword %0, %1"
                 :: "v"(voff), "s"(base), "{m0}"(__builtin_amdgcn_readfirstlane(lds_addr(lds_dst))) : "memory");
}

__device__ __forceinline__ int stage_slot(int G, int row, int u) { return 8 * G + ((u - (row >> 1)) & 7); }
__device__ __forceinline__ int stage_chunk(int slot, int row) { return ((slot & 7) + (row >> 1)) & 7; }

}  // namespace stage
}  // namespace mq4
