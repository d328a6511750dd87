// LDS DMA and an LDS-only barrier for the pipelined matrix-core kernels (conv3.hip, gemm.hip).
//
// global_load_lds_dwordx4 copies 16 bytes a lane from global memory straight into LDS (lane l at
// M0 + 16 l). Issued through the compiler's builtin, the copy makes the compiler wait for every
// copy in flight (vmcnt(0)) before any later LDS access it cannot prove disjoint, and
// __syncthreads waits for all memory operations: both would expose the latency the pipelines
// hide. Issued here, the copies are invisible to the compiler, so each kernel waits for them
// itself with explicit vmcnt counts before the barrier that publishes their data.
#pragma once

#include <hip/hip_runtime.h>

namespace ocr {

typedef __attribute__((address_space(3))) void *lds_ptr;

// 16 bytes from src (per lane) to LDS at dst + 16 * lane; dst must be the same for the whole
// wavefront. Completion: vmcnt.
__device__ inline void dma16(const void *src, void *dst) {
    const unsigned m0 = __builtin_amdgcn_readfirstlane(unsigned(reinterpret_cast<size_t>((lds_ptr)dst)));
    asm volatile("s_nop 0\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(src), "{m0}"(m0) : "memory");
}

// The same with the address as a uniform 64-bit base plus a per-lane 32-bit byte offset (the
// scalar-base addressing form: the per-lane part stays fixed while the base moves).
__device__ inline void dma16s(const void *base, unsigned voff, void *dst) {
    const unsigned m0 = __builtin_amdgcn_readfirstlane(unsigned(reinterpret_cast<size_t>((lds_ptr)dst)));
    asm volatile("s_nop 0\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(voff), "s"(base), "{m0}"(m0) : "memory");
}

// The byte address in LDS of p, a pointer into __shared__ memory.
__device__ inline unsigned lds_addr(const void *p) { return unsigned(reinterpret_cast<size_t>((lds_ptr)p)); }

// The same copies with the LDS destination as a byte address (uniform) and no memory clobber:
// the compiler keeps values it loaded across them (kernel arguments, tables) instead of loading
// them again, and may move ordinary loads and stores across them. Only for copies into a buffer
// that nothing reads or writes before the explicit wait and the barrier that publish it; the
// copies keep their order with respect to every other asm statement (the waits, the barriers).
__device__ inline void dma16_to(const void *src, unsigned lds) {
    asm volatile("s_nop 0\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(src), "{m0}"(__builtin_amdgcn_readfirstlane(lds)));
}
__device__ inline void dma16s_to(const void *base, unsigned voff, unsigned lds) {
    asm volatile("s_nop 0\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(voff), "s"(base),
                 "{m0}"(__builtin_amdgcn_readfirstlane(lds)));
}

// Workgroup barrier for LDS: this wavefront's LDS operations are complete and no memory operation
// moves across it; global loads, stores and LDS DMA stay in flight.
__device__ inline void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

}  // namespace ocr
