/*
 * lds_dma.h - direct global->LDS loads for gfx950 and the explicit waits
 * that go with them (shared by gemm_dl.hip and skinny.hip).
 *
 * buffer_load_dwordx4 ... lds moves 16 bytes per lane from global memory
 * into LDS at M0 + 16*lane without passing through VGPRs; one
 * wave-instruction fills 1 KiB. Offsets at or past the descriptor's
 * num_records load zeros, so tails need no branches.
 */
#ifndef SAM3_LDS_DMA_H
#define SAM3_LDS_DMA_H

#include "s3k_dev.h"

namespace s3k {

typedef __attribute__((address_space(3))) void *lds_ptr_t;
typedef int s3k_i32x4 __attribute__((ext_vector_type(4)));

#define S3K_OOB 0x80000000u /* buffer offset beyond any range: loads zero */

/* Buffer descriptor of a raw byte range (gfx9 layout: base, stride 0,
 * num_records = bytes, dword3 = 0x00020000); offsets >= bytes load 0. */
__device__ __forceinline__ s3k_i32x4 buf_rsrc(const void *base, unsigned bytes)
{
	const unsigned long long a = (unsigned long long)base;
	return (s3k_i32x4){(int)(unsigned)a, (int)(unsigned)(a >> 32), (int)bytes, 0x00020000};
}

/* 16 bytes per lane from global (rsrc + voff) into LDS at lds + 16*lane.
 * Issued as inline asm so the compiler does not treat the LDS image as
 * written here: kernels order it with explicit vmcnt waits and a barrier
 * (the builtin form makes the compiler wait for every pending load before
 * any LDS read). */
__device__ __forceinline__ void dma16(const void *lds, s3k_i32x4 rsrc, unsigned voff)
{
	const unsigned m0 = __builtin_amdgcn_readfirstlane((unsigned)(size_t)(lds_ptr_t)lds);
	asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tbuffer_load_dwordx4 %1, %2, 0 offen lds"
		     :: "s"(m0), "v"(voff), "s"(rsrc) : "memory");
}

/* The same with the LDS address already a wave-uniform 32-bit LDS byte
 * address (no pointer arithmetic per load) and a scalar byte offset added
 * to every lane's voff: lanes whose voff is at or past num_records still
 * load zeros. */
__device__ __forceinline__ void dma16s(unsigned lds_addr, s3k_i32x4 rsrc, unsigned voff,
				       unsigned soff)
{
	asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tbuffer_load_dwordx4 %1, %2, %3 offen lds"
		     :: "s"(lds_addr), "v"(voff), "s"(rsrc), "s"(soff) : "memory");
}

/* 32-bit LDS address of a __shared__ object. */
__device__ __forceinline__ unsigned lds_addr_of(const void *p)
{
	return (unsigned)(size_t)(lds_ptr_t)p;
}

/* s_waitcnt vmcnt(N) with lgkm/exp counters left alone. */
template <int N>
__device__ __forceinline__ void wait_vm()
{
	static_assert(N >= 0 && N < 64, "vmcnt range");
	__builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

/* Workgroup barrier without the vmcnt(0) HIP's __syncthreads implies. */
__device__ __forceinline__ void wg_barrier()
{
	asm volatile("s_barrier" ::: "memory");
}

} /* namespace s3k */

#endif /* SAM3_LDS_DMA_H */
