/*
 * gemm_dl.hip - bf16/f16 GEMM C = A * W^T (A [M,K], W [N,K], both k
 * contiguous) for gfx950 with direct global->LDS loads. This is the
 * production layout of sam3.c's linear layers once gh_linear's weight
 * transpose is folded (graph_helpers.c:297-320), and of attention's
 * Q K^T per head. Reference kernel: cpu_matmul_bf16.c:103-141 (f32
 * accumulate, one rounding of the output).
 *
 * Pipeline (per workgroup of NW waves, tile BM x BN, k-step BK):
 *   - buffer_load_dwordx4 ... lds moves 16 bytes per lane straight into
 *     LDS (no VGPR staging); a wave-instruction fills 1 KiB, i.e. 64
 *     consecutive 16-byte chunks. Each lane picks the global chunk whose
 *     swizzled LDS slot is lane-th of that KiB, so the LDS image has rows
 *     of BK k-values with the chunk index XOR-permuted per row
 *     (lds_swz: conflict-free 128-bit reads by 8 or 16 consecutive rows).
 *   - Rows past M/N and chunks past K are given an out-of-range buffer
 *     offset; the buffer unit returns zeros for them, so tails need no
 *     branches.
 *   - STAGES-deep ring: at step kt the loads of step kt+STAGES-1 are in
 *     flight while step kt is multiplied. Completion is tracked with an
 *     explicit s_waitcnt vmcnt(loads of the younger stages) followed by
 *     s_barrier; HIP's __syncthreads would wait for every load.
 *   - MFMA v_mfma_f32_32x32x16_{bf16,f16}, wave tile (BM/WGM) x (BN/WGN),
 *     with W as the first operand: the MFMA forms C^T, so a lane holds
 *     four consecutive columns of one row (same products and sums as A W^T).
 *   - Epilogue through LDS with 16-byte stores (gemm_common.h); the
 *     transposed accumulators are staged with 16-byte LDS writes.
 */
#include "gemm_common.h"
#include "lds_dma.h"

namespace s3k {

template <int CPR>
__device__ __forceinline__ int dl_off(int row, int c)
{
	return (row * CPR + (c ^ lds_swz<CPR>(row))) << 4;
}

/* The S3K_EPI_QKV epilogue needs f32 output and wave tiles whose width
 * in 4-column units divides 64 (each lane keeps its columns for the
 * whole tile); it is built for the pipelined kernel only. */
__host__ __device__ constexpr bool qkv_tiles(int ck, int wtn)
{
	return ck == S3K_F32 && 64 % (wtn / 4) == 0;
}

template <int BM, int BN, int BK, int WGM, int WGN, int STAGES, int FAM, int CK, int OCC>
__global__ void __launch_bounds__(64 * WGM * WGN, OCC) gemm_dl(GemmArgs p)
{
	constexpr int NW = WGM * WGN;
	constexpr int CPR = BK / 8;
	constexpr int A_BYTES = BM * BK * 2, B_BYTES = BN * BK * 2;
	constexpr int SB = A_BYTES + B_BYTES;
	constexpr int A_INS = BM * CPR / 64, B_INS = BN * CPR / 64; /* KiB per stage */
	static_assert(A_INS % NW == 0 && B_INS % NW == 0, "loads split evenly over waves");
	constexpr int A_PER = A_INS / NW, B_PER = B_INS / NW;
	constexpr int LOADS = A_PER + B_PER; /* vm ops per wave per stage */
	constexpr int WTM = BM / WGM, WTN = BN / WGN;
	constexpr int FM = WTM / 32, FN = WTN / 32;
	constexpr int KS = BK / 16;
	static_assert(NW * 32 * (WTN + 8) * 4 <= STAGES * SB, "epilogue staging fits");
	__shared__ __attribute__((aligned(1024))) char smem[STAGES * SB];

	const int lane = threadIdx.x & 63;
	const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
	const int wm0 = (wave / WGN) * WTM, wn0 = (wave % WGN) * WTN;
	const int bz = blockIdx.y;
	const unsigned lds0 = lds_addr_of(smem);
	int tm, tn;
	tile_of(blockIdx.x, p.tiles_m, p.tiles_n, tm, tn);

	const s3k_i32x4 ra = buf_rsrc(p.a + bz * p.sa_b, p.a_extent);
	const s3k_i32x4 rb = buf_rsrc(p.b + bz * p.sb_b, p.b_extent);

	/* Per-lane source of each load instruction (fixed across k). */
	unsigned a_off[A_PER], b_off[B_PER];
	int a_k[A_PER], b_k[B_PER];
#pragma unroll
	for (int j = 0; j < A_PER; ++j) {
		const int s = (j * NW + wave) * 64 + lane;
		const int row = s / CPR, c = (s % CPR) ^ lds_swz<CPR>(row);
		const int g = tm * BM + row;
		a_off[j] = g < p.M ? (unsigned)(g * p.lda_b + c * 16) : S3K_OOB;
		a_k[j] = c * 8;
	}
#pragma unroll
	for (int j = 0; j < B_PER; ++j) {
		const int s = (j * NW + wave) * 64 + lane;
		const int row = s / CPR, c = (s % CPR) ^ lds_swz<CPR>(row);
		const int g = tn * BN + row;
		b_off[j] = g < p.N ? (unsigned)(g * p.ldb_b + c * 16) : S3K_OOB;
		b_k[j] = c * 8;
	}

	/* A whole k-step moves every lane's chunk by 2*k0 bytes: that goes in
	 * the scalar offset (rows past M/N keep an offset past the range). Only
	 * a k-step that crosses K selects chunks per lane. */
	auto issue = [&](int kt) {
		const int k0 = kt * BK;
		const unsigned st = lds0 + (unsigned)((kt % STAGES) * SB) + (unsigned)wave * 1024u;
		if (k0 + BK <= p.K) {
#pragma unroll
			for (int j = 0; j < A_PER; ++j)
				dma16s(st + j * NW * 1024, ra, a_off[j], 2u * k0);
#pragma unroll
			for (int j = 0; j < B_PER; ++j)
				dma16s(st + A_BYTES + j * NW * 1024, rb, b_off[j], 2u * k0);
		} else {
#pragma unroll
			for (int j = 0; j < A_PER; ++j) {
				const unsigned o = k0 + a_k[j] < p.K ? a_off[j] + 2u * k0 : S3K_OOB;
				dma16s(st + j * NW * 1024, ra, o, 0u);
			}
#pragma unroll
			for (int j = 0; j < B_PER; ++j) {
				const unsigned o = k0 + b_k[j] < p.K ? b_off[j] + 2u * k0 : S3K_OOB;
				dma16s(st + A_BYTES + j * NW * 1024, rb, o, 0u);
			}
		}
	};

	s3k_f32x16 acc[FM][FN];
#pragma unroll
	for (int i = 0; i < FM; ++i)
#pragma unroll
		for (int j = 0; j < FN; ++j)
#pragma unroll
			for (int r = 0; r < 16; ++r)
				acc[i][j][r] = 0.0f;

	const int nk = (p.K + BK - 1) / BK;
#pragma unroll
	for (int s = 0; s < STAGES - 1; ++s)
		if (s < nk)
			issue(s);

	for (int kt = 0; kt < nk; ++kt) {
		/* own loads of step kt done: at most the younger stages pending */
		const int younger = min(nk - 1 - kt, STAGES - 2);
		if (younger >= 2)
			wait_vm<2 * LOADS>();
		else if (younger == 1)
			wait_vm<LOADS>();
		else
			wait_vm<0>();
		wg_barrier();
		if (kt + STAGES - 1 < nk)
			issue(kt + STAGES - 1);

		const char *As = smem + (kt % STAGES) * SB;
		const char *Bs = As + A_BYTES;
		/* fragments of k-step ks+1 are read while the MFMAs of ks run */
		uint4 af[2][FM], bfr[2][FN];
#pragma unroll
		for (int i = 0; i < FM; ++i)
			af[0][i] = *(const uint4 *)(As + dl_off<CPR>(wm0 + i * 32 + (lane & 31), lane >> 5));
#pragma unroll
		for (int j = 0; j < FN; ++j)
			bfr[0][j] = *(const uint4 *)(Bs + dl_off<CPR>(wn0 + j * 32 + (lane & 31), lane >> 5));
#pragma unroll
		for (int ks = 0; ks < KS; ++ks) {
			const int cur = ks & 1;
			if (ks + 1 < KS) {
				const int c = 2 * (ks + 1) + (lane >> 5);
#pragma unroll
				for (int i = 0; i < FM; ++i)
					af[cur ^ 1][i] = *(const uint4 *)(As + dl_off<CPR>(wm0 + i * 32 + (lane & 31), c));
#pragma unroll
				for (int j = 0; j < FN; ++j)
					bfr[cur ^ 1][j] = *(const uint4 *)(Bs + dl_off<CPR>(wn0 + j * 32 + (lane & 31), c));
			}
			__builtin_amdgcn_s_setprio(1);
#pragma unroll
			for (int i = 0; i < FM; ++i)
#pragma unroll
				for (int j = 0; j < FN; ++j)
					mfma_chunk<FAM>(acc[i][j], bfr[cur][j], af[cur][i]);
			__builtin_amdgcn_s_setprio(0);
		}
	}

	__syncthreads();
	write_tile_ck<FM, FN, WTN, CK, true>(p, acc, smem, wave, lane, tm * BM + wm0, tn * BN + wn0, bz);
}

/*
 * gemm_dlp: the same GEMM for K % 64 == 0 with a software pipeline that
 * keeps the matrix cores fed across k-steps (BK 64, two LDS stages).
 *   - LDS holds [A stage 0 | A stage 1 | B stage 0 | B stage 1], so every
 *     fragment read is one of eight per-lane base registers plus an
 *     immediate (the swizzle of fragment i is that of fragment 0 with the
 *     chunk's bit 2 flipped when i is odd).
 *   - Sub-steps 0-2 of a k-step read the next sub-step's fragments while
 *     their MFMAs issue. Before sub-step 3 a wave waits for its own LDS
 *     reads and for the next stage's DMA, and the workgroup meets at the
 *     barrier; the MFMAs issued before it keep the matrix pipe busy. Then
 *     sub-step 3's MFMAs issue together with the next stage's first
 *     fragment reads and the DMA of k-step kt + 2 into the stage every
 *     wave has just finished reading (INTER: one read or DMA after each
 *     MFMA; else grouped after them).
 *   - The steady-state loop has no branches: the last two k-steps are
 *     peeled.
 * Same per-element accumulation order as gemm_dl, so the same bits.
 */

/* QKV: the S3K_EPI_QKV epilogue (f32 output), instead of C */
template <int BM, int BN, int WGM, int WGN, int FAM, int CK, bool INTER, bool QKV = false>
__global__ void __launch_bounds__(64 * WGM * WGN, 1) gemm_dlp(GemmArgs p)
{
	constexpr int NW = WGM * WGN, BK = 64, CPR = 8;
	constexpr int A_BYTES = BM * BK * 2, B_BYTES = BN * BK * 2; /* one stage */
	constexpr int B_BASE = 2 * A_BYTES, LDS_BYTES = 2 * (A_BYTES + B_BYTES);
	static_assert((BM / 8) % NW == 0 && (BN / 8) % NW == 0, "loads split evenly over waves");
	constexpr int A_PER = BM / 8 / NW, B_PER = BN / 8 / NW, LOADS = A_PER + B_PER;
	constexpr int WTM = BM / WGM, WTN = BN / WGN;
	constexpr int FM = WTM / 32, FN = WTN / 32, NMF = FM * FN, NRD = FM + FN;
	static_assert(A_BYTES + (FM - 1) * 4096 < 65536 && B_BYTES + (FN - 1) * 4096 < 65536,
		      "fragment offsets fit the LDS instruction's immediate");
	static_assert(NW * 32 * (WTN + 8) * 4 <= LDS_BYTES, "epilogue staging fits");
	__shared__ __attribute__((aligned(1024))) char smem[LDS_BYTES];

	const int lane = threadIdx.x & 63;
	const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
	const int wm0 = (wave / WGN) * WTM, wn0 = (wave % WGN) * WTN;
	const int bz = blockIdx.y;
	const unsigned lds0 = lds_addr_of(smem);
	int tm, tn;
	tile_of(blockIdx.x, p.tiles_m, p.tiles_n, tm, tn, p.tstrip);
	const s3k_i32x4 ra = buf_rsrc(p.a + bz * p.sa_b, p.a_extent);
	const s3k_i32x4 rb = buf_rsrc(p.b + bz * p.sb_b, p.b_extent);

	/* per-lane source of DMA instruction t (A rows first, then B); rows
	 * past M / N read zeros */
	unsigned off[LOADS];
#pragma unroll
	for (int t = 0; t < LOADS; ++t) {
		const bool isa = t < A_PER;
		const int s = ((isa ? t : t - A_PER) * NW + wave) * 64 + lane;
		const int row = s / CPR, c = (s % CPR) ^ lds_swz<CPR>(row);
		const int g = (isa ? tm * BM : tn * BN) + row;
		off[t] = g < (isa ? p.M : p.N) ? (unsigned)(g * (isa ? p.lda_b : p.ldb_b) + c * 16)
					       : S3K_OOB;
	}
	auto dma = [&](int kt, int t, int stg) {
		if (t < A_PER)
			dma16s(lds0 + (unsigned)(stg * A_BYTES + (t * NW + wave) * 1024), ra, off[t],
			       (unsigned)(kt * BK * 2));
		else
			dma16s(lds0 + (unsigned)(B_BASE + stg * B_BYTES + ((t - A_PER) * NW + wave) * 1024),
			       rb, off[t], (unsigned)(kt * BK * 2));
	};

	unsigned abase[4], bbase[4];
	{
		const int l32 = lane & 31, h = lane >> 5, r0 = wm0 + l32, r1 = wn0 + l32;
#pragma unroll
		for (int ks = 0; ks < 4; ++ks) {
			abase[ks] = lds0 + (unsigned)((r0 * CPR + ((2 * ks + h) ^ lds_swz<CPR>(r0))) << 4);
			bbase[ks] = lds0 + B_BASE +
				    (unsigned)((r1 * CPR + ((2 * ks + h) ^ lds_swz<CPR>(r1))) << 4);
		}
	}

	s3k_f32x16 acc[FM][FN];
#pragma unroll
	for (int i = 0; i < FM; ++i)
#pragma unroll
		for (int j = 0; j < FN; ++j)
#pragma unroll
			for (int r = 0; r < 16; ++r)
				acc[i][j][r] = 0.0f;

	uint4 af[2][FM], bf[2][FN];
	/* read r of a sub-step: the FM A fragments, then the FN B fragments */
	auto frag = [&](int buf, int stg, int ks, int r) {
		if (r < FM)
			af[buf][r] = lds_rd16(abase[ks ^ (2 * (r & 1))], (unsigned)(stg * A_BYTES + r * 4096));
		else
			bf[buf][r - FM] = lds_rd16(bbase[ks ^ (2 * ((r - FM) & 1))],
						   (unsigned)(stg * B_BYTES + (r - FM) * 4096));
	};

	/* k-step kt from stage stg; next: a k-step follows; dmak: issue the
	 * DMA of k-step kt + 2 into stg */
	auto step = [&](int stg, int kt, bool next, bool dmak) {
#pragma unroll
		for (int ks = 0; ks < 4; ++ks) {
			const int cur = ks & 1, nxt = cur ^ 1;
			if (ks == 3) {
				__builtin_amdgcn_s_waitcnt(0xC07F); /* lgkmcnt(0): own reads done */
				if (next) {
					wait_vm<0>();
					wg_barrier();
				}
			}
			__builtin_amdgcn_sched_barrier(0);
#pragma unroll
			for (int m = 0; m < NMF; ++m) {
				mfma_chunk<FAM>(acc[m / FN][m % FN], bf[cur][m % FN], af[cur][m / FN]);
				if (INTER) {
					if (ks < 3) {
						if (m < NRD)
							frag(nxt, stg, ks + 1, m);
					} else {
						if (next && m < NRD)
							frag(0, stg ^ 1, 0, m);
						if (dmak && m < LOADS)
							dma(kt + 2, m, stg);
					}
					__builtin_amdgcn_sched_barrier(0);
				}
			}
			const int r0 = INTER ? NMF : 0;
#pragma unroll
			for (int r = r0; r < NRD; ++r) {
				if (ks < 3)
					frag(nxt, stg, ks + 1, r);
				else if (next)
					frag(0, stg ^ 1, 0, r);
			}
			if (ks == 3 && dmak) {
#pragma unroll
				for (int t = r0; t < LOADS; ++t)
					dma(kt + 2, t, stg);
			}
		}
	};

	const int nk = p.K / BK;
#pragma unroll
	for (int t = 0; t < LOADS; ++t)
		dma(0, t, 0);
	if (nk > 1) {
#pragma unroll
		for (int t = 0; t < LOADS; ++t)
			dma(1, t, 1);
		wait_vm<LOADS>();
	} else {
		wait_vm<0>();
	}
	wg_barrier();
#pragma unroll
	for (int r = 0; r < NRD; ++r)
		frag(0, 0, 0, r);
	int kt = 0;
	for (; kt + 2 < nk; ++kt)
		step(kt & 1, kt, true, true);
	if (kt + 1 < nk) {
		step(kt & 1, kt, true, false);
		++kt;
	}
	step(kt & 1, kt, false, false);

	__syncthreads();
	write_tile_ck<FM, FN, WTN, CK, true, QKV>(p, acc, smem, wave, lane, tm * BM + wm0,
						 tn * BN + wn0, bz);
}

/* One k-step GEMMs (K = 64: the attention scores Q K^T, batched over
 * windows and heads). With a single k-step a workgroup loads, multiplies
 * once and stores, and the next workgroup on the CU starts only after
 * that: the output stores, most of the bytes, do not overlap anything.
 * Here workgroups are persistent: each walks the tiles (all batch slices
 * together) gridDim.x apart, and after the MFMAs of tile i it issues the
 * direct-to-LDS loads of tile i + 1 into the other panel buffer and only
 * then the stores of tile i, so that waiting for those loads does not
 * wait for the stores (vmcnt counts both, in order). 192x192 tiles of
 * four 96x96 wave tiles; M and N multiples of 192, whole tiles only, so
 * every lane issues the same number of stores (the epilogue's fast
 * path) and the wait counts below are exact. Same MFMA sequence per
 * output as gemm_dl / gemm_dlp, so the same bits. */
constexpr int DLK_B = 192;

template <int FAM, int CK, int WGN>
__global__ void __launch_bounds__(128 * WGN, 1) gemm_dlk(GemmArgs p, int total)
{
	constexpr int BM = DLK_B, BN = DLK_B, NW = 2 * WGN, BK = 64, CPR = 8;
	constexpr int A_BYTES = BM * BK * 2, B_BYTES = BN * BK * 2, STAGE = A_BYTES + B_BYTES;
	constexpr int A_PER = BM / 8 / NW, B_PER = BN / 8 / NW, LOADS = A_PER + B_PER;
	constexpr int WTM = BM / 2, WTN = BN / WGN, FM = WTM / 32, FN = WTN / 32;
	constexpr int W = CK == S3K_F32 ? 4 : 8;
	constexpr int STORES = FM * (32 * WTN / W) / 64;   /* per lane and tile */
	static_assert((32 * WTN / W) % 64 == 0, "whole store rounds");
	static_assert(LOADS + STORES < 64, "vmcnt range");
	constexpr int STG = NW * 32 * (WTN + 4) * 4;      /* epilogue staging (transposed tiles) */
	__shared__ __attribute__((aligned(1024))) char smem[2 * STAGE + STG];

	const int lane = threadIdx.x & 63;
	const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
	const int wm0 = (wave / WGN) * WTM, wn0 = (wave % WGN) * WTN;
	const unsigned lds0 = lds_addr_of(smem);
	const int per_slice = p.tiles_m * p.tiles_n;

	/* per-lane chunk of DMA instruction t within a panel (rows past M / N
	 * never occur: whole tiles) */
	unsigned rowoff_a[A_PER], rowoff_b[B_PER];
#pragma unroll
	for (int t = 0; t < LOADS; ++t) {
		const bool isa = t < A_PER;
		const int s = ((isa ? t : t - A_PER) * NW + wave) * 64 + lane;
		const int row = s / CPR, c = (s % CPR) ^ lds_swz<CPR>(row);
		if (isa)
			rowoff_a[t] = (unsigned)(row * p.lda_b + c * 16);
		else
			rowoff_b[t - A_PER] = (unsigned)(row * p.ldb_b + c * 16);
	}
	/* tile -> (slice, tm, tn) and its panels' loads into buffer b */
	auto coords = [&](int t, int &bz, int &tm, int &tn) {
		bz = t / per_slice;
		tile_of(t - bz * per_slice, p.tiles_m, p.tiles_n, tm, tn);
	};
	auto load_tile = [&](int t, int b) {
		int bz, tm, tn;
		coords(t, bz, tm, tn);
		const s3k_i32x4 ra = buf_rsrc(p.a + bz * p.sa_b, p.a_extent);
		const s3k_i32x4 rb = buf_rsrc(p.b + bz * p.sb_b, p.b_extent);
		const unsigned oa = (unsigned)(tm * BM * p.lda_b), ob = (unsigned)(tn * BN * p.ldb_b);
#pragma unroll
		for (int u = 0; u < A_PER; ++u)
			dma16s(lds0 + (unsigned)(b * STAGE + (u * NW + wave) * 1024), ra, rowoff_a[u], oa);
#pragma unroll
		for (int u = 0; u < B_PER; ++u)
			dma16s(lds0 + (unsigned)(b * STAGE + A_BYTES + (u * NW + wave) * 1024), rb,
			       rowoff_b[u], ob);
	};

	unsigned abase[4], bbase[4];
	{
		const int l32 = lane & 31, h = lane >> 5, r0 = wm0 + l32, r1 = wn0 + l32;
#pragma unroll
		for (int ks = 0; ks < 4; ++ks) {
			abase[ks] = lds0 + (unsigned)((r0 * CPR + ((2 * ks + h) ^ lds_swz<CPR>(r0))) << 4);
			bbase[ks] = lds0 + A_BYTES +
				    (unsigned)((r1 * CPR + ((2 * ks + h) ^ lds_swz<CPR>(r1))) << 4);
		}
	}

	/* the walk: tile t = w, w + G, ... (G workgroups); or (xcd walk,
	 * G % 8 == 0) workgroup w, the (w / 8)-th of XCD w % 8 (workgroups
	 * are dispatched to the 8 XCDs round-robin), takes items w / 8,
	 * w / 8 + G / 8, ... of its XCD's list, the tiles of slices
	 * w % 8, w % 8 + 8, ...: a slice's tiles run on one XCD, whose L2
	 * then serves its panels to all of them */
	const bool xw = p.xwalk && (gridDim.x & 7) == 0;
	const int xr = (int)gridDim.x >> 3, xx = (int)blockIdx.x & 7;
	const int nslice = total / per_slice;
	const int xn = xw ? ((nslice - xx + 7) >> 3) * per_slice : 0;
	auto tile_at = [&](int q) { /* item q of this XCD's list */
		const int sl = q / per_slice;
		return (xx + 8 * sl) * per_slice + (q - sl * per_slice);
	};
	int q = xw ? (int)blockIdx.x >> 3 : (int)blockIdx.x;
	const int qend = xw ? xn : total, qstep = xw ? xr : (int)gridDim.x;
	if (q >= qend)
		return;
	int t = xw ? tile_at(q) : q;
	load_tile(t, 0);
	for (int i = 0; q < qend; ++i, q += qstep, t = xw ? tile_at(q) : q) {
		const int b = i & 1;
		/* this tile's panels: issued before the previous tile's stores */
		if (i == 0)
			wait_vm<0>();
		else
			wait_vm<STORES>();
		wg_barrier();
		s3k_f32x16 acc[FM][FN];
#pragma unroll
		for (int x = 0; x < FM; ++x)
#pragma unroll
			for (int y = 0; y < FN; ++y)
#pragma unroll
				for (int r = 0; r < 16; ++r)
					acc[x][y][r] = 0.0f;
#pragma unroll
		for (int ks = 0; ks < 4; ++ks) {
			uint4 af[FM], bf[FN];
			/* block x starts 32x rows further down: an odd x flips bit 2
			 * of the row's chunk permutation, i.e. k-substep ks ^ 2 */
#pragma unroll
			for (int x = 0; x < FM; ++x)
				af[x] = lds_rd16(abase[ks ^ (2 * (x & 1))], (unsigned)(b * STAGE + x * 4096));
#pragma unroll
			for (int y = 0; y < FN; ++y)
				bf[y] = lds_rd16(bbase[ks ^ (2 * (y & 1))], (unsigned)(b * STAGE + y * 4096));
			__builtin_amdgcn_s_waitcnt(0xC07F); /* lgkmcnt(0) */
#pragma unroll
			for (int x = 0; x < FM; ++x)
#pragma unroll
				for (int y = 0; y < FN; ++y)
					mfma_chunk<FAM>(acc[x][y], bf[y], af[x]);
		}
		/* every wave is done with buffer b ^ 1 (read in the previous
		 * tile) and with its own fragment reads of b */
		wg_barrier();
		if (q + qstep < qend)
			load_tile(xw ? tile_at(q + qstep) : q + qstep, b ^ 1);
		int bz, tm, tn;
		coords(t, bz, tm, tn);
		write_tile_ck<FM, FN, WTN, CK, true>(p, acc, smem + 2 * STAGE, wave, lane, tm * BM + wm0,
						      tn * BN + wn0, bz);
	}
}

/* B stored [K, N] (n contiguous: the attention's P V, whose V is
 * [keys, head dim]) with a narrow N: both panels arrive in LDS by
 * direct-to-LDS loads as they lie in memory, and the B fragments (eight
 * consecutive k of one n per lane, as the MFMA's first operand) are read
 * with ds_read_b64_tr_b16, which hands lane i of each 16-lane group
 * element i % 4 of the 8 bytes addressed by lanes i / 4 + 4q, q = 0..3:
 * with lane j of the group addressing row k0 + j / 4, columns
 * n0 + 4 (j % 4).., lane i receives rows k0..k0 + 3 of column n0 + i.
 * Two such reads give the lane's eight k. BMxBN tiles of WGM x WGN wave
 * tiles, k-steps of 64 double-buffered (192x64 for N <= 128, 192x256
 * for wide N); K a multiple of 64; rows past M read zeros and columns
 * past N are never stored. Same MFMA sequence per output as the other
 * kernels. */
typedef short dlt_v4i16 __attribute__((ext_vector_type(4)));

/* B's 16-byte chunks sit XOR-swizzled by k row so that the eight rows
 * one transposing read touches (row bits 0, 1 and 3) fall in different
 * banks; bits 2, 4 and 5 leave the swizzle unchanged, so the read's k
 * offsets stay immediates. */
template <int BCH>
__device__ __forceinline__ int dlt_bswz(int row)
{
	return BCH >= 32 ? 4 * ((row & 3) | ((row >> 1) & 4)) : 4 * ((row >> 1) & 1);
}

__device__ __forceinline__ uint2 dlt_read_tr(unsigned addr)
{
	const dlt_v4i16 r = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
		(__attribute__((address_space(3))) dlt_v4i16 *)(size_t)addr);
	return __builtin_bit_cast(uint2, r);
}

template <int BM, int BN, int WGM, int WGN, int OCC, int FAM, int CK>
__global__ void __launch_bounds__(64 * WGM * WGN, OCC) gemm_dlt(GemmArgs p)
{
	constexpr int BK = 64, NW = WGM * WGN, CPR = 8, BCH = BN / 8; /* B: 16-byte chunks per k row */
	constexpr int WTM = BM / WGM, WTN = BN / WGN, FM = WTM / 32, FN = WTN / 32;
	constexpr int A_BYTES = BM * BK * 2, B_BYTES = BK * BN * 2, STAGE = A_BYTES + B_BYTES;
	constexpr int A_PER = BM * CPR / 64 / NW, B_PER = BK * BCH / 64 / NW;
	static_assert(BM * CPR % (64 * NW) == 0 && BK * BCH % (64 * NW) == 0, "loads split evenly");
	constexpr int LOADS = A_PER + B_PER, LDS_BYTES = 2 * STAGE;
	static_assert(NW * 32 * (WTN + 8) * 4 <= LDS_BYTES, "epilogue staging fits");
	__shared__ __attribute__((aligned(1024))) char smem[LDS_BYTES];

	const int lane = threadIdx.x & 63;
	const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
	const int wm0 = (wave / WGN) * WTM, wn0 = (wave % WGN) * WTN;
	/* slice bz, tile tt: a 2-D grid (tiles, slices), or with xwalk a 1-D
	 * one in which the tiles of 8 slices in a row form a group, ordered
	 * so that each slice's tiles share a residue mod 8: workgroups go to
	 * the 8 XCDs round-robin, so a slice's tiles run on one XCD and its
	 * panels are fetched into one L2 */
	int bz = blockIdx.y, tt = blockIdx.x;
	if (p.xwalk) {
		const int ps = p.tiles_m * p.tiles_n, L = blockIdx.x;
		const int g8 = (p.xwalk >> 3) * 8 * ps; /* p.xwalk: the slice count */
		if (L < g8) {
			const int g = L / (8 * ps), r = L - g * 8 * ps;
			bz = 8 * g + (r & 7);
			tt = r >> 3;
		} else {
			bz = (p.xwalk >> 3) * 8 + (L - g8) / ps;
			tt = (L - g8) % ps;
		}
		/* uniform, but the integer division leaves them in vector
		 * registers: the direct-to-LDS loads need scalar ones */
		bz = __builtin_amdgcn_readfirstlane(bz);
		tt = __builtin_amdgcn_readfirstlane(tt);
	}
	const unsigned lds0 = lds_addr_of(smem);
	int tm, tn;
	tile_of(tt, p.tiles_m, p.tiles_n, tm, tn);
	const s3k_i32x4 ra = buf_rsrc(p.a + bz * p.sa_b, p.a_extent);
	const s3k_i32x4 rb = buf_rsrc(p.b + bz * p.sb_b, p.b_extent);

	/* A: rows of 8 swizzled 16-byte chunks (rows past M read zeros); B:
	 * k rows of BN n in BCH chunks, in memory order */
	unsigned off[LOADS];
#pragma unroll
	for (int t = 0; t < LOADS; ++t) {
		if (t < A_PER) {
			const int s = (t * NW + wave) * 64 + lane;
			const int row = s / CPR, c = (s % CPR) ^ lds_swz<CPR>(row);
			off[t] = tm * BM + row < p.M ? (unsigned)((tm * BM + row) * p.lda_b + c * 16)
						    : S3K_OOB;
		} else {
			const int s = ((t - A_PER) * NW + wave) * 64 + lane;
			const int kr = s / BCH, c = (s % BCH) ^ dlt_bswz<BCH>(kr);
			off[t] = (unsigned)(kr * p.ldb_b + tn * BN * 2 + c * 16);
		}
	}
	auto dma = [&](int kt, int stg) {
#pragma unroll
		for (int t = 0; t < LOADS; ++t) {
			if (t < A_PER)
				dma16s(lds0 + (unsigned)(stg * STAGE + (t * NW + wave) * 1024), ra, off[t],
				       (unsigned)(kt * BK * 2));
			else
				dma16s(lds0 + (unsigned)(stg * STAGE + A_BYTES + ((t - A_PER) * NW + wave) * 1024),
				       rb, off[t], (unsigned)(kt * BK * p.ldb_b));
		}
	};

	unsigned abase[4];
	{
		const int l32 = lane & 31, h = lane >> 5, r0 = wm0 + l32;
#pragma unroll
		for (int ks = 0; ks < 4; ++ks)
			abase[ks] = lds0 + (unsigned)((r0 * CPR + ((2 * ks + h) ^ lds_swz<CPR>(r0))) << 4);
	}
	/* B fragment read r (k 4r..4r+3 of the lane's eight) of k-substep ks:
	 * lane j of its group addresses row 16ks + 8(l >> 5) + 4r + j / 4,
	 * columns wn0 + 32 (fragment) + 16((l >> 4) & 1) + 4(j % 4).., at
	 * their chunk's swizzled place */
	const int j16 = lane & 15;
	const int brow = 8 * (lane >> 5) + (j16 >> 2), bsw = dlt_bswz<BCH>(brow);
	unsigned btr[FN];
#pragma unroll
	for (int j = 0; j < FN; ++j) {
		const int n = wn0 + 32 * j + 16 * ((lane >> 4) & 1) + 4 * (j16 & 3);
		btr[j] = lds0 + A_BYTES + (unsigned)(brow * (BN * 2) + (((n >> 3) ^ bsw) << 4) + (n & 7) * 2);
	}

	s3k_f32x16 acc[FM][FN];
#pragma unroll
	for (int i = 0; i < FM; ++i)
#pragma unroll
		for (int j = 0; j < FN; ++j)
#pragma unroll
			for (int r = 0; r < 16; ++r)
				acc[i][j][r] = 0.0f;

	const int nk = p.K / BK;
	dma(0, 0);
	if (nk > 1)
		dma(1, 1);
	for (int kt = 0; kt < nk; ++kt) {
		const int stg = kt & 1;
		/* this stage's loads; the next stage's may stay in flight */
		if (kt + 1 < nk)
			wait_vm<LOADS>();
		else
			wait_vm<0>();
		wg_barrier();
#pragma unroll
		for (int ks = 0; ks < 4; ++ks) {
			uint4 af[FM], bf[FN];
#pragma unroll
			for (int i = 0; i < FM; ++i)
				af[i] = lds_rd16(abase[ks ^ (2 * (i & 1))], (unsigned)(stg * STAGE + i * 4096));
#pragma unroll
			for (int j = 0; j < FN; ++j) {
				const unsigned a0 = btr[j] + (unsigned)(stg * STAGE + ks * 16 * (BN * 2));
				const uint2 lo = dlt_read_tr(a0), hi = dlt_read_tr(a0 + 4 * (BN * 2));
				bf[j] = make_uint4(lo.x, lo.y, hi.x, hi.y);
			}
			__builtin_amdgcn_s_waitcnt(0xC07F); /* lgkmcnt(0) */
#pragma unroll
			for (int i = 0; i < FM; ++i)
#pragma unroll
				for (int j = 0; j < FN; ++j)
					mfma_chunk<FAM>(acc[i][j], bf[j], af[i]);
		}
		/* every wave is done with this stage before it is refilled */
		wg_barrier();
		if (kt + 2 < nk)
			dma(kt + 2, stg);
	}
	__syncthreads();
	write_tile_ck<FM, FN, WTN, CK, true>(p, acc, smem, wave, lane, tm * BM + wm0, tn * BN + wn0, bz);
}

/* gemm_dlk's conditions: K = 64, M and N multiples of 192, plain f32 or
 * same-kind 16-bit output with 16-byte rows, no epilogue flags, enough
 * tiles to keep every CU busy. Its wait_vm<STORES> counts on every tile
 * taking write_tile_ck's fast path with whole tiles: exactly STORES
 * 16-byte stores per lane and no loads. The conditions here are the fast
 * path's (p.vec_ok: 16-byte aligned C, ldc and stride_c multiples of 8;
 * no bias, residual, row or column factors, row map or QKV stores; N a
 * multiple of the wave tile); a change to either must keep them equal. */
static bool dlk_ok(const struct s3k_gemm *g)
{
	return g->K == 64 && g->M % DLK_B == 0 && g->N % DLK_B == 0 &&
	       (g->flags & ~S3K_B_NT) == 0 && !g->rm_g && !g->res &&
	       (g->c_kind == S3K_F32 || g->c_kind == g->a_kind) && g->ldc % 8 == 0 &&
	       !((uintptr_t)g->c & 15u) && (g->batch <= 1 || g->stride_c % 8 == 0) &&
	       (long long)(g->M / DLK_B) * (g->N / DLK_B) * g->batch >= 1024 &&
	       (long long)(g->M / DLK_B) * (g->N / DLK_B) * g->batch < (1LL << 31);
}

template <int FAM, int WGN>
static int launch_dlk(const struct s3k_gemm *g, GemmArgs p, hipStream_t st)
{
	p.tiles_m = g->M / DLK_B;
	p.tiles_n = g->N / DLK_B;
	const int total = p.tiles_m * p.tiles_n * g->batch;
	static int cu_count[64];
	int dev = 0, cus = 256;
	if (hipGetDevice(&dev) == hipSuccess && dev >= 0 && dev < 64) {
		if (!cu_count[dev] &&
		    hipDeviceGetAttribute(&cu_count[dev], hipDeviceAttributeMultiprocessorCount, dev) !=
			    hipSuccess)
			cu_count[dev] = 0;
		if (cu_count[dev] > 0)
			cus = cu_count[dev];
	}
	const dim3 grid((unsigned)(total < cus ? total : cus));
	const dim3 block(128 * WGN);
	/* a slice's tiles on one XCD: Q K^T over 1296 slices of 576 x 576,
	 * 206-209 -> 188-190 us (one box, three interleaved runs) */
	p.xwalk = 1;
	if (g->c_kind == S3K_F32)
		hipLaunchKernelGGL((gemm_dlk<FAM, S3K_F32, WGN>), grid, block, 0, st, p, total);
	else if (FAM == FAM_BF16)
		hipLaunchKernelGGL((gemm_dlk<FAM, S3K_BF16, WGN>), grid, block, 0, st, p, total);
	else
		hipLaunchKernelGGL((gemm_dlk<FAM, S3K_F16, WGN>), grid, block, 0, st, p, total);
	return (int)hipGetLastError();
}

template <int BM, int BN, int WGM, int WGN, int FAM, int CK, bool INTER, bool QKV = false>
static void launch_dlp_k(const struct s3k_gemm *g, const GemmArgs &p, hipStream_t st)
{
	dim3 grid(p.tiles_m * p.tiles_n, g->batch);
	hipLaunchKernelGGL((gemm_dlp<BM, BN, WGM, WGN, FAM, CK, INTER, QKV>), grid,
			   dim3(64 * WGM * WGN), 0, st, p);
}

template <int BM, int BN, int WGM, int WGN, bool INTER, int FAM>
static int launch_dlp_fam(const struct s3k_gemm *g, const GemmArgs &p, hipStream_t st)
{
	constexpr int SAME = FAM == FAM_BF16 ? S3K_BF16 : S3K_F16;
	if (g->flags & S3K_EPI_QKV) {
		if constexpr (qkv_tiles(S3K_F32, BN / WGN)) {
			if (g->c_kind != S3K_F32)
				return (int)hipErrorInvalidValue;
			launch_dlp_k<BM, BN, WGM, WGN, FAM, S3K_F32, INTER, true>(g, p, st);
			return (int)hipGetLastError();
		}
		return (int)hipErrorInvalidValue;
	}
	switch (g->c_kind) {
	case S3K_F32:      launch_dlp_k<BM, BN, WGM, WGN, FAM, S3K_F32, INTER>(g, p, st); break;
	case SAME:         launch_dlp_k<BM, BN, WGM, WGN, FAM, SAME, INTER>(g, p, st); break;
	case S3K_C_F16OP:  launch_dlp_k<BM, BN, WGM, WGN, FAM, S3K_C_F16OP, INTER>(g, p, st); break;
	case S3K_C_PLANES: launch_dlp_k<BM, BN, WGM, WGN, FAM, S3K_C_PLANES, INTER>(g, p, st); break;
	default:           return (int)hipErrorInvalidValue;
	}
	return (int)hipGetLastError();
}

/* the pipelined kernel needs whole 64-k steps */
template <int BM, int BN, int WGM, int WGN, bool INTER>
static int launch_dlp_cfg(const struct s3k_gemm *g, GemmArgs p, hipStream_t st)
{
	if (g->K % 64)
		return (int)hipErrorInvalidValue;
	p.tiles_m = (p.M + BM - 1) / BM;
	p.tiles_n = (p.N + BN - 1) / BN;
	/* tiles in N strips of 8 columns, cut into the XCDs' runs: each XCD
	 * reads fewer distinct A and W panels (fc1: a floor of 57 MB of
	 * fetches against 68 for the grouped order). One box, three
	 * interleaved runs: fc2 821-835 -> 840-849 TFLOP/s, config 1
	 * 28.4-28.9 -> 27.9-28.1 us, f16 fc1 +0.8 %, fc1 +0.4 % (within
	 * noise); 6-column strips favoured fc1 (+0.9 %) but not config 1
	 * or the Q8 step */
	p.tstrip = 8;
	if (g->a_kind == S3K_BF16)
		return launch_dlp_fam<BM, BN, WGM, WGN, INTER, FAM_BF16>(g, p, st);
	return launch_dlp_fam<BM, BN, WGM, WGN, INTER, FAM_F16>(g, p, st);
}

template <int BM, int BN, int BK, int WGM, int WGN, int STAGES, int FAM, int CK, int OCC>
static void launch_dl_k(const struct s3k_gemm *g, const GemmArgs &p, hipStream_t st)
{
	dim3 grid(p.tiles_m * p.tiles_n, g->batch);
	hipLaunchKernelGGL((gemm_dl<BM, BN, BK, WGM, WGN, STAGES, FAM, CK, OCC>), grid,
			   dim3(64 * WGM * WGN), 0, st, p);
}

/* OPK: the configuration is also built for the operand output kinds
 * (S3K_C_F16OP, S3K_C_PLANES); the others reject them. */
template <int BM, int BN, int BK, int WGM, int WGN, int STAGES, int OCC, int FAM, bool OPK>
static int launch_dl_fam(const struct s3k_gemm *g, const GemmArgs &p, hipStream_t st)
{
	constexpr int SAME = FAM == FAM_BF16 ? S3K_BF16 : S3K_F16;
	switch (g->c_kind) {
	case S3K_F32:
		launch_dl_k<BM, BN, BK, WGM, WGN, STAGES, FAM, S3K_F32, OCC>(g, p, st);
		break;
	case SAME:
		launch_dl_k<BM, BN, BK, WGM, WGN, STAGES, FAM, SAME, OCC>(g, p, st);
		break;
	case S3K_C_F16OP:
	case S3K_C_PLANES:
		if constexpr (OPK) {
			if (g->c_kind == S3K_C_F16OP)
				launch_dl_k<BM, BN, BK, WGM, WGN, STAGES, FAM, S3K_C_F16OP, OCC>(g, p, st);
			else
				launch_dl_k<BM, BN, BK, WGM, WGN, STAGES, FAM, S3K_C_PLANES, OCC>(g, p, st);
			break;
		}
		return (int)hipErrorInvalidValue;
	default:
		return (int)hipErrorInvalidValue;
	}
	return (int)hipGetLastError();
}

template <int BM, int BN, int BK, int WGM, int WGN, int STAGES, int OCC, bool OPK = false>
static int launch_dl_cfg(const struct s3k_gemm *g, GemmArgs p, hipStream_t st)
{
	if (g->flags & S3K_EPI_QKV) /* the pipelined kernels only */
		return (int)hipErrorInvalidValue;
	p.tiles_m = (p.M + BM - 1) / BM;
	p.tiles_n = (p.N + BN - 1) / BN;
	if (g->a_kind == S3K_BF16)
		return launch_dl_fam<BM, BN, BK, WGM, WGN, STAGES, OCC, FAM_BF16, OPK>(g, p, st);
	return launch_dl_fam<BM, BN, BK, WGM, WGN, STAGES, OCC, FAM_F16, OPK>(g, p, st);
}

} /* namespace s3k */

using namespace s3k;

/* bf16 x bf16 or f16 x f16, B as [N,K], 16-byte aligned rows, each batch
 * slice within a 2 GiB buffer range. */
/* gemm_dlt's conditions: B [K, N] 16-bit like A, K a multiple of 64, N
 * of 64 (at most 128) or of 256, 16-byte rows, enough tiles. */
static bool dlt_narrow(const struct s3k_gemm *g)
{
	return g->N % 64 == 0 && g->N <= 128;
}

bool s3k_dlt_ok(const struct s3k_gemm *g)
{
	if ((g->flags & S3K_B_NT) || g->a_kind != g->b_kind ||
	    (g->a_kind != S3K_BF16 && g->a_kind != S3K_F16) || g->rm_g)
		return false;
	if (g->M <= 0 || (!dlt_narrow(g) && g->N % 256) || g->N <= 0 || g->K <= 0 || g->K % 64 ||
	    g->batch <= 0)
		return false;
	if (((uintptr_t)g->a | (uintptr_t)g->b) & 15u || (g->lda * 2LL) % 16 || (g->ldb * 2LL) % 16)
		return false;
	if (g->batch > 1 && ((g->stride_a * 2) % 16 || (g->stride_b * 2) % 16))
		return false;
	if ((long long)g->M * g->lda * 2 > 0x7FFFFFF0LL || (long long)g->K * g->ldb * 2 > 0x7FFFFFF0LL)
		return false;
	return (long long)((g->M + 191) / 192) * (g->N / (dlt_narrow(g) ? 64 : 256)) * g->batch >= 256;
}

int s3k_dlt_launch(const struct s3k_gemm *g, GemmArgs p, hipStream_t st)
{
	if (!s3k_dlt_ok(g))
		return (int)hipErrorInvalidValue;
	p.a_extent = (unsigned)((long long)g->M * g->lda * 2);
	p.b_extent = (unsigned)((long long)g->K * g->ldb * 2);
	const bool narrow = dlt_narrow(g);
	p.tiles_m = (g->M + 191) / 192;
	p.tiles_n = g->N / (narrow ? 64 : 256);
	dim3 grid(p.tiles_m * p.tiles_n, g->batch);
	/* 8 slices or more: the 1-D grid whose groups keep each slice's
	 * tiles on one XCD (attention P V over 1296 slices: 195-199 -> 188-191
	 * us, one box, three interleaved runs) */
	const long long nwg = (long long)p.tiles_m * p.tiles_n * g->batch;
	p.xwalk = 0;
	if (g->batch >= 8 && nwg < (1LL << 31)) {
		p.xwalk = g->batch;
		grid = dim3((unsigned)nwg, 1);
	}
	if (!(g->c_kind == S3K_F32 || g->c_kind == g->a_kind))
		return (int)hipErrorInvalidValue;
#define S3K_DLT(BN_, WGN_, OCC_, FAM_, CK_)                                                  \
	hipLaunchKernelGGL((gemm_dlt<192, BN_, 2, WGN_, OCC_, FAM_, CK_>), grid, dim3(128 * WGN_), \
			   0, st, p)
#define S3K_DLT_K(FAM_, CKS_)                                      \
	do {                                                       \
		if (narrow && g->c_kind == S3K_F32)                \
			S3K_DLT(64, 2, 2, FAM_, S3K_F32);          \
		else if (narrow)                                   \
			S3K_DLT(64, 2, 2, FAM_, CKS_);             \
		else if (g->c_kind == S3K_F32)                     \
			S3K_DLT(256, 4, 1, FAM_, S3K_F32);         \
		else                                               \
			S3K_DLT(256, 4, 1, FAM_, CKS_);            \
	} while (0)
	if (g->a_kind == S3K_BF16)
		S3K_DLT_K(FAM_BF16, S3K_BF16);
	else
		S3K_DLT_K(FAM_F16, S3K_F16);
#undef S3K_DLT_K
#undef S3K_DLT
	return (int)hipGetLastError();
}

bool s3k_dl_ok(const struct s3k_gemm *g)
{
	if (!(g->flags & S3K_B_NT) || g->a_kind != g->b_kind ||
	    (g->a_kind != S3K_BF16 && g->a_kind != S3K_F16))
		return false;
	if (g->M <= 0 || g->N <= 0 || g->K <= 0 || g->K % 8 || g->batch <= 0)
		return false;
	if (((uintptr_t)g->a | (uintptr_t)g->b) & 15u)
		return false;
	if ((g->lda * 2LL) % 16 || (g->ldb * 2LL) % 16)
		return false;
	if (g->batch > 1 && ((g->stride_a * 2) % 16 || (g->stride_b * 2) % 16))
		return false;
	if ((long long)g->M * g->lda * 2 > 0x7FFFFFF0LL || (long long)g->N * g->ldb * 2 > 0x7FFFFFF0LL)
		return false;
	return true;
}

extern "C" int s3k_dl_eligible(const struct s3k_gemm *g)
{
	return s3k_dl_ok(g) ? 1 : 0;
}

/* Tile shape, from measurements on the ViT-L shapes (bench data, one
 * process, interleaved repetitions). With K % 64 == 0 the pipelined
 * kernel (gemm_dlp) runs; it was 1-9 % faster than gemm_dl on every
 * shape:
 *   - 256x256 (cfg 20 / 9, 8 waves) when the problem is one nearly full
 *     round of 224..256 such tiles (qkv 5184x3072: 32.1 against 33.3 us;
 *     4096^3: 1266 against 1201 TFLOP/s), and (K % 64 == 0) from 160
 *     such tiles when 192x256 tiles would spill into a second round
 *     (4096x3072x1024: 29.2 against 37.1 us for 192x128);
 *   - 192x256 (cfg 23, 8 waves) from 384 such tiles (fc1: 45.5 against
 *     49.7 us for 192x128);
 *   - 192x128 (cfg 24 / 10, 8 waves) when that gives at least 192 tiles
 *     (fc2, proj, batched attention), and first of all for N <= 128 (P V
 *     as an NT product: 200 against 303 us for 192x256);
 *   - 128x128 (cfg 4, 4 waves) for mid-size problems, 64x64 (cfg 2) for
 *     small ones.
 *   - K = 64 with M, N multiples of 192 and at least 1024 such tiles
 *     (attention scores over many slices): the persistent gemm_dlk,
 *     six waves (cfg 30; cfg 31 the four-wave form, as fast within the
 *     run-to-run spread).
 * SAM3_HIP_DL_CFG forces a configuration (tuning and tests). */
static long long dl_tiles(const struct s3k_gemm *g, int bm, int bn)
{
	return (long long)((g->M + bm - 1) / bm) * ((g->N + bn - 1) / bn) * g->batch;
}

int s3k_dl_launch(const struct s3k_gemm *g, GemmArgs p, hipStream_t st)
{
	if (!s3k_dl_ok(g))
		return (int)hipErrorInvalidValue;
	p.a_extent = (unsigned)((long long)g->M * g->lda * 2);
	p.b_extent = (unsigned)((long long)g->N * g->ldb * 2);
	int cfg = s3h_settings()->dl_cfg;
	if (cfg < 0) {
		const long long t9 = dl_tiles(g, 256, 256), t10 = dl_tiles(g, 192, 128);
		const bool pipe = g->K % 64 == 0;
		if (pipe && g->N <= 128 && t10 >= 192)
			cfg = 24; /* narrow N: wider tiles would only compute padding */
		else if (t9 >= 224 && t9 <= 256)
			cfg = pipe ? 20 : 9;
		else if (pipe && t9 >= 160 && t9 <= 256 && dl_tiles(g, 192, 256) > 256)
			cfg = 20;
		else if (pipe && dl_tiles(g, 192, 256) >= 384)
			cfg = 23;
		else if (t10 >= 192)
			cfg = pipe ? 24 : 10;
		else if (dl_tiles(g, 128, 128) >= 64)
			cfg = 4;
		else
			cfg = 2;
	}
	/* the S3K_EPI_QKV epilogue exists for the pipelined kernel with wave
	 * tiles of 64 columns or 128: the small problems take its 128x128
	 * tile */
	if ((g->flags & S3K_EPI_QKV) && (cfg < 20 || cfg == 25))
		cfg = 26;
	if ((s3h_settings()->dl_cfg < 0 || cfg == 30) && dlk_ok(g))
		return g->a_kind == S3K_BF16 ? launch_dlk<FAM_BF16, 3>(g, p, st)
					     : launch_dlk<FAM_F16, 3>(g, p, st);
	if (cfg == 31 && dlk_ok(g))
		return g->a_kind == S3K_BF16 ? launch_dlk<FAM_BF16, 2>(g, p, st)
					     : launch_dlk<FAM_F16, 2>(g, p, st);
	if (cfg == 30 || cfg == 31)
		cfg = 2;
	switch (cfg) {
	case 0:  return launch_dl_cfg<256, 128, 32, 2, 2, 3, 2>(g, p, st);
	case 1:  return launch_dl_cfg<128, 128, 32, 2, 2, 3, 2>(g, p, st);
	case 2:  return launch_dl_cfg<64, 64, 32, 2, 2, 3, 2, true>(g, p, st);
	case 3:  return launch_dl_cfg<128, 256, 32, 2, 2, 3, 2>(g, p, st);
	case 4:  return launch_dl_cfg<128, 128, 64, 2, 2, 2, 2, true>(g, p, st);
	case 6:  return launch_dl_cfg<192, 256, 32, 2, 2, 4, 1>(g, p, st);
	case 7:  return launch_dl_cfg<192, 256, 64, 2, 4, 2, 1>(g, p, st);
	case 8:  return launch_dl_cfg<256, 256, 32, 2, 4, 3, 1>(g, p, st);
	case 9:  return launch_dl_cfg<256, 256, 64, 2, 4, 2, 1, true>(g, p, st);
	case 10: return launch_dl_cfg<192, 128, 64, 2, 4, 2, 1, true>(g, p, st);
	case 11: return launch_dl_cfg<256, 128, 64, 2, 4, 2, 1>(g, p, st);
	case 12: return launch_dl_cfg<128, 256, 64, 2, 4, 2, 1>(g, p, st);
	case 13: return launch_dl_cfg<256, 256, 32, 2, 4, 4, 1>(g, p, st);
	case 20: return launch_dlp_cfg<256, 256, 2, 4, false>(g, p, st);
	case 21: return launch_dlp_cfg<256, 256, 2, 4, true>(g, p, st);
	case 22: return launch_dlp_cfg<192, 256, 2, 4, true>(g, p, st);
	case 23: return launch_dlp_cfg<192, 256, 2, 4, false>(g, p, st);
	case 24: return launch_dlp_cfg<192, 128, 2, 4, true>(g, p, st);
	case 25: return launch_dlp_cfg<256, 192, 4, 2, true>(g, p, st);
	case 26: return launch_dlp_cfg<128, 128, 2, 2, true>(g, p, st);
	default: return (int)hipErrorInvalidValue;
	}
}
