/*
 * gemm_dlq8.hip - C[M,N] (f32) = A[M,K] (f16) * W^T with W[N,K] in sam3.c's
 * Q8_0 blocks along k ({f32 scale; int8 q[32]}, 36 bytes, the converter's
 * layout, cli_convert.c:374-422), for gfx950. Reference arithmetic:
 * cpu_matmul_q8.c:124-131 (a * q * scale, f32 accumulate); f32 and bf16
 * activations are converted to f16 once per call before this kernel.
 *
 * The weights are never expanded in memory:
 *   - each k-step (BK = 64, two blocks) moves the raw 72-byte segment of
 *     every weight row straight into LDS with buffer_load ... lds, as five
 *     16-byte pieces at segment bytes 0, 16, 32, 48 and 56 (the last one
 *     overlaps, so no piece leaves the row); an LDS row is 80 bytes and
 *     segment byte b sits at b, or b + 8 for b >= 64;
 *   - the A tile arrives the same way, XOR-swizzled per row (lds_swz);
 *   - when a wave reads its B fragment (8 consecutive k of one row) it
 *     turns the 8 int8 into exact f16 integers with one byte permute and
 *     one packed subtract per pair (bytes biased by 128 under the f16
 *     exponent of 1024, then 1152 subtracted) and multiplies them by the
 *     block scale divided by the weight row's factor (S3K_EPI_COLSCALE,
 *     a power of two that keeps the row's largest scale an f16 normal)
 *     and rounded to f16; the epilogue multiplies the factor back;
 *   - v_mfma_f32_32x32x16_f16, f32 accumulate; each wave covers 128 rows
 *     of A so one dequantized B fragment serves 4 MFMAs. The B fragment
 *     is the MFMA's first operand (the MFMA forms C^T; the epilogue stages
 *     the transposed layout).
 * The ring, the waits and the epilogue follow gemm_dl.hip.
 */
#include "gemm_common.h"
#include "lds_dma.h"

namespace s3k {

typedef __attribute__((ext_vector_type(2))) _Float16 q8h2_t;

__device__ __forceinline__ uint32_t q8_pair_f16(uint32_t wx, uint32_t sel, q8h2_t s2)
{
	q8h2_t h = __builtin_bit_cast(q8h2_t, __builtin_amdgcn_perm(0x64646464u, wx, sel));
	h = (h - (q8h2_t){(_Float16)1152.0f, (_Float16)1152.0f}) * s2;
	return __builtin_bit_cast(uint32_t, h);
}

/* S3K_Q8_WAUTO after a k-loop run with factor 1: each lane holds the
 * largest |scale| of its B rows (row wn0 + 32 j + (lane & 31)); a row's
 * factor is s3k_q8_wfactors' 2^wscale_exp_of(127 * that). When a row of
 * the workgroup's tile needs one (rare: rows of tiny or huge scales),
 * q8_wauto_again returns true (workgroup-uniform) with binv set and the
 * accumulators cleared, the caller runs its k-loop again, and
 * q8_wauto_scale multiplies the accumulators of each column by its
 * factor, as the S3K_EPI_COLSCALE epilogue does: the same bits. */
template <int FM, int FN>
__device__ __forceinline__ bool q8_wauto_again(s3k_f32x16 (&acc)[FM][FN], const float (&smax)[FN],
					       float (&binv)[FN], int (&e)[FN])
{
	int any = 0;
#pragma unroll
	for (int j = 0; j < FN; ++j) {
		e[j] = wscale_exp_of(smax[j] * 127.0f);
		any |= e[j] != 0;
	}
	if (!__syncthreads_or(any))
		return false;
#pragma unroll
	for (int j = 0; j < FN; ++j)
		binv[j] = e[j] ? inv_pow2(pow2f(e[j])) : 1.0f;
#pragma unroll
	for (int i = 0; i < FM; ++i)
#pragma unroll
		for (int j = 0; j < FN; ++j)
#pragma unroll
			for (int r = 0; r < 16; ++r)
				acc[i][j][r] = 0.0f;
	return true;
}

/* The factors reach the lanes holding each column through LDS (smem,
 * free after the k-loop). Transposed accumulators: lane l holds columns
 * 8t + 4(l >> 5) + q of each 32-column block. */
template <int FM, int FN>
__device__ __forceinline__ void q8_wauto_scale(s3k_f32x16 (&acc)[FM][FN], const int (&e)[FN],
					       char *smem, int lane, int wn0)
{
	__syncthreads();
	float *fac = (float *)smem;
	if (lane < 32)
#pragma unroll
		for (int j = 0; j < FN; ++j)
			fac[wn0 + j * 32 + lane] = pow2f(e[j]);
	__syncthreads();
#pragma unroll
	for (int j = 0; j < FN; ++j) {
		s3k_f32x16 f;
#pragma unroll
		for (int t = 0; t < 4; ++t) {
			const float4 f4 = *(const float4 *)(fac + wn0 + j * 32 + 8 * t + 4 * (lane >> 5));
			f[4 * t] = f4.x, f[4 * t + 1] = f4.y, f[4 * t + 2] = f4.z, f[4 * t + 3] = f4.w;
		}
#pragma unroll
		for (int i = 0; i < FM; ++i)
			acc[i][j] *= f;
	}
}

template <int BM, int BN, int WGM, int WGN, int STAGES, int OCC>
__global__ void __launch_bounds__(64 * WGM * WGN, OCC) gemm_dlq8(GemmArgs p)
{
	constexpr int NW = WGM * WGN;
	constexpr int BK = 64, CPR = 8;
	constexpr int A_BYTES = BM * BK * 2;
	constexpr int A_INS = BM * CPR / 64;
	constexpr int PW = 5;                             /* 16-B slots per W row */
	constexpr int B_SLOTS = BN * PW;
	constexpr int B_INS = (B_SLOTS + 63) / 64;
	constexpr int SB = A_BYTES + B_INS * 1024;
	constexpr int A_PER = (A_INS + NW - 1) / NW, B_PER = (B_INS + NW - 1) / NW;
	constexpr int NPW = A_PER + B_PER;                /* loads per wave per stage */
	constexpr int WTM = BM / WGM, WTN = BN / WGN;
	constexpr int FM = WTM / 32, FN = WTN / 32;
	constexpr int KS = BK / 16;
	static_assert(STAGES >= 2 && STAGES <= 4, "ring depth");
	static_assert(NPW * (STAGES - 1) < 64, "vmcnt range");
	static_assert(NW * 32 * (WTN + 8) * 4 <= STAGES * SB, "epilogue staging fits");
	__shared__ __attribute__((aligned(1024))) char smem[STAGES * SB + 1024];

	const int lane = threadIdx.x & 63;
	const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
	const int wm0 = (wave / WGN) * WTM, wn0 = (wave % WGN) * WTN;
	const int bz = blockIdx.y;
	const unsigned lds0 = lds_addr_of(smem);
	int tm, tn;
	tile_of(blockIdx.x, p.tiles_m, p.tiles_n, tm, tn);

	const s3k_i32x4 ra = buf_rsrc(p.a + bz * p.sa_b, p.a_extent);
	const s3k_i32x4 rb = buf_rsrc(p.b + bz * p.sb_b, p.b_extent);
	const unsigned rowbytes = (unsigned)(p.K / 32) * 36u;

	/* Source of each of this lane's loads for k-step 0. A wave issues A_PER
	 * A chunks (load t*NW + wave) and B_PER W pieces; the last round of
	 * either may run past the tile and then loads zeros into a spare KiB,
	 * so every wave issues NPW loads per stage. */
	unsigned a_off[A_PER], b_off[B_PER];
	bool a_real[A_PER], b_real[B_PER];
#pragma unroll
	for (int t = 0; t < A_PER; ++t) {
		const int j = t * NW + wave;
		const int s = j * 64 + lane;
		const int row = s / CPR, c = (s % CPR) ^ lds_swz<CPR>(row);
		const int g = tm * BM + row;
		a_real[t] = j < A_INS;
		a_off[t] = (j < A_INS && g < p.M) ? (unsigned)(g * p.lda_b + c * 16) : S3K_OOB;
	}
#pragma unroll
	for (int t = 0; t < B_PER; ++t) {
		const int j = t * NW + wave;
		const int s = j * 64 + lane;
		const int row = s / PW, q = s % PW;
		const int n = tn * BN + row;
		b_real[t] = j < B_INS;
		b_off[t] = (j < B_INS && s < B_SLOTS && n < p.N)
			? (unsigned)n * rowbytes + (unsigned)(q < 4 ? q * 16 : 56) : S3K_OOB;
	}
	const unsigned trash = lds0 + STAGES * SB;

	auto issue = [&](int kt) {
		const unsigned st = lds0 + (unsigned)((kt % STAGES) * SB);
#pragma unroll
		for (int t = 0; t < A_PER; ++t)
			dma16s(a_real[t] ? st + (t * NW + wave) * 1024 : trash, ra, a_off[t], 128u * kt);
#pragma unroll
		for (int t = 0; t < B_PER; ++t)
			dma16s(b_real[t] ? st + A_BYTES + (t * NW + wave) * 1024 : trash, rb, b_off[t],
			       72u * kt);
	};

	/* B fragments: lane (row n = lane & 31 of each 32-row tile, k half
	 * h = lane >> 5) reads, for k-step ks, 8 q bytes at segment byte
	 * b = 36*(ks>>1) + 4 + 16*(ks&1) + 8h (LDS b + 8 when b >= 64) and the
	 * scale of block ks>>1. */
	const int h = lane >> 5;
	int qo[KS];
#pragma unroll
	for (int ks = 0; ks < KS; ++ks) {
		const int b = 36 * (ks >> 1) + 4 + 16 * (ks & 1) + 8 * h;
		qo[ks] = b + (b >= 64 ? 8 : 0);
	}
	int brow[FN];
	/* weight row n's block scales are divided by its factor cs[n] (a
	 * power of two, so exactly) before their rounding to f16 */
	float binv[FN];
#pragma unroll
	for (int j = 0; j < FN; ++j) {
		brow[j] = (wn0 + j * 32 + (lane & 31)) * (PW * 16);
		const int n = tn * BN + wn0 + j * 32 + (lane & 31);
		binv[j] = (p.flags & S3K_EPI_COLSCALE) && n < p.N
				  ? inv_pow2(p.cs[(long long)bz * p.cs_sb + n]) : 1.0f;
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
	/* S3K_Q8_WAUTO: the largest |scale| of each of this lane's B rows */
	const bool wauto = (p.flags & S3K_Q8_WAUTO) != 0;
	float smax[FN];
#pragma unroll
	for (int j = 0; j < FN; ++j)
		smax[j] = 0.0f;

	int fe[FN];
	bool again = false;
	for (int pass = 0;; ++pass) {
#pragma unroll
	for (int s = 0; s < STAGES - 1; ++s)
		if (s < nk)
			issue(s);

	for (int kt = 0; kt < nk; ++kt) {
		/* own loads of step kt done: at most the younger stages pending */
		const int younger = min(nk - 1 - kt, STAGES - 2);
		if (younger >= 2)
			wait_vm<2 * NPW>();
		else if (younger == 1)
			wait_vm<NPW>();
		else
			wait_vm<0>();
		wg_barrier();
		if (kt + STAGES - 1 < nk)
			issue(kt + STAGES - 1);

		const char *As = smem + (kt % STAGES) * SB;
		const char *Bs = As + A_BYTES;
		/* dequantize this wave's B fragments of the whole k-step first */
		uint4 bfr[KS][FN];
#pragma unroll
		for (int j = 0; j < FN; ++j) {
			const char *row = Bs + brow[j];
			q8h2_t s2[2];
#pragma unroll
			for (int blk = 0; blk < 2; ++blk) {
				const float sv = *(const float *)(row + 36 * blk);
				smax[j] = fmaxf(smax[j], finite_abs(sv));
				const _Float16 sh = (_Float16)(sv * binv[j]);
				s2[blk] = (q8h2_t){sh, sh};
			}
#pragma unroll
			for (int ks = 0; ks < KS; ++ks) {
				const uint32_t w0 = *(const uint32_t *)(row + qo[ks]) ^ 0x80808080u;
				const uint32_t w1 = *(const uint32_t *)(row + qo[ks] + 4) ^ 0x80808080u;
				const q8h2_t sc = s2[ks >> 1];
				bfr[ks][j] = make_uint4(q8_pair_f16(w0, 0x04010400u, sc),
							q8_pair_f16(w0, 0x04030402u, sc),
							q8_pair_f16(w1, 0x04010400u, sc),
							q8_pair_f16(w1, 0x04030402u, sc));
			}
		}
		uint4 af[2][FM];
#pragma unroll
		for (int i = 0; i < FM; ++i) {
			const int r = wm0 + i * 32 + (lane & 31);
			af[0][i] = *(const uint4 *)(As + ((r * CPR + (h ^ lds_swz<CPR>(r))) << 4));
		}
#pragma unroll
		for (int ks = 0; ks < KS; ++ks) {
			const int cur = ks & 1;
			if (ks + 1 < KS) {
				const int c = 2 * (ks + 1) + h;
#pragma unroll
				for (int i = 0; i < FM; ++i) {
					const int r = wm0 + i * 32 + (lane & 31);
					af[cur ^ 1][i] = *(const uint4 *)(As + ((r * CPR + (c ^ lds_swz<CPR>(r))) << 4));
				}
			}
#pragma unroll
			for (int i = 0; i < FM; ++i)
#pragma unroll
				for (int j = 0; j < FN; ++j)
					mfma_chunk<FAM_F16>(acc[i][j], bfr[ks][j], af[cur][i]);
		}
	}
	if (!wauto || pass == 1 || !(again = q8_wauto_again<FM, FN>(acc, smax, binv, fe)))
		break;
	}
	if (again)
		q8_wauto_scale<FM, FN>(acc, fe, smem, lane, wn0);
	__syncthreads();
	write_tile_ck<FM, FN, WTN, S3K_F32, true>(p, acc, smem, wave, lane, tm * BM + wm0, tn * BN + wn0, bz);
}

/*
 * gemm_dlpq: the Q8 GEMM for many rows, on the k-step schedule of the
 * pipelined f16 kernel (gemm_dlp, gemm_dl.hip): two stages, one wait and
 * one barrier per k-step, and the fragments of sub-step ks + 1 read while
 * the MFMAs of sub-step ks run (the non-interleaved order, whose grouped
 * reads measured fastest there). The weight tile is gemm_dlq8's: the raw
 * 72-byte segment of each row, 80 bytes per LDS row, moved by five
 * direct-to-LDS pieces (padded to whole loads per wave; the spare ones
 * load zeros into a trash KiB). A wave's B fragment is dequantized when
 * it is read: q exactly in f16 by the byte permute, then multiplied by
 * the block scale over the row factor rounded to f16 (gemm_dlq8's
 * arithmetic, so the same bits as gemm_dlq8 per product; the sums run
 * in the same k order). The block scales of a stage are read when the
 * stage's first fragments are. 192x256 tiles of eight 96x64 wave tiles,
 * one workgroup per CU, f32 C.
 */
template <int BM, int BN, int WGM, int WGN, bool INTER>
__global__ void __launch_bounds__(64 * WGM * WGN, 1) gemm_dlpq(GemmArgs p)
{
	constexpr int NW = WGM * WGN, BK = 64, CPR = 8, PW = 5, KS = BK / 16;
	constexpr int A_BYTES = BM * BK * 2;
	constexpr int A_INS = BM * CPR / 64, B_INS = (BN * PW + 63) / 64;
	constexpr int A_PER = (A_INS + NW - 1) / NW, B_PER = (B_INS + NW - 1) / NW;
	constexpr int LOADS = A_PER + B_PER;
	constexpr int B_BYTES = B_INS * 1024, B_BASE = 2 * A_BYTES;
	constexpr int TRASH = B_BASE + 2 * B_BYTES, LDS_BYTES = TRASH + 1024;
	constexpr int WTM = BM / WGM, WTN = BN / WGN;
	constexpr int FM = WTM / 32, FN = WTN / 32, NMF = FM * FN;
	static_assert(A_BYTES + (FM - 1) * 4096 < 65536, "fragment offsets fit the immediate");
	static_assert(NW * 32 * (WTN + 8) * 4 <= LDS_BYTES, "epilogue staging fits");
	static_assert(2 * LOADS < 64, "vmcnt range");
	__shared__ __attribute__((aligned(1024))) char smem[LDS_BYTES];

	const int lane = threadIdx.x & 63;
	const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
	const int wm0 = (wave / WGN) * WTM, wn0 = (wave % WGN) * WTN;
	const int bz = blockIdx.y;
	const unsigned lds0 = lds_addr_of(smem);
	int tm, tn;
	tile_of(blockIdx.x, p.tiles_m, p.tiles_n, tm, tn);
	const s3k_i32x4 ra = buf_rsrc(p.a + bz * p.sa_b, p.a_extent);
	const s3k_i32x4 rb = buf_rsrc(p.b + bz * p.sb_b, p.b_extent);
	const unsigned rowbytes = (unsigned)(p.K / 32) * 36u;

	/* per-lane source of DMA instruction t: A chunks (t < A_PER), then W
	 * pieces; loads past the tile go to the trash KiB */
	unsigned off[LOADS], dst[LOADS];
#pragma unroll
	for (int t = 0; t < LOADS; ++t) {
		const bool isa = t < A_PER;
		const int j = (isa ? t : t - A_PER) * NW + wave;
		const int s = j * 64 + lane;
		unsigned o = S3K_OOB;
		if (isa) {
			const int row = s / CPR, c = (s % CPR) ^ lds_swz<CPR>(row);
			const int g = tm * BM + row;
			if (j < A_INS && g < p.M)
				o = (unsigned)(g * p.lda_b + c * 16);
			dst[t] = j < A_INS ? (unsigned)(j * 1024) : (unsigned)TRASH;
		} else {
			const int row = s / PW, q = s % PW;
			const int n = tn * BN + row;
			if (j < B_INS && s < BN * PW && n < p.N)
				o = (unsigned)n * rowbytes + (unsigned)(q < 4 ? q * 16 : 56);
			dst[t] = j < B_INS ? (unsigned)(B_BASE + j * 1024) : (unsigned)TRASH;
		}
		off[t] = o;
	}
	auto dma = [&](int kt, int t, int stg) {
		const bool isa = t < A_PER;
		const unsigned d = dst[t] == (unsigned)TRASH ? (unsigned)TRASH
				 : dst[t] + (unsigned)(stg * (isa ? A_BYTES : B_BYTES));
		dma16s(lds0 + d, isa ? ra : rb, off[t], isa ? (unsigned)(kt * BK * 2) : 72u * kt);
	};

	unsigned abase[4];
	{
		const int l32 = lane & 31, h = lane >> 5, r0 = wm0 + l32;
#pragma unroll
		for (int ks = 0; ks < 4; ++ks)
			abase[ks] = lds0 + (unsigned)((r0 * CPR + ((2 * ks + h) ^ lds_swz<CPR>(r0))) << 4);
	}
	/* B fragment of sub-step ks: row n = lane & 31 of each 32-row tile, 8
	 * q bytes at segment byte 36 (ks >> 1) + 4 + 16 (ks & 1) + 8 h (+8 past
	 * byte 64), the scale of block ks >> 1 at 36 (ks >> 1) */
	const int h = lane >> 5;
	int qo[KS];
#pragma unroll
	for (int ks = 0; ks < KS; ++ks) {
		const int b = 36 * (ks >> 1) + 4 + 16 * (ks & 1) + 8 * h;
		qo[ks] = b + (b >= 64 ? 8 : 0);
	}
	int brow[FN];
	float binv[FN];
#pragma unroll
	for (int j = 0; j < FN; ++j) {
		brow[j] = B_BASE + (wn0 + j * 32 + (lane & 31)) * (PW * 16);
		const int n = tn * BN + wn0 + j * 32 + (lane & 31);
		binv[j] = (p.flags & S3K_EPI_COLSCALE) && n < p.N
				  ? inv_pow2(p.cs[(long long)bz * p.cs_sb + n]) : 1.0f;
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
	q8h2_t s2[FN][2];
	/* S3K_Q8_WAUTO: the largest |scale| of each of this lane's B rows */
	const bool wauto = (p.flags & S3K_Q8_WAUTO) != 0;
	float smax[FN];
#pragma unroll
	for (int j = 0; j < FN; ++j)
		smax[j] = 0.0f;
	auto scales = [&](int stg) {
#pragma unroll
		for (int j = 0; j < FN; ++j) {
			const char *row = smem + stg * B_BYTES + brow[j];
#pragma unroll
			for (int blk = 0; blk < 2; ++blk) {
				const float sv = *(const float *)(row + 36 * blk);
				smax[j] = fmaxf(smax[j], finite_abs(sv));
				const _Float16 sh = (_Float16)(sv * binv[j]);
				s2[j][blk] = (q8h2_t){sh, sh};
			}
		}
	};
	auto frag = [&](int buf, int stg, int ks, int r) {
		if (r < FM) {
			af[buf][r] = lds_rd16(abase[ks ^ (2 * (r & 1))], (unsigned)(stg * A_BYTES + r * 4096));
		} else {
			const int j = r - FM;
			const char *row = smem + stg * B_BYTES + brow[j] + qo[ks];
			const uint32_t w0 = *(const uint32_t *)row ^ 0x80808080u;
			const uint32_t w1 = *(const uint32_t *)(row + 4) ^ 0x80808080u;
			const q8h2_t sc = s2[j][ks >> 1];
			bf[buf][j] = make_uint4(q8_pair_f16(w0, 0x04010400u, sc),
						q8_pair_f16(w0, 0x04030402u, sc),
						q8_pair_f16(w1, 0x04010400u, sc),
						q8_pair_f16(w1, 0x04030402u, sc));
		}
	};

	/* k-step kt from stage stg; next: a k-step follows; dmak: issue the
	 * DMA of k-step kt + 2 into stg */
	auto step = [&](int stg, int kt, bool next, bool dmak) {
#pragma unroll
		for (int ks = 0; ks < KS; ++ks) {
			const int cur = ks & 1, nxt = cur ^ 1;
			if (ks == 3) {
				__builtin_amdgcn_s_waitcnt(0xC07F); /* lgkmcnt(0): own reads done */
				if (next) {
					wait_vm<0>();
					wg_barrier();
				}
			}
			__builtin_amdgcn_sched_barrier(0);
			if (ks == 3 && next)
				scales(stg ^ 1);
			/* INTER: one fragment read (B: read and dequantization) or
			 * DMA after each MFMA; else grouped after them */
#pragma unroll
			for (int m = 0; m < NMF; ++m) {
				mfma_chunk<FAM_F16>(acc[m / FN][m % FN], bf[cur][m % FN], af[cur][m / FN]);
				if (INTER) {
					if (ks < 3) {
						if (m < FM + FN)
							frag(nxt, stg, ks + 1, m);
					} else {
						if (next && m < FM + FN)
							frag(0, stg ^ 1, 0, m);
						if (dmak && m < LOADS)
							dma(kt + 2, m, stg);
					}
					__builtin_amdgcn_sched_barrier(0);
				}
			}
			const int r0 = INTER ? NMF : 0;
#pragma unroll
			for (int r = r0; r < FM + FN; ++r) {
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
	int fe[FN];
	bool again = false;
	for (int pass = 0;; ++pass) {
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
		scales(0);
#pragma unroll
		for (int r = 0; r < FM + FN; ++r)
			frag(0, 0, 0, r);
		int kt = 0;
		for (; kt + 2 < nk; ++kt)
			step(kt & 1, kt, true, true);
		if (kt + 1 < nk) {
			step(kt & 1, kt, true, false);
			++kt;
		}
		step(kt & 1, kt, false, false);
		/* the barrier in q8_wauto_again also keeps the next pass's
		 * loads behind every wave's last fragment reads */
		if (!wauto || pass == 1 || !(again = q8_wauto_again<FM, FN>(acc, smax, binv, fe)))
			break;
	}
	if (again)
		q8_wauto_scale<FM, FN>(acc, fe, smem, lane, wn0);
	__syncthreads();
	write_tile_ck<FM, FN, WTN, S3K_F32, true>(p, acc, smem, wave, lane, tm * BM + wm0,
						 tn * BN + wn0, bz);
}

template <int BM, int BN, int WGM, int WGN, bool INTER = false>
static int launch_dlpq_cfg(const struct s3k_gemm *g, GemmArgs p, hipStream_t st)
{
	p.tiles_m = (p.M + BM - 1) / BM;
	p.tiles_n = (p.N + BN - 1) / BN;
	dim3 grid(p.tiles_m * p.tiles_n, g->batch);
	hipLaunchKernelGGL((gemm_dlpq<BM, BN, WGM, WGN, INTER>), grid, dim3(64 * WGM * WGN), 0, st, p);
	return (int)hipGetLastError();
}

template <int BM, int BN, int WGM, int WGN, int STAGES, int OCC>
static int launch_dlq8_cfg(const struct s3k_gemm *g, GemmArgs p, hipStream_t st)
{
	p.tiles_m = (p.M + BM - 1) / BM;
	p.tiles_n = (p.N + BN - 1) / BN;
	dim3 grid(p.tiles_m * p.tiles_n, g->batch);
	hipLaunchKernelGGL((gemm_dlq8<BM, BN, WGM, WGN, STAGES, OCC>), grid, dim3(64 * WGM * WGN), 0,
			   st, p);
	return (int)hipGetLastError();
}

} /* namespace s3k */

using namespace s3k;

/* f16 A [M,K] (16-byte aligned rows) times Q8_0 W [N,K] with K % 64 == 0,
 * f32 C; each batch slice within a 2 GiB buffer range. */
bool s3k_dlq8_ok(const struct s3k_gemm *g)
{
	if (g->b_kind != S3K_Q8 || !(g->flags & S3K_B_NT) || g->a_kind != S3K_F16 ||
	    g->c_kind != S3K_F32)
		return false;
	if (g->M <= 0 || g->N <= 0 || g->K <= 0 || g->K % 64 || g->batch <= 0)
		return false;
	if (((uintptr_t)g->a & 15u) || (g->lda * 2LL) % 16 || ((uintptr_t)g->b & 3u))
		return false;
	if (g->batch > 1 && ((g->stride_a * 2) % 16 || g->stride_b % 4))
		return false;
	if ((long long)g->M * g->lda * 2 > 0x7FFFFFF0LL ||
	    (long long)g->N * (g->K / 32) * 36 > 0x7FFFFFF0LL)
		return false;
	return true;
}

/*
 * Tile choice. Above 96 rows the pipelined kernel with 128x256 tiles of
 * eight 128x32 wave tiles (cfg 15; each wave dequantizes its own weight
 * fragments, none twice; two workgroups fit a CU): fc1 5184x4096x1024
 * with bf16 A 74-75 us per step against 87 for gemm_dlq8's 128x128 tiles
 * (cfg 2), 75-76 for 192x256 in the same layout (13), 78-81 for 192x256
 * and 192x128 with 2x4 waves (10, 11), 85-88 for 256x256 (12, 14); the
 * interleaved schedule (16-18) gained nothing. Config 3 (32 ViT-L
 * layers, every weight read as blocks): 7.99 ms against 8.84. M <= 96
 * (batched streams of weight copies) takes one tile of 32, 64 or 96
 * rows, so no weight tile is read twice. SAM3_HIP_DLQ8_CFG forces another
 * configuration (tests and tuning).
 */
int s3k_dlq8_launch(const struct s3k_gemm *g, GemmArgs p, hipStream_t st)
{
	if (!s3k_dlq8_ok(g))
		return (int)hipErrorInvalidValue;
	p.a_extent = (unsigned)((long long)g->M * g->lda * 2);
	p.b_extent = (unsigned)((long long)g->N * (g->K / 32) * 36);
	int cfg = s3h_settings()->dlq8_cfg;
	if (cfg < 0)
		cfg = g->M <= 32 ? 7 : g->M <= 64 ? 8 : g->M <= 96 ? 9 : 15;
	switch (cfg) {
	case 0:  return launch_dlq8_cfg<256, 256, 2, 4, 3, 1>(g, p, st);
	case 1:  return launch_dlq8_cfg<256, 128, 2, 4, 3, 1>(g, p, st);
	case 2:  return launch_dlq8_cfg<128, 128, 1, 4, 3, 2>(g, p, st);
	case 3:  return launch_dlq8_cfg<128, 256, 1, 8, 3, 1>(g, p, st);
	case 5:  return launch_dlq8_cfg<256, 128, 1, 4, 3, 1>(g, p, st);
	case 6:  return launch_dlq8_cfg<256, 128, 1, 4, 2, 1>(g, p, st);
	case 7:  return launch_dlq8_cfg<32, 128, 1, 4, 3, 2>(g, p, st);
	case 8:  return launch_dlq8_cfg<64, 128, 1, 4, 3, 2>(g, p, st);
	case 9:  return launch_dlq8_cfg<96, 128, 1, 4, 3, 2>(g, p, st);
	case 10: return launch_dlpq_cfg<192, 256, 2, 4>(g, p, st);
	case 11: return launch_dlpq_cfg<192, 128, 2, 4>(g, p, st);
	case 12: return launch_dlpq_cfg<256, 256, 2, 4>(g, p, st);
	case 13: return launch_dlpq_cfg<192, 256, 1, 8>(g, p, st);
	case 14: return launch_dlpq_cfg<256, 256, 1, 8>(g, p, st);
	case 15: return launch_dlpq_cfg<128, 256, 1, 8>(g, p, st);
	case 16: return launch_dlpq_cfg<192, 256, 1, 8, true>(g, p, st);
	case 17: return launch_dlpq_cfg<128, 256, 1, 8, true>(g, p, st);
	case 18: return launch_dlpq_cfg<192, 256, 2, 4, true>(g, p, st);
	default: return (int)hipErrorInvalidValue;
	}
}

extern "C" int s3k_dlq8_eligible(const struct s3k_gemm *g)
{
	if (g->batch != 1 && g->a_kind != S3K_F16)
		return 0;
	if (g->a_kind != S3K_F16 && (g->lda != g->K || ((uintptr_t)g->a & 15u)))
		return 0;
	/* f32 activations too: one cast pass plus this kernel measured faster
	 * than the register-staged kernel converting in its loader on the
	 * ViT-L shapes (5184 x {3072, 1024, 4096} x {1024, 4096}: 67 / 37 /
	 * 90 / 95 us against 102 / 39 / 143 / 120 us). SAM3_HIP_Q8_F32CAST=0
	 * keeps f32 activations on the register-staged kernel. */
	const bool f32_cast = s3h_settings()->q8_f32cast != 0;
	if (g->a_kind != S3K_F16 && g->a_kind != S3K_BF16 && !(g->a_kind == S3K_F32 && f32_cast))
		return 0;
	struct s3k_gemm h = *g;
	h.a_kind = S3K_F16;
	return s3k_dlq8_ok(&h) ? 1 : 0;
}
