/*
 * gemm.hip - LDS-tiled MFMA GEMM for gfx950 (MI355X), and the generic
 * one-thread-per-output GEMM used for shapes the tiled kernel cannot take.
 *
 * Replaces the reference CPU matmul kernels of sam3.c:
 *   f32   src/backend/cpu/kernels/cpu_matmul.c:40-63,178-257
 *   f16   src/backend/cpu/kernels/cpu_matmul_f16.c:73-101,167-244
 *   bf16  src/backend/cpu/kernels/cpu_matmul_bf16.c:103-141,183-251
 *   Q8_0  src/backend/cpu/kernels/cpu_matmul_q8.c:39-134,168-235
 *
 * Tiled kernel structure (one workgroup = 4 waves of 64 lanes):
 *   - A tile [BM x BK] and B tile [BN x BK] are staged in LDS with k
 *     contiguous, as 16-byte chunks whose index is XOR-permuted per row
 *     (lds_swz) so that the 128-bit LDS reads of 8 or 16 consecutive rows
 *     hit distinct banks. Two stages: global loads of tile k+1 are issued before the
 *     MFMAs of tile k and written to the other stage after them.
 *   - Loaders convert on the way in: f32 activations -> f16, bf16 -> f16,
 *     Q8_0 weight blocks {f32 scale, 32 x int8} -> f16 (q*scale), and
 *     [K,N] B tiles are transposed in registers, so the MFMA loop only
 *     ever sees k-contiguous 16-bit (or f32) rows.
 *   - MFMA: v_mfma_f32_32x32x16_{bf16,f16} (f32 accumulate), or
 *     v_mfma_f32_32x32x2_f32 for f32 GEMM. Lane l supplies row (l & 31)
 *     and the 8-element k chunk (l >> 5) of each 16-k step; the same
 *     (lane, slot) -> k map is used for A and B, so the product is exact
 *     in the MFMA's own summation order.
 *   - Epilogue: bias and tanh-GELU fused, rounding to the output type at
 *     the same points as the reference's MATMUL -> ADD -> GELU nodes.
 *   - Workgroup -> tile map is XCD-aware: consecutive workgroup ids are
 *     dealt round-robin over the 8 XCDs, so ids are regrouped such that
 *     each XCD receives a contiguous block of tiles, walked in groups of
 *     8 tile-rows so neighbouring workgroups share A and B in its L2.
 */
#include "gemm_common.h"

namespace s3k {

template <int CPR>
__device__ __forceinline__ int lds_off(int row, int c)
{
	return (row * CPR + (c ^ lds_swz<CPR>(row))) << 4;
}

/* ------------------------------------------------------------------ */
/* Loaders. Each fills an LDS tile of R rows x CPR 16-byte k-chunks.    */
/* IS_B selects the B operand (rows are N) instead of A (rows are M).   */
/* ------------------------------------------------------------------ */

/* Rows whose 16-byte chunks are copied as they are (bf16, f16, f32). */
template <int R, int CPR, int NT, int ESZ, bool IS_B>
struct LoadRows {
	static constexpr int TOT = R * CPR;
	static constexpr int NCH = (TOT + NT - 1) / NT;
	uint4 v[NCH];
	const char *src;
	long long ld;
	int rows, kch, tid;

	__device__ void init(const GemmArgs &p, int bz, int row0, int t)
	{
		const char *base = IS_B ? p.b + bz * p.sb_b : p.a + bz * p.sa_b;
		ld = IS_B ? p.ldb_b : p.lda_b;
		src = base + (long long)row0 * ld;
		rows = (IS_B ? p.N : p.M) - row0;
		kch = p.K * ESZ / 16;
		tid = t;
	}
	__device__ void load(int kc0)
	{
#pragma unroll
		for (int i = 0; i < NCH; ++i) {
			int q = tid + i * NT;
			if (TOT % NT != 0 && q >= TOT)
				continue;
			int row = q / CPR, c = q % CPR;
			int r = row < rows ? row : rows - 1;
			if (kc0 + c < kch)
				v[i] = *(const uint4 *)(src + r * ld + (long long)(kc0 + c) * 16);
			else
				v[i] = make_uint4(0, 0, 0, 0);
		}
	}
	__device__ void store(char *lds)
	{
#pragma unroll
		for (int i = 0; i < NCH; ++i) {
			int q = tid + i * NT;
			if (TOT % NT != 0 && q >= TOT)
				continue;
			*(uint4 *)(lds + lds_off<CPR>(q / CPR, q % CPR)) = v[i];
		}
	}
};

/* A rows in f32 (or bf16), stored to LDS as f16 chunks of 8. */
template <int R, int CPR, int NT, bool SRC_BF16>
struct LoadRowsToF16 {
	static constexpr int TOT = R * CPR;
	static constexpr int NCH = (TOT + NT - 1) / NT;
	static constexpr int SUB = SRC_BF16 ? 1 : 2; /* 16-B loads per chunk */
	uint4 v[NCH][SUB];
	const char *src;
	long long ld;
	int rows, kch, tid;

	__device__ void init(const GemmArgs &p, int bz, int row0, int t)
	{
		ld = p.lda_b;
		src = p.a + bz * p.sa_b + (long long)row0 * ld;
		rows = p.M - row0;
		kch = p.K / 8;
		tid = t;
	}
	__device__ void load(int kc0)
	{
#pragma unroll
		for (int i = 0; i < NCH; ++i) {
			int q = tid + i * NT;
			if (TOT % NT != 0 && q >= TOT)
				continue;
			int row = q / CPR, c = q % CPR;
			int r = row < rows ? row : rows - 1;
			const uint4 *g = (const uint4 *)(src + r * ld +
				(long long)(kc0 + c) * (16 * SUB));
#pragma unroll
			for (int s = 0; s < SUB; ++s)
				v[i][s] = (kc0 + c < kch) ? g[s] : make_uint4(0, 0, 0, 0);
		}
	}
	__device__ void store(char *lds)
	{
#pragma unroll
		for (int i = 0; i < NCH; ++i) {
			int q = tid + i * NT;
			if (TOT % NT != 0 && q >= TOT)
				continue;
			uint4 o;
			if (SRC_BF16) {
				const uint4 x = v[i][0];
				o.x = pack_f16x2(bf16_to_f32(x.x & 0xFFFF), bf16_to_f32(x.x >> 16));
				o.y = pack_f16x2(bf16_to_f32(x.y & 0xFFFF), bf16_to_f32(x.y >> 16));
				o.z = pack_f16x2(bf16_to_f32(x.z & 0xFFFF), bf16_to_f32(x.z >> 16));
				o.w = pack_f16x2(bf16_to_f32(x.w & 0xFFFF), bf16_to_f32(x.w >> 16));
			} else {
				const uint4 x = v[i][0], y = v[i][1];
				o.x = pack_f16x2(__uint_as_float(x.x), __uint_as_float(x.y));
				o.y = pack_f16x2(__uint_as_float(x.z), __uint_as_float(x.w));
				o.z = pack_f16x2(__uint_as_float(y.x), __uint_as_float(y.y));
				o.w = pack_f16x2(__uint_as_float(y.z), __uint_as_float(y.w));
			}
			*(uint4 *)(lds + lds_off<CPR>(q / CPR, q % CPR)) = o;
		}
	}
};

/* Component k (a compile-time constant after unrolling) of a uint4. */
__device__ __forceinline__ uint32_t dword_of(const uint4 &q, int k)
{
	return k == 0 ? q.x : k == 1 ? q.y : k == 2 ? q.z : q.w;
}

/* B stored [K,N] (n contiguous): each thread loads an E(k) x E(n) block
 * (E = elements per 16 bytes) and writes its transpose as E k-chunks. */
template <int R, int CPR, int NT, int ESZ>
struct LoadColsT {
	static constexpr int E = 16 / ESZ;
	static constexpr int NG = R / E;          /* n groups */
	static constexpr int TOT = CPR * NG;      /* micro-tiles */
	static constexpr int NMT = (TOT + NT - 1) / NT;
	uint4 v[NMT][E];
	const char *src;
	long long ld;
	int ncols, K, tid;

	__device__ void init(const GemmArgs &p, int bz, int col0, int t)
	{
		ld = p.ldb_b;
		src = p.b + bz * p.sb_b + (long long)col0 * ESZ;
		ncols = p.N - col0;
		K = p.K;
		tid = t;
	}
	__device__ void load(int kc0)
	{
#pragma unroll
		for (int i = 0; i < NMT; ++i) {
			int q = tid + i * NT;
			if (TOT % NT != 0 && q >= TOT)
				continue;
			int ng = q % NG, kg = q / NG;
			int k = (kc0 + kg) * E;
			bool nok = ng * E < ncols;
#pragma unroll
			for (int r = 0; r < E; ++r)
				v[i][r] = (nok && k + r < K)
					? *(const uint4 *)(src + (long long)(k + r) * ld + ng * 16)
					: make_uint4(0, 0, 0, 0);
		}
	}
	__device__ void store(char *lds)
	{
#pragma unroll
		for (int i = 0; i < NMT; ++i) {
			int q = tid + i * NT;
			if (TOT % NT != 0 && q >= TOT)
				continue;
			int ng = q % NG, kg = q / NG;
#pragma unroll
			for (int j = 0; j < E; ++j) {
				uint32_t d[4];
				if (ESZ == 2) {
#pragma unroll
					for (int e = 0; e < 4; ++e) {
						const uint32_t x = dword_of(v[i][2 * e], j >> 1);
						const uint32_t y = dword_of(v[i][2 * e + 1], j >> 1);
						d[e] = (j & 1) ? ((x >> 16) | (y & 0xFFFF0000u))
							       : ((x & 0xFFFFu) | (y << 16));
					}
				} else {
#pragma unroll
					for (int e = 0; e < 4; ++e)
						d[e] = dword_of(v[i][e], j);
				}
				*(uint4 *)(lds + lds_off<CPR>(ng * E + j, kg)) =
					make_uint4(d[0], d[1], d[2], d[3]);
			}
		}
	}
};

/* B = Q8_0 weights W[N,K], blocks along k (K % 32 == 0): each thread
 * loads whole 36-byte blocks and writes 32 dequantized f16 values. */
template <int R, int CPR, int NT>
struct LoadQ8NT {
	static constexpr int BPR = CPR / 4;        /* blocks per row per tile */
	static constexpr int TOT = R * BPR;
	static constexpr int NB = (TOT + NT - 1) / NT;
	uint32_t v[NB][9];
	float inv[NB];
	const char *src;
	const float *cs;
	long long rowbytes;
	int rows, kbt, tid;

	__device__ void init(const GemmArgs &p, int bz, int row0, int t)
	{
		rowbytes = (long long)(p.K / 32) * 36;
		src = p.b + bz * p.sb_b + (long long)row0 * rowbytes;
		rows = p.N - row0;
		kbt = p.K / 32;
		tid = t;
		/* weight row r's values go to f16 as q * scale / cs[r] */
		cs = (p.flags & S3K_EPI_COLSCALE) ? p.cs + bz * p.cs_sb + row0 : nullptr;
	}
	__device__ void load(int kc0)
	{
		const int kb0 = kc0 / 4;
#pragma unroll
		for (int i = 0; i < NB; ++i) {
			int q = tid + i * NT;
			if (TOT % NT != 0 && q >= TOT)
				continue;
			int row = q / BPR, j = q % BPR;
			int r = row < rows ? row : rows - 1;
			const uint32_t *g = (const uint32_t *)(src + r * rowbytes +
							      (long long)(kb0 + j) * 36);
			bool ok = kb0 + j < kbt;
			inv[i] = cs ? inv_pow2(cs[r]) : 1.0f;
#pragma unroll
			for (int d = 0; d < 9; ++d)
				v[i][d] = ok ? g[d] : 0u;
		}
	}
	__device__ void store(char *lds)
	{
#pragma unroll
		for (int i = 0; i < NB; ++i) {
			int q = tid + i * NT;
			if (TOT % NT != 0 && q >= TOT)
				continue;
			int row = q / BPR, j = q % BPR;
			float s = __uint_as_float(v[i][0]) * inv[i];
#pragma unroll
			for (int cc = 0; cc < 4; ++cc) {
				uint2 lo = dequant4_f16(v[i][1 + 2 * cc], s);
				uint2 hi = dequant4_f16(v[i][2 + 2 * cc], s);
				*(uint4 *)(lds + lds_off<CPR>(row, j * 4 + cc)) =
					make_uint4(lo.x, lo.y, hi.x, hi.y);
			}
		}
	}
};

template <int BM, int BN, int BK, int WGM, int WGN, int FAM, int CK, class LA, class LB>
__global__ void __launch_bounds__(256, 1) gemm_tiled(GemmArgs p)
{
	constexpr int NT = 256;
	static_assert(WGM * WGN == 4, "4 waves");
	constexpr int ESZ = FAM == FAM_F32 ? 4 : 2;
	constexpr int CPR = BK * ESZ / 16;
	constexpr int WTM = BM / WGM, WTN = BN / WGN;
	constexpr int FM = WTM / 32, FN = WTN / 32;
	constexpr int A_BYTES = BM * BK * ESZ, B_BYTES = BN * BK * ESZ;
	constexpr int STAGE = A_BYTES + B_BYTES;
	__shared__ __attribute__((aligned(16))) char smem[2 * STAGE];

	const int tid = threadIdx.x;
	const int lane = tid & 63, wave = tid >> 6;
	const int wm0 = (wave / WGN) * WTM, wn0 = (wave % WGN) * WTN;
	const int bz = blockIdx.y;
	int tm, tn;
	tile_of(blockIdx.x, p.tiles_m, p.tiles_n, tm, tn);

	LA la;
	LB lb;
	la.init(p, bz, tm * BM, tid);
	lb.init(p, bz, tn * BN, tid);

	s3k_f32x16 acc[FM][FN];
#pragma unroll
	for (int i = 0; i < FM; ++i)
#pragma unroll
		for (int j = 0; j < FN; ++j)
#pragma unroll
			for (int r = 0; r < 16; ++r)
				acc[i][j][r] = 0.0f;

	const int nk = (p.K + BK - 1) / BK;
	la.load(0);
	lb.load(0);
	la.store(smem);
	lb.store(smem + A_BYTES);
	__syncthreads();

	for (int kt = 0; kt < nk; ++kt) {
		char *As = smem + (kt & 1) * STAGE;
		char *Bs = As + A_BYTES;
		const bool more = kt + 1 < nk;
		if (more) {
			la.load((kt + 1) * CPR);
			lb.load((kt + 1) * CPR);
		}
#pragma unroll
		for (int ks = 0; ks < CPR / 2; ++ks) {
			const int c = 2 * ks + (lane >> 5);
			uint4 af[FM], bfr[FN];
#pragma unroll
			for (int i = 0; i < FM; ++i)
				af[i] = *(const uint4 *)(As + lds_off<CPR>(wm0 + i * 32 + (lane & 31), c));
#pragma unroll
			for (int j = 0; j < FN; ++j)
				bfr[j] = *(const uint4 *)(Bs + lds_off<CPR>(wn0 + j * 32 + (lane & 31), c));
#pragma unroll
			for (int i = 0; i < FM; ++i)
#pragma unroll
				for (int j = 0; j < FN; ++j)
					mfma_chunk<FAM>(acc[i][j], af[i], bfr[j]);
		}
		if (more) {
			char *An = smem + ((kt + 1) & 1) * STAGE;
			la.store(An);
			lb.store(An + A_BYTES);
		}
		__syncthreads();
	}

	static_assert(4 * 32 * (WTN + 8) * 4 <= 2 * STAGE, "epilogue staging fits");
	write_tile_ck<FM, FN, WTN, CK>(p, acc, smem, wave, lane, tm * BM + wm0, tn * BN + wn0, bz);
}

/* ------------------------------------------------------------------ */
/* Generic GEMM: one thread per output element, the reference's         */
/* per-element arithmetic (k ascending, no FMA contraction):            */
/*   dense: acc += a*b            (cpu_matmul.c:54-58,                   */
/*                                 cpu_matmul_bf16.c:118-130)            */
/*   Q8:    acc += (a*(float)q)*s (cpu_matmul_q8.c:124-131), the block   */
/*          found from the flat index of B (k*N+n, or n*K+k for [N,K]).  */
/* f16 accumulates in f32 (the reference's fp16 accumulator is not      */
/* reproduced; see the f16 parity target in the oracle).                */
/* ------------------------------------------------------------------ */
template <int AK, int BK_>
__global__ void __launch_bounds__(256) gemm_generic(GemmArgs p, int a_ld, int b_ld)
{
	const long long per = (long long)p.M * p.N;
	const long long idx = (long long)blockIdx.x * 256 + threadIdx.x;
	const int bz = blockIdx.y;
	if (idx >= per)
		return;
	const int m = (int)(idx / p.N), n = (int)(idx % p.N);
	const bool nt = p.flags & S3K_B_NT;
	const char *A = p.a + bz * p.sa_b;
	const char *B = p.b + bz * p.sb_b;
	float acc = 0.0f;
	for (int k = 0; k < p.K; ++k) {
		const float a = load_as_f32(A, (long long)m * a_ld + k, AK);
		if (BK_ == S3K_Q8) {
			const long long lin = nt ? (long long)n * p.K + k : (long long)k * p.N + n;
			const char *blk = B + (lin >> 5) * 36;
			const float s = *(const float *)blk;
			const float q = (float)(int)(int8_t)blk[4 + (lin & 31)];
			acc = add_rn(acc, mul_rn(mul_rn(a, q), s));
		} else {
			const long long bi = nt ? (long long)n * b_ld + k : (long long)k * b_ld + n;
			acc = add_rn(acc, mul_rn(a, load_as_f32(B, bi, BK_)));
		}
	}
	if (p.flags & S3K_EPI_ROWSCALE)
		acc *= p.rs[(long long)bz * p.rs_sb + m];
	float bv = 0.0f;
	if (p.flags & S3K_EPI_BIAS)
		bv = load_as_f32(p.bias, n, p.bias_kind);
	float v;
	if (p.c_kind == S3K_BF16)
		v = epilogue<2>(acc, bv, p.flags);
	else if (p.c_kind == S3K_F16)
		v = epilogue<1>(acc, bv, p.flags);
	else
		v = epilogue<0>(acc, bv, p.flags);
	store_from_f32(p.c + (long long)bz * p.sc * (p.c_kind == 0 ? 4 : 2),
		       (long long)m * p.ldc + n, p.c_kind, v);
}

} /* namespace s3k */

using namespace s3k;

/* ------------------------------------------------------------------ */
/* Host-side selection                                                  */
/* ------------------------------------------------------------------ */
static int esize(int kind)
{
	return kind == S3K_F32 ? 4 : 2;
}

static bool aligned16(const void *p)
{
	return ((uintptr_t)p & 15u) == 0;
}

/* Tile configurations: 0 = 256x128, 1 = 128x128, 2 = 64x64. */
static int pick_cfg(const struct s3k_gemm *g, bool f32)
{
	const long long tiles0 = (long long)((g->M + 255) / 256) * ((g->N + 127) / 128) * g->batch;
	const long long tiles1 = (long long)((g->M + 127) / 128) * ((g->N + 127) / 128) * g->batch;
	if (!f32 && tiles0 >= 256)
		return 0;
	if (tiles1 >= 192 || f32)
		return tiles1 >= 128 ? 1 : 2;
	return 2;
}

static bool mfma_ok(const struct s3k_gemm *g)
{
	const int ak = g->a_kind, bk = g->b_kind;
	const bool nt = g->flags & S3K_B_NT;
	if (g->M <= 0 || g->N <= 0 || g->K <= 0 || g->batch <= 0)
		return false;
	if (!aligned16(g->a))
		return false;
	if (bk == S3K_Q8) {
		if (!nt || g->K % 32 || ((uintptr_t)g->b & 3u))
			return false;
		if (ak != S3K_F32 && ak != S3K_BF16 && ak != S3K_F16)
			return false;
		if ((long long)g->lda * esize(ak) % 16 || g->K % 8)
			return false;
		if (g->batch > 1 && ((g->stride_a * esize(ak)) % 16 || (g->stride_b % 36)))
			return false;
		return true;
	}
	if (ak != bk) {
		/* f32/bf16 activations against an unpacked f16 weight [N,K] */
		if (bk != S3K_F16 || !nt || (ak != S3K_F32 && ak != S3K_BF16))
			return false;
		if (!aligned16(g->b) || g->K % 8 || (long long)g->ldb * 2 % 16 ||
		    (long long)g->lda * esize(ak) % 16)
			return false;
		if (g->batch > 1 && ((g->stride_a * esize(ak)) % 16 || (g->stride_b * 2) % 16))
			return false;
		return true;
	}
	const int es = esize(ak), epc = 16 / es;
	if (!aligned16(g->b))
		return false;
	if (g->K % epc)
		return false;
	if ((long long)g->lda * es % 16 || (long long)g->ldb * es % 16)
		return false;
	if (!nt && g->N % epc)
		return false;
	if (g->batch > 1 && ((g->stride_a * es) % 16 || (g->stride_b * es) % 16))
		return false;
	return true;
}

extern "C" int s3k_gemm_path(const struct s3k_gemm *g)
{
	if (g->M <= 0 || g->N <= 0 || g->K < 0 || g->batch <= 0)
		return S3K_PATH_NONE;
	if (s3k_skinny_ok(g))
		return S3K_PATH_SKINNY;
	return mfma_ok(g) ? S3K_PATH_MFMA : S3K_PATH_GENERIC;
}

static GemmArgs make_args(const struct s3k_gemm *g)
{
	GemmArgs p;
	p.tstrip = 0;
	p.xwalk = 0;
	const int ea = esize(g->a_kind);
	p.a = (const char *)g->a;
	p.b = (const char *)g->b;
	p.c = (char *)g->c;
	p.bias = (const char *)g->bias;
	p.res = (const char *)g->res;
	p.ldr = g->N;
	p.rm_g = g->rm_g;
	p.rm_d1 = g->rm_d1;
	p.rm_d2 = g->rm_d2;
	p.rs = g->rs;
	p.rs_sb = g->rs_sb;
	p.cs = g->cs;
	p.cs_sb = g->cs_sb;
	p.ovf = g->ovf;
	p.ovf_tag = g->ovf_tag;
	p.rowf = g->rowf;
	p.M = g->M;
	p.N = g->N;
	p.K = g->K;
	p.lda_b = (long long)g->lda * ea;
	if (g->b_kind == S3K_Q8) {
		p.ldb_b = (long long)(g->K / 32) * 36;
		p.sb_b = g->stride_b; /* Q8 batch stride is given in bytes */
	} else {
		p.ldb_b = (long long)g->ldb * esize(g->b_kind);
		p.sb_b = g->stride_b * esize(g->b_kind);
	}
	p.ldc = g->ldc;
	p.sa_b = g->stride_a * ea;
	p.sc = g->stride_c;
	p.flags = g->flags;
	p.c_kind = g->c_kind;
	/* the operand output kinds compute in f32 and take an f32 bias */
	p.bias_kind = g->c_kind >= S3K_C_F16OP ? S3K_F32 : g->c_kind;
	p.vec_ok = aligned16(g->c) && g->ldc % 8 == 0 && (g->batch <= 1 || g->stride_c % 8 == 0);
	p.tiles_m = p.tiles_n = 0;
	p.a_extent = p.b_extent = 0;
	for (int y = 0; y < 3; ++y)
		p.qkv_out[y] = g->qkv_out[y];
	p.qkv_cos = g->qkv_cos;
	p.qkv_sin = g->qkv_sin;
	p.qkv_S = g->qkv_S;
	p.qkv_H = g->qkv_H;
	p.qkv_dsh = g->qkv_D > 0 ? __builtin_ctz((unsigned)g->qkv_D) : 0;
	p.qkv_rope = g->qkv_rope;
	return p;
}

/* What the S3K_EPI_QKV epilogue assumes (struct s3k_gemm) on `path`:
 * f32 output, one batch slice, no residual, row map or GELU, the operand
 * geometry below, and either the pipelined direct-to-LDS kernel (whole
 * 64-k steps, sequences of at least 32 rows) or the streaming skinny
 * kernel (no RoPE; its own checks in s3k_skinny_launch). */
static bool qkv_ok(const struct s3k_gemm *g, int path)
{
	const int D = g->qkv_D, H = g->qkv_H, S = g->qkv_S;
	const bool sk = path == S3K_PATH_SKINNY;
	if (g->c_kind != S3K_F32 || g->batch != 1 || (g->flags & (S3K_EPI_RES | S3K_EPI_GELU)) ||
	    g->rm_g || (!sk && g->K % 64) || D < 4 || (D & (D - 1)) || H <= 0 || S < (sk ? 1 : 32) ||
	    g->M % S || (sk && g->qkv_rope) || (long long)H * D > (1 << 28) ||
	    (long long)S * D > 0x7FFFFFFFLL)
		return false;
	const int E = H * D, n_out = g->N / E;
	if (g->N % E || n_out < 1 || n_out > 3 || g->qkv_rope < 0 || (g->qkv_rope >> n_out))
		return false;
	for (int y = 0; y < n_out; ++y)
		if (!g->qkv_out[y] || ((uintptr_t)g->qkv_out[y] & 15u))
			return false;
	if (g->qkv_rope && (!g->qkv_cos || !g->qkv_sin ||
			    (((uintptr_t)g->qkv_cos | (uintptr_t)g->qkv_sin) & 7u)))
		return false;
	if ((g->flags & S3K_EPI_BIAS) && (!g->bias || ((uintptr_t)g->bias & 15u)))
		return false;
	return sk ? s3k_skinny_ok(g) != 0 : s3k_dl_ok(g);
}

template <int BM, int BN, int BK, int WGM, int WGN, int FAM, int CK, class LA, class LB>
static int launch_tiled(GemmArgs p, int batch, hipStream_t st)
{
	p.tiles_m = (p.M + BM - 1) / BM;
	p.tiles_n = (p.N + BN - 1) / BN;
	dim3 grid(p.tiles_m * p.tiles_n, batch);
	hipLaunchKernelGGL((gemm_tiled<BM, BN, BK, WGM, WGN, FAM, CK, LA, LB>), grid, dim3(256), 0, st, p);
	return (int)hipGetLastError();
}

/* 16-bit operands of one kind: C is that kind or f32. */
template <int BM, int BN, int BK, int WGM, int WGN, int FAM, int KIND, class LA, class LB>
static int launch_tiled16(const struct s3k_gemm *g, GemmArgs p, hipStream_t st)
{
	if (g->c_kind == S3K_F32)
		return launch_tiled<BM, BN, BK, WGM, WGN, FAM, S3K_F32, LA, LB>(p, g->batch, st);
	return launch_tiled<BM, BN, BK, WGM, WGN, FAM, KIND, LA, LB>(p, g->batch, st);
}

/* One tile shape, all operand kinds. Q8 and mixed f32/bf16 x f16 write
 * f32 (the reference Q8 output, cpu_matmul_q8.c:181-185). */
template <int BM, int BN, int WGM, int WGN>
static int launch_cfg(const struct s3k_gemm *g, GemmArgs p, hipStream_t st)
{
	const bool nt = g->flags & S3K_B_NT;
	const int ak = g->a_kind, bk = g->b_kind;
	constexpr int BK16 = 64, C16 = BK16 * 2 / 16;
	if (bk == S3K_Q8 || (bk == S3K_F16 && ak != S3K_F16)) {
		if (g->c_kind != S3K_F32)
			return (int)hipErrorInvalidValue;
		if (bk == S3K_Q8) {
			typedef LoadQ8NT<BN, C16, 256> LB;
			if (ak == S3K_F32)
				return launch_tiled<BM, BN, BK16, WGM, WGN, FAM_F16, S3K_F32,
					LoadRowsToF16<BM, C16, 256, false>, LB>(p, g->batch, st);
			if (ak == S3K_BF16)
				return launch_tiled<BM, BN, BK16, WGM, WGN, FAM_F16, S3K_F32,
					LoadRowsToF16<BM, C16, 256, true>, LB>(p, g->batch, st);
			return launch_tiled<BM, BN, BK16, WGM, WGN, FAM_F16, S3K_F32,
				LoadRows<BM, C16, 256, 2, false>, LB>(p, g->batch, st);
		}
		typedef LoadRows<BN, C16, 256, 2, true> LB;
		if (ak == S3K_F32)
			return launch_tiled<BM, BN, BK16, WGM, WGN, FAM_F16, S3K_F32,
				LoadRowsToF16<BM, C16, 256, false>, LB>(p, g->batch, st);
		return launch_tiled<BM, BN, BK16, WGM, WGN, FAM_F16, S3K_F32,
			LoadRowsToF16<BM, C16, 256, true>, LB>(p, g->batch, st);
	}
	typedef LoadRows<BM, C16, 256, 2, false> LA;
	if (ak == S3K_BF16) {
		if (nt)
			return launch_tiled16<BM, BN, BK16, WGM, WGN, FAM_BF16, S3K_BF16, LA,
				LoadRows<BN, C16, 256, 2, true>>(g, p, st);
		return launch_tiled16<BM, BN, BK16, WGM, WGN, FAM_BF16, S3K_BF16, LA,
			LoadColsT<BN, C16, 256, 2>>(g, p, st);
	}
	if (ak == S3K_F16) {
		if (nt)
			return launch_tiled16<BM, BN, BK16, WGM, WGN, FAM_F16, S3K_F16, LA,
				LoadRows<BN, C16, 256, 2, true>>(g, p, st);
		return launch_tiled16<BM, BN, BK16, WGM, WGN, FAM_F16, S3K_F16, LA,
			LoadColsT<BN, C16, 256, 2>>(g, p, st);
	}
	return (int)hipErrorInvalidValue;
}

template <int BM, int BN, int WGM, int WGN>
static int launch_cfg_f32(const struct s3k_gemm *g, GemmArgs p, hipStream_t st)
{
	const bool nt = g->flags & S3K_B_NT;
	constexpr int BK = 32, C = BK * 4 / 16;
	if (nt)
		return launch_tiled<BM, BN, BK, WGM, WGN, FAM_F32, S3K_F32,
			LoadRows<BM, C, 256, 4, false>, LoadRows<BN, C, 256, 4, true>>(p, g->batch, st);
	return launch_tiled<BM, BN, BK, WGM, WGN, FAM_F32, S3K_F32,
		LoadRows<BM, C, 256, 4, false>, LoadColsT<BN, C, 256, 4>>(p, g->batch, st);
}

static int launch_generic(const struct s3k_gemm *g, GemmArgs p, hipStream_t st)
{
	const long long per = (long long)g->M * g->N;
	dim3 grid((unsigned)((per + 255) / 256), g->batch);
	const int ald = g->lda, bld = g->ldb;
#define S3K_GEN(AK, BKK) \
	hipLaunchKernelGGL((gemm_generic<AK, BKK>), grid, dim3(256), 0, st, p, ald, bld)
	switch (g->a_kind * 8 + g->b_kind) {
	case S3K_F32 * 8 + S3K_F32:   S3K_GEN(S3K_F32, S3K_F32); break;
	case S3K_F16 * 8 + S3K_F16:   S3K_GEN(S3K_F16, S3K_F16); break;
	case S3K_BF16 * 8 + S3K_BF16: S3K_GEN(S3K_BF16, S3K_BF16); break;
	case S3K_F32 * 8 + S3K_Q8:    S3K_GEN(S3K_F32, S3K_Q8); break;
	case S3K_BF16 * 8 + S3K_Q8:   S3K_GEN(S3K_BF16, S3K_Q8); break;
	case S3K_F16 * 8 + S3K_Q8:    S3K_GEN(S3K_F16, S3K_Q8); break;
	case S3K_F32 * 8 + S3K_F16:   S3K_GEN(S3K_F32, S3K_F16); break;
	case S3K_BF16 * 8 + S3K_F16:  S3K_GEN(S3K_BF16, S3K_F16); break;
	default:
		return (int)hipErrorInvalidValue;
	}
#undef S3K_GEN
	return (int)hipGetLastError();
}

extern "C" int s3k_skinny_launch(const struct s3k_gemm *g, void *stream);

extern "C" int s3k_gemm_launch_path(const struct s3k_gemm *g, int path, void *stream)
{
	hipStream_t st = (hipStream_t)stream;
	GemmArgs p = make_args(g);
	/* the LDS epilogue adds a residual and maps rows; the skinny kernels
	 * add a residual (f32 output, batch 1) */
	if (((g->flags & S3K_EPI_RES) || g->rm_g) &&
	    ((path != S3K_PATH_MFMA && !(path == S3K_PATH_SKINNY && !g->rm_g)) ||
	     ((g->flags & S3K_EPI_RES) && !g->res) || g->batch != 1 ||
	     g->c_kind == S3K_BF16 || g->c_kind == S3K_F16 ||
	     (path == S3K_PATH_SKINNY && (g->c_kind != S3K_F32 || g->ldc != g->N)) ||
	     (g->rm_g && (g->rm_d1 <= 0 || g->rm_d2 <= 0 ||
			  g->M % ((long long)g->rm_g * g->rm_d1 * g->rm_d2)))))
		return (int)hipErrorInvalidValue;
	if ((g->flags & S3K_EPI_QKV) &&
	    ((path != S3K_PATH_MFMA && path != S3K_PATH_SKINNY) ||
	     (path == S3K_PATH_MFMA && !mfma_ok(g)) || !qkv_ok(g, path)))
		return (int)hipErrorInvalidValue;
	/* the weight-row factors: every MFMA GEMM rounding q*scale to f16
	 * applies them (S3K_EPI_COLSCALE), and only the MFMA epilogue takes
	 * them (the skinny and generic kernels keep q*scale in f32) */
	if ((g->flags & S3K_EPI_COLSCALE) ? (path != S3K_PATH_MFMA || !g->cs)
					  : (path == S3K_PATH_MFMA && g->b_kind == S3K_Q8 &&
					     !((g->flags & S3K_Q8_WAUTO) && s3k_dlq8_ok(g))))
		return (int)hipErrorInvalidValue;
	if ((g->flags & S3K_Q8_WAUTO) &&
	    ((g->flags & S3K_EPI_COLSCALE) || path != S3K_PATH_MFMA || !s3k_dlq8_ok(g)))
		return (int)hipErrorInvalidValue;
	/* a LayerNorm's input rows, or the v of one-key attention, as A:
	 * the skinny kernels only */
	if ((g->flags & (S3K_A_LN | S3K_A_ATT1)) && path != S3K_PATH_SKINNY)
		return (int)hipErrorInvalidValue;
	if (path == S3K_PATH_SKINNY) {
		if (!s3k_skinny_ok(g))
			return (int)hipErrorInvalidValue;
		return s3k_skinny_launch(g, stream);
	}
	if (path == S3K_PATH_GENERIC)
		return launch_generic(g, p, st);
	if (path != S3K_PATH_MFMA || !mfma_ok(g))
		return (int)hipErrorInvalidValue;
	if (s3k_dl_ok(g))
		return s3k_dl_launch(g, p, st);
	/* B stored [K, N]: the attention's P V (narrow N) and weights kept
	 * [K, N] (N a multiple of 256) */
	if (s3k_dlt_ok(g) && !(g->flags & S3K_EPI_QKV) && s3h_settings()->dl_cfg < 0 &&
	    (g->c_kind == S3K_F32 || g->c_kind == g->a_kind))
		return s3k_dlt_launch(g, p, st);
	if (g->c_kind >= S3K_C_F16OP) /* only the direct-to-LDS GEMM writes operand forms */
		return (int)hipErrorInvalidValue;
	if (s3k_dlq8_ok(g))
		return s3k_dlq8_launch(g, p, st);
	if (g->a_kind == S3K_F32 && g->b_kind == S3K_F32) {
		switch (pick_cfg(g, true)) {
		case 1:  return launch_cfg_f32<128, 128, 2, 2>(g, p, st);
		default: return launch_cfg_f32<64, 64, 2, 2>(g, p, st);
		}
	}
	int cfg = pick_cfg(g, false);
	/* the 256-row [K,N]-layout tile needs more than 256 VGPRs: use 128 */
	if (cfg == 0 && !(g->flags & S3K_B_NT) && g->b_kind != S3K_Q8)
		cfg = 1;
	switch (cfg) {
	case 0:  return launch_cfg<256, 128, 2, 2>(g, p, st);
	case 1:  return launch_cfg<128, 128, 2, 2>(g, p, st);
	default: return launch_cfg<64, 64, 2, 2>(g, p, st);
	}
}

extern "C" int s3k_gemm_launch(const struct s3k_gemm *g, void *stream)
{
	const int path = s3k_gemm_path(g);
	if (path == S3K_PATH_NONE)
		return (int)hipErrorInvalidValue;
	return s3k_gemm_launch_path(g, path, stream);
}
