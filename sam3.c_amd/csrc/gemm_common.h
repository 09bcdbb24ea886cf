/*
 * gemm_common.h - pieces shared by the tiled GEMM kernels (gemm.hip,
 * gemm_dl.hip): launch arguments, the MFMA step, the XCD-aware tile map
 * and the LDS-staged epilogue (bias, tanh-GELU, rounding, 16-byte stores).
 */
#ifndef SAM3_GEMM_COMMON_H
#define SAM3_GEMM_COMMON_H

#include "s3k.h"
#include "s3k_dev.h"

namespace s3k {

struct GemmArgs {
	const char *a;
	const char *b;
	char       *c;
	const char *bias;
	const char *res;              /* S3K_EPI_RES: f32 rows of ldr values */
	int M, N, K;
	long long lda_b, ldb_b, ldc;  /* A/B row pitch in bytes, C in elements */
	long long sa_b, sb_b, sc;     /* batch strides: bytes, bytes, elements */
	long long ldr;                /* residual row pitch, elements */
	int rm_g, rm_d1, rm_d2;       /* output row map (s3k_gemm), rm_g 0 = none */
	const float *rs;              /* S3K_EPI_ROWSCALE factors, rows apart   */
	long long rs_sb;              /* ... per batch slice                    */
	const float *cs;              /* S3K_EPI_COLSCALE factors, columns apart */
	long long cs_sb;              /* ... per batch slice                    */
	unsigned *ovf;                /* S3K_C_F16OP range flag (or NULL)       */
	unsigned ovf_tag;
	unsigned *rowf;               /* S3K_C_F16OP per-row tags (s3k_gemm)    */
	int flags;
	int c_kind;
	int bias_kind;
	int vec_ok;   /* rows of C (and the base) allow 16-byte stores */
	int tiles_m, tiles_n;
	unsigned a_extent, b_extent; /* bytes of one batch slice (buffer range) */
	/* S3K_EPI_QKV (struct s3k_gemm): head size 1 << qkv_dsh */
	float *qkv_out[3];
	const float *qkv_cos, *qkv_sin;
	int qkv_S, qkv_H, qkv_dsh, qkv_rope;
	int tstrip;   /* tile order (tile_of): 0, or N strips of this many tiles */
	int xwalk;    /* each slice's tiles on one XCD: gemm_dlk 1; gemm_dlt the
		       * slice count of its grouped 1-D grid; 0 off */
};

enum { FAM_BF16 = 0, FAM_F16 = 1, FAM_F32 = 2 };

/* LDS tiles hold rows of CPR 16-byte k-chunks; the chunk index of row r
 * is XORed with lds_swz(r). The MFMA operand reads have lane l fetch 16
 * bytes of row (l & 31) at one logical chunk per half-wave. The two
 * permutations below were chosen by measurement on gfx950
 * (SQ_LDS_BANK_CONFLICT of a ds_read_b128 probe with exactly this lane
 * pattern: zero conflict cycles, ~4 LDS cycles per instruction), against
 * 3.2 (row&7, and other XORs that look conflict-free in a simple
 * 64-bank model) to 22.4 extra cycles per read (no permutation):
 *   CPR 4 (64-B rows):  c ^ ((r >> 2) & 3)
 *   CPR 8 (128-B rows): c ^ ((r ^ (r >> 3)) & 7) */
/* 16 bytes from the LDS byte address base + off (a 32-bit LDS address,
 * so the offset can fold into the instruction's immediate) */
typedef unsigned lds_u4v __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) const lds_u4v lds_cu4;

__device__ __forceinline__ uint4 lds_rd16(unsigned base, unsigned off)
{
	const lds_u4v v = *(lds_cu4 *)(size_t)(base + off);
	return make_uint4(v.x, v.y, v.z, v.w);
}

template <int CPR>
__device__ __forceinline__ int lds_swz(int row)
{
	static_assert(CPR == 4 || CPR == 8, "LDS rows of 4 or 8 chunks");
	if constexpr (CPR == 8)
		return (row ^ (row >> 3)) & 7;
	else
		return (row >> 2) & 3;
}

/* One 16-k step (or 8-k for f32) of a 32x32 output tile. Lane l supplies
 * row (l & 31) and the 16-byte k-chunk (l >> 5); A and B use the same
 * (lane, slot) -> k map, so the MFMA computes the exact tile product. */
template <int FAM>
__device__ __forceinline__ void mfma_chunk(s3k_f32x16 &acc, const uint4 &a, const uint4 &b)
{
	if constexpr (FAM == FAM_BF16) {
		acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(
			__builtin_bit_cast(s3k_bf16x8, a), __builtin_bit_cast(s3k_bf16x8, b),
			acc, 0, 0, 0);
	} else if constexpr (FAM == FAM_F16) {
		acc = __builtin_amdgcn_mfma_f32_32x32x16_f16(
			__builtin_bit_cast(s3k_f16x8, a), __builtin_bit_cast(s3k_f16x8, b),
			acc, 0, 0, 0);
	} else {
		/* k slot (l >> 5) of MFMA s holds element s of the lane's chunk */
		acc = __builtin_amdgcn_mfma_f32_32x32x2f32(__uint_as_float(a.x), __uint_as_float(b.x), acc, 0, 0, 0);
		acc = __builtin_amdgcn_mfma_f32_32x32x2f32(__uint_as_float(a.y), __uint_as_float(b.y), acc, 0, 0, 0);
		acc = __builtin_amdgcn_mfma_f32_32x32x2f32(__uint_as_float(a.z), __uint_as_float(b.z), acc, 0, 0, 0);
		acc = __builtin_amdgcn_mfma_f32_32x32x2f32(__uint_as_float(a.w), __uint_as_float(b.w), acc, 0, 0, 0);
	}
}

/* Workgroup id -> (tile_m, tile_n). Workgroups are dealt round-robin to
 * the 8 XCDs; ids are regrouped so each XCD gets a contiguous range of
 * tiles, walked in groups of 8 tile-rows so that workgroups resident on
 * one XCD share A rows and B columns in that XCD's L2. */
__device__ __forceinline__ void tile_of(int wg, int tiles_m, int tiles_n, int &tm, int &tn,
					int strip = 0)
{
	const int nwg = tiles_m * tiles_n;
	int t = wg;
	if ((nwg & 7) == 0)
		t = (wg & 7) * (nwg >> 3) + (wg >> 3);
	if (strip > 0 && (nwg & 7) == 0) {
		/* N strips of `strip` tile columns, each walked row by row, cut
		 * into the XCDs' runs of nwg / 8 */
		const int full = tiles_n / strip, per = tiles_m * strip;
		const int s = t / per;
		if (s < full) {
			const int i = t - s * per;
			tm = i / strip;
			tn = s * strip + i % strip;
		} else {
			const int w = tiles_n - full * strip, i = t - full * per;
			tm = i / w;
			tn = full * strip + i % w;
		}
		return;
	}
	const int G = 8;
	const int per_group = G * tiles_n;
	const int g = t / per_group;
	const int first = g * G;
	const int gsz = min(tiles_m - first, G);
	const int in = t - g * per_group;
	tm = first + in % gsz;
	tn = in / gsz;
}

/* Orders this wave's LDS accesses before and after it (compiler fence at
 * wavefront scope; the hardware performs one wave's LDS operations in
 * order). */
__device__ __forceinline__ void wave_lds_fence()
{
	__builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
	__builtin_amdgcn_wave_barrier();
	__builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

/* Output row of logical row m under the row map (identity when rm_g is 0). */
__device__ __forceinline__ long long out_row(const GemmArgs &p, int m)
{
	if (!p.rm_g)
		return m;
	const int gi = m / p.rm_g, w = m - gi * p.rm_g;
	const int c = gi % p.rm_d2, t = gi / p.rm_d2;
	const int b = t % p.rm_d1, a = t / p.rm_d1;
	return ((long long)(a * p.rm_d2 + c) * p.rm_d1 + b) * p.rm_g + w;
}

/* Store of C[m][n..n+W-1] from W f32 values at v (LDS), output kind CK,
 * W = 4 for f32 C and 8 for 16-bit C (one 16-byte store either way).
 * EPI adds the bias and/or GELU (p.flags) with the reference's rounding
 * points; without it the values are only converted. */
/* The f16 operand output's range checks. f16 copies lose more than f16
 * rounding where |x| >= 2^15 (finite): f16_big, checked per value and
 * flagged at once. A row whose nonzero values all lie below 2^-10 would
 * round to a few bits too, but whether a row is such depends on all of
 * it, which spans several workgroups: each writer reports the largest
 * |x| of its part of a row (f16_row_tags). */
template <int W>
__device__ __forceinline__ bool f16_big(const float *x)
{
	bool big = false;
#pragma unroll
	for (int e = 0; e < W; ++e) {
		const float a = __builtin_fabsf(x[e]);
		big |= a >= 32768.0f && a <= 3.402823466e38f;
	}
	return big;
}

template <int W>
__device__ __forceinline__ float f16_part_max(const float *x)
{
	float mx = 0.0f;
#pragma unroll
	for (int e = 0; e < W; ++e)
		mx = fmaxf(mx, finite_abs(x[e]));
	return mx;
}

/* Row m's tags (p.rowf, two words per row, the eval's tag p.ovf_tag):
 * word 2m when a part of the row holds a value of |x| >= 2^-10, word
 * 2m + 1 when a part holds nonzero values only below it. A row tagged
 * in the second word and not in the first is tiny throughout
 * (s3k_rowflag_check). Plain stores of the same value, in any order. */
__device__ __forceinline__ void f16_row_tag(const GemmArgs &p, long long m, float mx)
{
	if (mx >= 0x1p-10f)
		p.rowf[2 * m] = p.ovf_tag;
	else if (mx > 0.0f)
		p.rowf[2 * m + 1] = p.ovf_tag;
}

/* The global inputs of one output chunk's epilogue (C[m][n..n+W-1]):
 * bias and residual, each when its flag is set. */
template <int W>
struct EpiIn {
	float b[W];
	float f;
	float r[W];
};

template <int W>
__device__ __forceinline__ void epi_bias(const GemmArgs &p, int n, float *bv)
{
	const bool full = n + W <= p.N;
#pragma unroll
	for (int e = 0; e < W; ++e)
		bv[e] = 0.f;
	/* n is a multiple of W here: 16-byte (f32) or 8/16-byte (16-bit)
	 * loads need only an aligned bias base */
	const bool vec = full && (((uintptr_t)p.bias & 15u) == 0);
	if (vec && p.bias_kind != S3K_F32) {
		uint32_t d[W / 2];
		if constexpr (W == 8) {
			const uint4 w = *(const uint4 *)((const uint16_t *)p.bias + n);
			d[0] = w.x; d[1] = w.y; d[2] = w.z; d[3] = w.w;
		} else {
			const uint2 w = *(const uint2 *)((const uint16_t *)p.bias + n);
			d[0] = w.x; d[1] = w.y;
		}
#pragma unroll
		for (int e = 0; e < W / 2; ++e) {
			bv[2 * e] = p.bias_kind == S3K_BF16 ? bf16_to_f32(d[e] & 0xFFFFu)
							     : f16_to_f32(d[e] & 0xFFFFu);
			bv[2 * e + 1] = p.bias_kind == S3K_BF16 ? bf16_to_f32(d[e] >> 16)
								 : f16_to_f32(d[e] >> 16);
		}
	} else if (vec) {
#pragma unroll
		for (int e = 0; e < W; e += 4) {
			const float4 b = *(const float4 *)((const float *)p.bias + n + e);
			bv[e] = b.x; bv[e + 1] = b.y; bv[e + 2] = b.z; bv[e + 3] = b.w;
		}
	} else {
#pragma unroll
		for (int e = 0; e < W; ++e)
			if (n + e < p.N)
				bv[e] = load_as_f32(p.bias, n + e, p.bias_kind);
	}
}

/* Loads of chunk (m, n); the bias only when fetch_bias (else the caller
 * filled it from registers it loaded once). */
template <int W>
__device__ __forceinline__ void epi_fetch(const GemmArgs &p, int m, int n, int bz, bool fetch_bias,
					  EpiIn<W> &e)
{
	if (fetch_bias && (p.flags & S3K_EPI_BIAS))
		epi_bias<W>(p, n, e.b);
	if (p.flags & S3K_EPI_RES) {
		/* the residual ADD node that follows, in f32 */
		const float *r = (const float *)p.res + out_row(p, m) * p.ldr + n;
		if (n + W <= p.N && (((uintptr_t)r & 15u) == 0)) {
#pragma unroll
			for (int q = 0; q < W; q += 4) {
				const float4 v = *(const float4 *)(r + q);
				e.r[q] = v.x; e.r[q + 1] = v.y; e.r[q + 2] = v.z; e.r[q + 3] = v.w;
			}
		} else {
#pragma unroll
			for (int q = 0; q < W; ++q)
				e.r[q] = n + q < p.N ? r[q] : 0.0f;
		}
	}
}

/* Returns the largest finite |value| stored (S3K_C_F16OP; 0 otherwise). */
template <int CK, bool EPI, int W>
__device__ __forceinline__ float finishw(const GemmArgs &p, int flags, char *cb, int m, int n,
					const float (&xv)[W], const EpiIn<W> &ein)
{
	typedef float f4v __attribute__((ext_vector_type(4)));
	typedef unsigned u4v __attribute__((ext_vector_type(4)));
	static_assert(W == 4 || W == 8, "4 or 8 outputs per store");
	const bool full = n + W <= p.N;
	float x[W];
#pragma unroll
	for (int e = 0; e < W; ++e)
		x[e] = xv[e];
	if (EPI) {
#pragma unroll
		for (int e = 0; e < W; ++e)
			x[e] = epilogue<CK>(x[e], ein.b[e], flags);
		if (flags & S3K_EPI_RES) {
#pragma unroll
			for (int e = 0; e < W; ++e)
				x[e] = add_rn(x[e], ein.r[e]);
		}
	}
	const long long o = out_row(p, m) * p.ldc + n;
	if constexpr (CK == S3K_C_PLANES) {
		/* the split of split3_bf16_k: hi = bf16(x), lo = bf16(x - hi) */
		uint32_t hi[4], lo[4];
#pragma unroll
		for (int e = 0; e < 4; ++e)
			split_bf16x2(x[2 * e], x[2 * e + 1], hi[e], lo[e]);
		uint16_t *c = (uint16_t *)cb + o;
		if (W == 8 && full && p.vec_ok) {
			*(u4v *)c = (u4v){hi[0], hi[1], hi[2], hi[3]};
			*(u4v *)(c + p.N) = (u4v){lo[0], lo[1], lo[2], lo[3]};
			*(u4v *)(c + 2LL * p.N) = (u4v){hi[0], hi[1], hi[2], hi[3]};
		} else {
#pragma unroll
			for (int e = 0; e < W; ++e) {
				if (n + e >= p.N)
					continue;
				const uint16_t h = (uint16_t)(e & 1 ? hi[e / 2] >> 16 : hi[e / 2] & 0xFFFFu);
				const uint16_t l = (uint16_t)(e & 1 ? lo[e / 2] >> 16 : lo[e / 2] & 0xFFFFu);
				c[e] = h;
				c[p.N + e] = l;
				c[2LL * p.N + e] = h;
			}
		}
	} else if (CK == S3K_F32) {
		float *c = (float *)cb + o;
		if (full && p.vec_ok) {
#pragma unroll
			for (int e = 0; e < W; e += 4)
				*(f4v *)(c + e) = (f4v){x[e], x[e + 1], x[e + 2], x[e + 3]};
		} else {
#pragma unroll
			for (int e = 0; e < W; ++e)
				if (n + e < p.N)
					c[e] = x[e];
		}
	} else {
		if (CK == S3K_C_F16OP && p.ovf && f16_big<W>(x))
			*p.ovf = p.ovf_tag;
		uint32_t h[W];
#pragma unroll
		for (int e = 0; e < W; e += 2) {
			/* S3K_C_F16OP: f16 store of the f32 result (pack_f16x2) */
			const uint32_t w = CK == S3K_BF16 ? pack_bf16x2(x[e], x[e + 1]) : pack_f16x2(x[e], x[e + 1]);
			h[e] = w & 0xFFFFu;
			h[e + 1] = w >> 16;
		}
		uint16_t *c = (uint16_t *)cb + o;
		if (W == 8 && full && p.vec_ok) {
			*(u4v *)c = (u4v){h[0] | (h[1] << 16), h[2] | (h[3] << 16), h[4 % W] | (h[5 % W] << 16),
					  h[6 % W] | (h[7 % W] << 16)};
		} else {
#pragma unroll
			for (int e = 0; e < W; ++e)
				if (n + e < p.N)
					c[e] = (uint16_t)h[e];
		}
	}
	return CK == S3K_C_F16OP ? f16_part_max<W>(x) : 0.0f;
}

template <bool B>
struct epi_b {
	static constexpr bool value = B;
};

/* Epilogue of a wave tile, one 32-row strip at a time: the MFMA layout is
 * turned into row-contiguous runs of columns through LDS, so each lane
 * finishes 4 (f32) or 8 (16-bit) outputs and writes them with one 16-byte
 * store. Two accumulator layouts:
 *   - TR false (C = A W^T, A as the MFMA's first operand): lane l holds
 *     column l & 31 of rows 8*(r>>2) + 4*(l>>5) + (r&3), staged with one
 *     4-byte LDS write per value;
 *   - TR true (the operands swapped, the MFMA forms C^T): lane l holds row
 *     l & 31 and columns 8*(r>>2) + 4*(l>>5) + (r&3), four consecutive
 *     columns per 16-byte LDS write (a quarter of the write instructions).
 *     The swap does not change any product or the order of the sums.
 * `smem` must be free (all waves past their last LDS read) and hold
 * NW*32*(WTN+8) floats. Each wave stages through its own region of smem,
 * and the LDS operations of one wave are performed in program order, so
 * the waves need no barrier between them here: a wavefront-scope fence
 * keeps the compiler from moving the staging reads above the writes.
 * Without a residual (or a per-row bias) a wave reads all of a strip's
 * staged values and then issues its stores, so the LDS latency is paid
 * once per strip; the residual loop is kept rolled (it loads inside the
 * loop, and unrolled it would not fit the instruction cache), and each of
 * its iterations reads the next iteration's staged values first.
 * QKV_OK (TR, f32 output): the S3K_EPI_QKV epilogue only, a kernel of
 * its own (the other paths' registers would not leave room for it). */
template <int FM, int FN, int WTN, int CK, bool TR = false, bool QKV_OK = false>
__device__ __forceinline__ void write_tile_ck(const GemmArgs &p, s3k_f32x16 (&acc)[FM][FN],
					      char *smem, int wave, int lane, int m0, int n0, int bz)
{
	/* floats per staged row, 16-byte aligned: rows 4 apart land 32 banks
	 * apart for the 4-byte writes, and 16 consecutive rows on distinct
	 * banks for the 16-byte ones */
	constexpr int PITCH = TR ? WTN + 4 : WTN + 8;
	float *stg = (float *)smem + wave * 32 * PITCH;
	char *cb = p.c + (long long)bz * p.sc * (CK == S3K_F32 ? 4 : 2);
	static_assert(CK != S3K_C_PLANES || WTN % 8 == 0, "planes are written 8 outputs at a time");
	/* one 16-byte store per lane and unit: 4 f32 or 8 16-bit outputs,
	 * so consecutive lanes write consecutive 16 bytes of a row */
	constexpr int W = CK == S3K_F32 ? 4 : 8;
	constexpr int UNITS = 32 * WTN / W; /* per strip, a multiple of 64 */
	static_assert(UNITS % 64 == 0, "whole store rounds per strip");
	/* when WTN / W divides 64, a lane keeps the same W columns for every
	 * row it finishes: their bias is loaded once per tile */
	constexpr bool FIXED = 64 % (WTN / W) == 0;
	/* Global loads inside the store loops would be expensive: vmcnt counts
	 * stores as well as loads, so the wait for a load issued after a store
	 * also waits for that store. So the row factors are applied to the
	 * accumulators and the bias is loaded before the first store; only the
	 * residual (S3K_EPI_RES) is loaded inside a store loop. */
	if (p.flags & S3K_EPI_ROWSCALE) {
		if constexpr (TR) {
			/* lane l holds row l & 31 of each 32-row strip */
#pragma unroll
			for (int i = 0; i < FM; ++i) {
				const int r = m0 + i * 32 + (lane & 31);
				const float f = r < p.M ? p.rs[(long long)bz * p.rs_sb + r] : 1.0f;
#pragma unroll
				for (int j = 0; j < FN; ++j)
#pragma unroll
					for (int q = 0; q < 16; ++q)
						acc[i][j][q] *= f;
			}
		} else {
			/* lane l holds rows 8t + 4(l >> 5) + q (q < 4) of each strip */
#pragma unroll
			for (int i = 0; i < FM; ++i)
#pragma unroll
				for (int t = 0; t < 4; ++t) {
					const int r0 = m0 + i * 32 + 8 * t + 4 * (lane >> 5);
					const float *rp = p.rs + (long long)bz * p.rs_sb + r0;
					float f[4];
#pragma unroll
					for (int q = 0; q < 4; ++q)
						f[q] = r0 + q < p.M ? rp[q] : 1.0f;
#pragma unroll
					for (int j = 0; j < FN; ++j)
#pragma unroll
						for (int q = 0; q < 4; ++q)
							acc[i][j][4 * t + q] *= f[q];
				}
		}
	}
	if (p.flags & S3K_EPI_COLSCALE) {
		/* the weight-row factors of a Q8_0 weight, per output column */
		const float *cp = p.cs + (long long)bz * p.cs_sb;
		if constexpr (TR) {
			/* lane l holds columns 8t + 4(l >> 5) + q (q < 4) of each
			 * 32-column block */
#pragma unroll
			for (int j = 0; j < FN; ++j)
#pragma unroll
				for (int t = 0; t < 4; ++t) {
					const int c0 = n0 + j * 32 + 8 * t + 4 * (lane >> 5);
					float f[4];
#pragma unroll
					for (int q = 0; q < 4; ++q)
						f[q] = c0 + q < p.N ? cp[c0 + q] : 1.0f;
#pragma unroll
					for (int i = 0; i < FM; ++i)
#pragma unroll
						for (int q = 0; q < 4; ++q)
							acc[i][j][4 * t + q] *= f[q];
				}
		} else {
			/* lane l holds column l & 31 of each 32-column block */
#pragma unroll
			for (int j = 0; j < FN; ++j) {
				const int c = n0 + j * 32 + (lane & 31);
				const float f = c < p.N ? cp[c] : 1.0f;
#pragma unroll
				for (int i = 0; i < FM; ++i)
#pragma unroll
					for (int q = 0; q < 16; ++q)
						acc[i][j][q] *= f;
			}
		}
	}
	const int flags = p.flags & ~(S3K_EPI_ROWSCALE | S3K_EPI_COLSCALE);
	const bool heavy = (flags & S3K_EPI_RES) || (!FIXED && (flags & S3K_EPI_BIAS));
	const bool light = !heavy && (flags & (S3K_EPI_BIAS | S3K_EPI_GELU));
	/* the common cases (plain rows, whole 16-byte vectors, no residual,
	 * a bias loaded once per tile): a store path whose flag tests are
	 * made once per tile instead of once per element. gemm_dlk's vmcnt
	 * arithmetic relies on this path issuing exactly FM * UNITS / 64
	 * stores per lane and no load for whole tiles (dlk_ok admits only
	 * problems that take it). */
	constexpr bool PLAIN_CK = CK == S3K_F32 || CK == S3K_BF16 || CK == S3K_F16;
	const bool fast = PLAIN_CK && !(flags & S3K_EPI_RES) && (FIXED || !(flags & S3K_EPI_BIAS)) &&
			  !p.rm_g && p.vec_ok && n0 + WTN <= p.N;
	EpiIn<W> ein;
#pragma unroll
	for (int q = 0; q < W; ++q) {
		ein.b[q] = 0.f;
		ein.r[q] = 0.f;
	}
	ein.f = 1.0f;
	if (FIXED && (flags & S3K_EPI_BIAS)) {
		const int cw = (lane % (WTN / W)) * W;
		if (n0 + cw < p.N)
			epi_bias<W>(p, n0 + cw, ein.b);
	}
	/* staged values of unit s: row s / (WTN / W), columns cw.. cw + W - 1 */
	auto staged = [&](int s, float (&x)[W]) {
		const float *v = stg + (s / (WTN / W)) * PITCH + (s % (WTN / W)) * W;
#pragma unroll
		for (int e = 0; e < W; e += 4) {
			const float4 q = *(const float4 *)(v + e);
			x[e] = q.x; x[e + 1] = q.y; x[e + 2] = q.z; x[e + 3] = q.w;
		}
	};
	/* stage strip i's accumulators (the wave's own LDS region) */
	auto stage = [&](const s3k_f32x16 (&a)[FN]) {
		if constexpr (TR) {
			const int h = lane >> 5, l32 = lane & 31;
#pragma unroll
			for (int j = 0; j < FN; ++j)
#pragma unroll
				for (int t = 0; t < 4; ++t)
					*(float4 *)(stg + l32 * PITCH + 32 * j + 8 * t + 4 * h) =
						make_float4(a[j][4 * t], a[j][4 * t + 1], a[j][4 * t + 2], a[j][4 * t + 3]);
		} else {
#pragma unroll
			for (int j = 0; j < FN; ++j)
#pragma unroll
				for (int r = 0; r < 16; ++r)
					stg[((r >> 2) * 8 + (lane >> 5) * 4 + (r & 3)) * PITCH + j * 32 + (lane & 31)] =
						a[j][r];
		}
	};
	/* the strips unrolled (little code per strip, and the compiler may
	 * start a strip's stores under the MFMAs still finishing the others);
	 * EB / EG: bias / GELU with epilogue<CK>'s rounding points */
	auto fast_strips = [&](auto eb_t, auto eg_t) {
		constexpr bool EB = decltype(eb_t)::value, EG = decltype(eg_t)::value;
		constexpr int IT = UNITS / 64;
#pragma unroll
		for (int i = 0; i < FM; ++i) {
			stage(acc[i]);
			wave_lds_fence();
			float v[IT][W];
#pragma unroll
			for (int it = 0; it < IT; ++it)
				staged(lane + 64 * it, v[it]);
#pragma unroll
			for (int it = 0; it < IT; ++it) {
				const int s = lane + 64 * it;
				const int m = m0 + i * 32 + s / (WTN / W), n = n0 + (s % (WTN / W)) * W;
				if constexpr (EB || EG) {
#pragma unroll
					for (int e = 0; e < W; ++e)
						v[it][e] = epilogue<CK>(v[it][e], ein.b[e], (EB ? S3K_EPI_BIAS : 0) |
												(EG ? S3K_EPI_GELU : 0));
				}
				if (m < p.M) {
					/* streaming (non-temporal) stores: the tile is
					 * written once and not read back by this kernel,
					 * so it need not displace the operand panels
					 * other workgroups still read from the caches
					 * (fc1 983 -> 994 TFLOP/s, config 1 30.4 -> 29.0 us,
					 * Q K^T scores 241 -> 208 us). The general path
					 * below keeps plain stores: its operand copies
					 * and residual sums are read by the next kernel
					 * at once, and streaming stores there made the
					 * ViT block 3 % slower. */
					const long long o = (long long)m * p.ldc + n;
					if constexpr (CK == S3K_F32) {
						__builtin_nontemporal_store((s3k_f32x4){v[it][0], v[it][1], v[it][2], v[it][3]},
									    (s3k_f32x4 *)((float *)cb + o));
					} else {
						uint32_t w[4];
#pragma unroll
						for (int e = 0; e < 4; ++e)
							w[e] = CK == S3K_BF16 ? pack_bf16x2(v[it][2 * e], v[it][2 * e + 1])
									      : pack_f16x2(v[it][2 * e], v[it][2 * e + 1]);
						__builtin_nontemporal_store((s3k_u32x4){w[0], w[1], w[2], w[3]},
									    (s3k_u32x4 *)((uint16_t *)cb + o));
					}
				}
			}
			wave_lds_fence();
		}
	};
	/* S3K_EPI_QKV: the strips go out through LDS as in the fast path;
	 * each lane finishes four consecutive columns of a row (bias, then
	 * RoPE: the pairs (d, d + 1) and (d + 2, d + 3) never leave the lane)
	 * and writes them to one run of a head-split row. A row's 16 or 32
	 * lanes read one contiguous run of each table row, so a table load
	 * touches as many cache lines as a store does. The tables of strip
	 * i + 1 are loaded before strip i's stores: a load issued after a
	 * store would wait for that store too. */
	if constexpr (QKV_OK) {
		static_assert(TR && CK == S3K_F32 && FIXED, "QKV stores: transposed f32 tiles");
		{
			const int S = p.qkv_S, dsh = p.qkv_dsh, D = 1 << dsh, E = p.qkv_H << dsh;
			const bool eb = flags & S3K_EPI_BIAS;
			/* unit u of a strip: row u / LPR, columns (u % LPR) * 4 + [0, 4) */
			constexpr int LPR = WTN / W, RPI = 64 / LPR, IT = UNITS / 64;
			const int n = n0 + (lane % LPR) * W;
			const bool nok = n < p.N;
			const int y = (n >= E) + (n >= 2 * E), r = n - y * E;
			float *ob = nok ? (y == 0 ? p.qkv_out[0] : y == 1 ? p.qkv_out[1] : p.qkv_out[2]) +
						  (long long)(r >> dsh) * S * D + (r & (D - 1))
					: nullptr;
			const long long hsd = (long long)p.qkv_H * S * D;
			const bool rope = nok && ((p.qkv_rope >> y) & 1);
			/* this lane's rows: m1 + RPI*k for k = 0, 1, ... over the strips;
			 * (b, sr): the next row to store, st: the next row whose
			 * tables are loaded (RPI <= S, so one wrap at a time) */
			const int m1 = m0 + lane / LPR;
			int b = m1 / S, sr = m1 - b * S, st = sr;
			const unsigned tbytes = (unsigned)S * (unsigned)D * 2u;
			const __amdgpu_buffer_rsrc_t rc = __builtin_amdgcn_make_buffer_rsrc(
				(void *)p.qkv_cos, (short)0, (int)tbytes, 0x00020000);
			const __amdgpu_buffer_rsrc_t rsn = __builtin_amdgcn_make_buffer_rsrc(
				(void *)p.qkv_sin, (short)0, (int)tbytes, 0x00020000);
			/* byte offset of the lane's first pair in a table row; every
			 * offset stays inside the tables (s < S, d + 3 < D) */
			const unsigned dp = (unsigned)(n & (D - 1)) * 2u;
			float2 tc[2][IT], ts[2][IT];
			auto load_tables = [&](float2 (&c)[IT], float2 (&sn)[IT]) {
#pragma unroll
				for (int it = 0; it < IT; ++it) {
					const unsigned off = (unsigned)st * (unsigned)D * 2u + dp;
					c[it] = __builtin_bit_cast(float2, __builtin_amdgcn_raw_buffer_load_b64(rc, off, 0, 0));
					sn[it] = __builtin_bit_cast(float2, __builtin_amdgcn_raw_buffer_load_b64(rsn, off, 0, 0));
					st += RPI;
					if (st >= S)
						st -= S;
				}
			};
			if (p.qkv_rope)
				load_tables(tc[0], ts[0]);
#pragma unroll
			for (int i = 0; i < FM; ++i) {
				if (p.qkv_rope && i + 1 < FM)
					load_tables(tc[(i + 1) & 1], ts[(i + 1) & 1]);
				stage(acc[i]);
				wave_lds_fence();
				float v[IT][W];
#pragma unroll
				for (int it = 0; it < IT; ++it)
					staged(lane + 64 * it, v[it]);
#pragma unroll
				for (int it = 0; it < IT; ++it) {
					float x[4] = {v[it][0], v[it][1], v[it][2], v[it][3]};
					if (eb) {
#pragma unroll
						for (int q = 0; q < 4; ++q)
							x[q] = add_rn(x[q], ein.b[q]);
					}
					if (rope) {
						const float2 cc = tc[i & 1][it], ss = ts[i & 1][it];
						const float u0 = x[0], u1 = x[1], u2 = x[2], u3 = x[3];
						x[0] = sub_rn(mul_rn(u0, cc.x), mul_rn(u1, ss.x));
						x[1] = add_rn(mul_rn(u0, ss.x), mul_rn(u1, cc.x));
						x[2] = sub_rn(mul_rn(u2, cc.y), mul_rn(u3, ss.y));
						x[3] = add_rn(mul_rn(u2, ss.y), mul_rn(u3, cc.y));
					}
					const int m = m1 + 32 * i + RPI * it;
					if (m < p.M && nok)
						*(float4 *)(ob + b * hsd + (long long)sr * D) = make_float4(x[0], x[1], x[2], x[3]);
					sr += RPI;
					if (sr >= S) {
						sr -= S;
						++b;
					}
				}
				wave_lds_fence();
			}
			return;
		}
	}
	if (fast) {
		const bool eb = flags & S3K_EPI_BIAS, eg = flags & S3K_EPI_GELU;
		if (!eb && !eg)
			fast_strips(epi_b<false>{}, epi_b<false>{});
		else if (eb && eg)
			fast_strips(epi_b<true>{}, epi_b<true>{});
		else if (eb)
			fast_strips(epi_b<true>{}, epi_b<false>{});
		else
			fast_strips(epi_b<false>{}, epi_b<true>{});
		return;
	}
	/* S3K_C_F16OP: the largest |value| of this wave's part of each row
	 * (the WTN / W lanes holding the row's units in one round, when they
	 * divide the round; else each unit on its own) as row tags. Every lane
	 * calls it, so the shuffles see the whole wave. */
	auto row_tags = [&](float mx, int row) {
		constexpr int L = WTN / W;
		if constexpr (FIXED) {
#pragma unroll
			for (int off = 1; off < L; off <<= 1)
				mx = fmaxf(mx, __shfl_xor(mx, off));
			if ((lane & (L - 1)) == 0 && row < p.M)
				f16_row_tag(p, row, mx);
		} else {
			if (row < p.M)
				f16_row_tag(p, row, mx);
		}
	};
	/* The strip loop is rolled so that the store code exists once; the
	 * staging of strip i picks acc[i] by a wave-uniform branch (the
	 * accumulators stay in registers). */
#pragma unroll 1
	for (int i = 0; i < FM; ++i) {
#pragma unroll
		for (int ii = 0; ii < FM; ++ii)
			if (ii == i)
				stage(acc[ii]);
		wave_lds_fence();
		const int mrow = m0 + i * 32;
		float cur[W];
		staged(lane, cur);
		if (heavy) {
#pragma unroll 1
			for (int s = lane; s < UNITS; s += 64) {
				float nxt[W];
				if (s + 64 < UNITS)
					staged(s + 64, nxt);
				const int row = s / (WTN / W), cw = (s % (WTN / W)) * W;
				float mx = 0.0f;
				if (mrow + row < p.M && n0 + cw < p.N) {
					EpiIn<W> e = ein;
					epi_fetch<W>(p, mrow + row, n0 + cw, bz, !FIXED, e);
					mx = finishw<CK, true, W>(p, flags, cb, mrow + row, n0 + cw, cur, e);
				}
				if (CK == S3K_C_F16OP && p.rowf)
					row_tags(mx, mrow + row);
#pragma unroll
				for (int e = 0; e < W; ++e)
					cur[e] = nxt[e];
			}
		} else {
			/* all of the strip's staged values first, then the stores */
			constexpr int IT = UNITS / 64;
			float v[IT][W];
#pragma unroll
			for (int e = 0; e < W; ++e)
				v[0][e] = cur[e];
#pragma unroll
			for (int it = 1; it < IT; ++it)
				staged(lane + 64 * it, v[it]);
#pragma unroll
			for (int it = 0; it < IT; ++it) {
				const int s = lane + 64 * it;
				const int row = s / (WTN / W), cw = (s % (WTN / W)) * W;
				float mx = 0.0f;
				if (mrow + row < p.M && n0 + cw < p.N) {
					if (light)
						mx = finishw<CK, true, W>(p, flags, cb, mrow + row, n0 + cw, v[it], ein);
					else
						mx = finishw<CK, false, W>(p, flags, cb, mrow + row, n0 + cw, v[it], ein);
				}
				if (CK == S3K_C_F16OP && p.rowf)
					row_tags(mx, mrow + row);
			}
		}
		wave_lds_fence();
	}
}

/* Output kind chosen at run time (the register-staged kernels). */
template <int FM, int FN, int WTN>
__device__ __forceinline__ void write_tile(const GemmArgs &p, s3k_f32x16 (&acc)[FM][FN], char *smem,
					   int wave, int lane, int m0, int n0, int bz)
{
	if (p.c_kind == S3K_F32)
		write_tile_ck<FM, FN, WTN, S3K_F32>(p, acc, smem, wave, lane, m0, n0, bz);
	else if (p.c_kind == S3K_BF16)
		write_tile_ck<FM, FN, WTN, S3K_BF16>(p, acc, smem, wave, lane, m0, n0, bz);
	else
		write_tile_ck<FM, FN, WTN, S3K_F16>(p, acc, smem, wave, lane, m0, n0, bz);
}

} /* namespace s3k */

/* Direct-to-LDS bf16/f16 NT GEMM (gemm_dl.hip). */
bool s3k_dl_ok(const struct s3k_gemm *g);
int s3k_dl_launch(const struct s3k_gemm *g, s3k::GemmArgs p, hipStream_t st);
/* Direct-to-LDS GEMM with B stored [K, N], N <= 128 (gemm_dl.hip). */
bool s3k_dlt_ok(const struct s3k_gemm *g);
int s3k_dlt_launch(const struct s3k_gemm *g, s3k::GemmArgs p, hipStream_t st);

/* Direct-to-LDS f16 x Q8_0 NT GEMM, f32 out (gemm_dlq8.hip). */
bool s3k_dlq8_ok(const struct s3k_gemm *g);
int s3k_dlq8_launch(const struct s3k_gemm *g, s3k::GemmArgs p, hipStream_t st);

#endif /* SAM3_GEMM_COMMON_H */
