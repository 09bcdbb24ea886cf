/*
 * aux.hip - the small HBM-bound kernels around the matmul:
 *
 *   - Q8_0 -> f16 unpacking for Q8 layouts the tiled GEMM does not read
 *     directly: B[K,N] with blocks over the flat index k*N+n (the
 *     reference kernel contract, cpu_matmul_q8.c:29-35) and W[N,K] with
 *     K % 32 != 0 (blocks straddle rows), and the expansion of W[N,K]
 *     for the f16 GEMM. Output is f16 [N,K], value q*scale times the
 *     weight row's power-of-two factor, rounded once to f16
 *     (src/core/quant.c:134-165 gives q*scale), and the factors.
 *   - Q8_0 quantize / dequantize of flat f32 arrays on the device
 *     (src/core/quant.c:67-165), bit-exact with the reference's x86 build;
 *   - bias add over the last dim, same-shape add, tanh-GELU and 2-D
 *     transpose, with the reference's per-op rounding
 *     (cpu_elementwise.c:28-63, cpu_add_bf16.c:62-63, cpu_gelu.c:23-38,
 *     cpu_transpose.c:355-366), used when a graph pattern cannot fuse.
 */
#include <limits.h>

#include "s3k.h"
#include "s3k_dev.h"

namespace s3k {

/* Q8_0 [N,K] blocks along k (K % 32 == 0, every row whole blocks) ->
 * f16 [N,K] with the weight-row factors of s3k_q8_wfactors: one wave per
 * row, CPL 16-byte output chunks (8 values, a quarter of a block) per
 * lane. Every lane first loads its chunks' block scales and q dwords;
 * the row's largest |scale| over those (every block is some lane's)
 * gives the factor 2^e, stored to cs[n]; then the outputs
 * f16(q * (scale * 2^-e)), q * scale' formed in f32 and rounded once. At
 * e = 0 these are the plain q * scale. A wave's stores are one
 * contiguous KiB per round. */
__device__ __forceinline__ uint32_t q8_pair_to_f16(uint32_t d, int sh, float s)
{
	return f32_to_f16((float)(int)(int8_t)(d >> sh) * s) |
	       (f32_to_f16((float)(int)(int8_t)(d >> (sh + 8)) * s) << 16);
}

template <int CPL>
__device__ __forceinline__ void expand_row(const char *blk, uint16_t *out, float *cs, int K, int n,
					   int lane)
{
	const int chunks = K / 8;
	const char *row = blk + (long long)n * (K / 32) * 36;
	float s[CPL];
	uint32_t d0[CPL], d1[CPL];
	float m = 0.0f;
#pragma unroll
	for (int u = 0; u < CPL; ++u) {
		const int c = lane + 64 * u;
		s[u] = 0.0f;
		d0[u] = d1[u] = 0u;
		if (c < chunks) {
			const char *b = row + (c >> 2) * 36;
			s[u] = *(const float *)b;
			d0[u] = *(const uint32_t *)(b + 4 + 8 * (c & 3));
			d1[u] = *(const uint32_t *)(b + 8 + 8 * (c & 3));
			m = fmaxf(m, finite_abs(s[u]));
		}
	}
	const int e = wscale_exp_of(127.0f * wave_max_f32(m));
	if (lane == 0)
		cs[n] = pow2f(e);
	const float inv = pow2f(-e);
	uint4 *o = (uint4 *)(out + (long long)n * K);
#pragma unroll
	for (int u = 0; u < CPL; ++u) {
		const int c = lane + 64 * u;
		const float sc = s[u] * inv;
		if (c < chunks)
			o[c] = make_uint4(q8_pair_to_f16(d0[u], 0, sc), q8_pair_to_f16(d0[u], 16, sc),
					  q8_pair_to_f16(d1[u], 0, sc), q8_pair_to_f16(d1[u], 16, sc));
	}
}

/* four rows per workgroup (K <= 512 * CPL) */
template <int CPL>
__global__ void __launch_bounds__(256) q8_expand_rows_k(const char *blk, uint16_t *out, float *cs,
							int K, int N)
{
	const int n = blockIdx.x * 4 + (threadIdx.x >> 6);
	if (n < N)
		expand_row<CPL>(blk, out, cs, K, n, threadIdx.x & 63);
}

/* The factors alone (s3k_q8_wfactors). [N,K] over the flat index (slices
 * sb bytes apart): one wave per row n. Rows of whole blocks (K % 32 ==
 * 0) take 127 * their largest |scale|; a row that shares blocks with its
 * neighbours (another row's values may have set a block's scale) takes
 * the largest |q| * |scale| over its own elements. */
__global__ void __launch_bounds__(256) q8_wfac_nk_k(const char *blk, float *cs, int K, int N,
						    long long sb)
{
	const int lane = threadIdx.x & 63;
	const int n = blockIdx.x * 4 + (threadIdx.x >> 6);
	if (n >= N)
		return;
	const char *b = blk + (long long)blockIdx.y * sb;
	float m = 0.0f;
	if (K % 32 == 0) {
		const long long b0 = (long long)n * (K / 32);
		for (int i = lane; i < K / 32; i += 64)
			m = fmaxf(m, finite_abs(*(const float *)(b + (b0 + i) * 36)));
		m *= 127.0f;
	} else {
		for (int k = lane; k < K; k += 64) {
			const long long lin = (long long)n * K + k;
			const char *bk = b + (lin >> 5) * 36;
			const float q = (float)__builtin_abs((int)(int8_t)bk[4 + (lin & 31)]);
			m = fmaxf(m, finite_abs(*(const float *)bk) * q);
		}
	}
	m = wave_max_f32(m);
	if (lane == 0)
		cs[(long long)blockIdx.y * N + n] = pow2f(wscale_exp_of(m));
}

/* [K,N] with blocks over k*N+n (a block spans 32 columns): column n
 * takes the largest |q| * |scale| over its own elements; 64 columns per
 * workgroup, its four waves splitting k. */
__global__ void __launch_bounds__(256) q8_wfac_kn_k(const char *blk, float *cs, int K, int N)
{
	__shared__ float part[4][64];
	const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
	const int n = blockIdx.x * 64 + lane;
	float m = 0.0f;
	if (n < N)
		for (int k = w; k < K; k += 4) {
			const long long lin = (long long)k * N + n;
			const char *bk = blk + (lin >> 5) * 36;
			const float q = (float)__builtin_abs((int)(int8_t)bk[4 + (lin & 31)]);
			m = fmaxf(m, finite_abs(*(const float *)bk) * q);
		}
	part[w][lane] = m;
	__syncthreads();
	if (w == 0 && n < N)
		cs[n] = pow2f(wscale_exp_of(fmaxf(fmaxf(part[0][lane], part[1][lane]),
						  fmaxf(part[2][lane], part[3][lane]))));
}

/* Row tags of f16 operand writers (s3k_rowflag_check): one thread per
 * row, over up to 32 tag arrays (blockIdx.y). */
struct RowFlagSet {
	unsigned *f[32];
	int rows[32];
};

__global__ void __launch_bounds__(256) rowflag_check_k(RowFlagSet s, unsigned tag, unsigned *ovf)
{
	const int y = blockIdx.y;
	const long long m = (long long)blockIdx.x * 256 + threadIdx.x;
	if (m >= s.rows[y])
		return;
	const unsigned *f = s.f[y] + 2 * m;
	if (f[1] == tag && f[0] != tag)
		*ovf = tag;
}

/* One thread per output of f16 [N,K]; element (n,k) reads block lin/32
 * of the flat Q8 array, lin = k*N+n (KN) or n*K+k (NK, rows that split
 * blocks), and is stored as f16(q * (scale / cs[n])). */
template <bool KN>
__global__ void __launch_bounds__(256) q8_to_f16_nk(const char *blk, uint16_t *out,
						    const float *cs, int K, int N)
{
	const long long i = (long long)blockIdx.x * 256 + threadIdx.x;
	const long long tot = (long long)N * K;
	if (i >= tot)
		return;
	const int n = (int)(i / K), k = (int)(i % K);
	const long long lin = KN ? (long long)k * N + n : i;
	const char *b = blk + (lin >> 5) * 36;
	const float s = *(const float *)b * inv_pow2(cs[n]);
	const float q = (float)(int)(int8_t)b[4 + (lin & 31)];
	out[i] = (uint16_t)f32_to_f16(q * s);
}

/*
 * Q8_0 quantization of a flat f32 array, the x86 branch of
 * sam3_q8_quantize (src/core/quant.c:67-130): per block of 32,
 * amax = max |x| over the block's elements (NaN never wins, as with
 * `if (a > amax)`), scale = amax / 127.0f, and if scale != 0,
 * q = clamp((int)roundf(x * (1.0f / scale)), -127, 127) with roundf
 * rounding halves away from zero. (int) of a NaN or of a value outside the
 * int range gives INT_MIN there (cvttss2si), which the clamp maps to -127;
 * the same rule is applied here. Elements past n, and whole blocks with a
 * zero scale, store q = 0. Eight lanes per block, four elements per lane:
 * the block's amax is a max over the 8 lanes (exact in any order), and
 * each lane stores its four q as one dword.
 */
__global__ void __launch_bounds__(256) q8_quantize_k(const float *src, char *dst, int n)
{
	const long long t = (long long)blockIdx.x * 256 + threadIdx.x;
	const long long b = t >> 3;
	const int part = (int)(t & 7);
	if (b >= ((long long)n + 31) / 32)
		return; /* whole 8-lane groups leave together */
	const long long e0 = b * 32 + part * 4;
	float x[4];
	float amax = 0.0f;
#pragma unroll
	for (int i = 0; i < 4; ++i) {
		x[i] = e0 + i < n ? src[e0 + i] : 0.0f;
		const float a = fabsf(x[i]);
		if (e0 + i < n && a > amax)
			amax = a;
	}
#pragma unroll
	for (int o = 1; o < 8; o <<= 1) {
		const float v = __shfl_xor(amax, o, 8);
		if (v > amax)
			amax = v;
	}
	const float scale = amax / 127.0f;
	char *blk = dst + b * 36;
	if (part == 0)
		*(float *)blk = scale;
	uint32_t word = 0;
	if (scale != 0.0f) {
		const float inv = 1.0f / scale;
#pragma unroll
		for (int i = 0; i < 4; ++i) {
			if (e0 + i >= n)
				continue;
			const float r = roundf(x[i] * inv);
			int q = (r >= -2147483648.0f && r < 2147483648.0f) ? (int)r : INT_MIN;
			q = q > 127 ? 127 : q < -127 ? -127 : q;
			word |= (uint32_t)(uint8_t)(int8_t)q << (8 * i);
		}
	}
	*(uint32_t *)(blk + 4 + 4 * part) = word;
}

/* x = (float)q * scale (src/core/quant.c:134-165), four per lane. */
__global__ void __launch_bounds__(256) q8_dequantize_k(const char *src, float *dst, int n)
{
	const long long t = (long long)blockIdx.x * 256 + threadIdx.x;
	const long long b = t >> 3;
	const int part = (int)(t & 7);
	if (b >= ((long long)n + 31) / 32)
		return;
	const char *blk = src + b * 36;
	const float s = *(const float *)blk;
	const uint32_t w = *(const uint32_t *)(blk + 4 + 4 * part);
	const long long e0 = b * 32 + part * 4;
#pragma unroll
	for (int i = 0; i < 4; ++i)
		if (e0 + i < n)
			dst[e0 + i] = (float)(int)(int8_t)(w >> (8 * i)) * s;
}

/* f32 or bf16 -> f16 (round to nearest even); the f16 staging of
 * activations for the Q8 GEMM. A thread converts U chunks of 8 values,
 * chunks gridDim*256 apart, and issues all of its loads before the first
 * conversion, so each wave keeps U 16-byte (bf16) or 2U (f32) loads per
 * lane in flight instead of one. The n % 8 tail goes to the first lanes
 * of workgroup 0. */
template <bool BF16, int U>
__global__ void __launch_bounds__(256) cast_f16_k(const void *src, uint16_t *dst, long long n)
{
	constexpr int L = BF16 ? 1 : 2; /* 16-byte loads per chunk */
	const long long chunks = n / 8, stride = (long long)gridDim.x * 256;
	for (long long c0 = (long long)blockIdx.x * 256 + threadIdx.x; c0 < chunks; c0 += stride * U) {
		uint4 v[U][L];
#pragma unroll
		for (int u = 0; u < U; ++u) {
			const long long c = c0 + u * stride;
			if (c < chunks) {
#pragma unroll
				for (int l = 0; l < L; ++l)
					v[u][l] = ((const uint4 *)src)[c * L + l];
			}
		}
#pragma unroll
		for (int u = 0; u < U; ++u) {
			const long long c = c0 + u * stride;
			if (c >= chunks)
				break;
			float x[8];
			if (BF16) {
				const uint32_t w[4] = {v[u][0].x, v[u][0].y, v[u][0].z, v[u][0].w};
#pragma unroll
				for (int e = 0; e < 4; ++e) {
					x[2 * e] = bf16_to_f32(w[e] & 0xFFFFu);
					x[2 * e + 1] = bf16_to_f32(w[e] >> 16);
				}
			} else {
#pragma unroll
				for (int l = 0; l < L; ++l) {
					x[4 * l] = __uint_as_float(v[u][l].x);
					x[4 * l + 1] = __uint_as_float(v[u][l].y);
					x[4 * l + 2] = __uint_as_float(v[u][l].z);
					x[4 * l + 3] = __uint_as_float(v[u][l].w);
				}
			}
			((uint4 *)dst)[c] = make_uint4(pack_f16x2(x[0], x[1]), pack_f16x2(x[2], x[3]),
						       pack_f16x2(x[4], x[5]), pack_f16x2(x[6], x[7]));
		}
	}
	if (blockIdx.x == 0 && threadIdx.x < (n & 7)) {
		const long long i = chunks * 8 + threadIdx.x;
		dst[i] = (uint16_t)f32_to_f16(BF16 ? bf16_to_f32(((const uint16_t *)src)[i])
						  : ((const float *)src)[i]);
	}
}

/* Row-scaled f16 copy of activations (s3k_cast_f16_rows): one wave per
 * row. The row's largest finite |x| picks a power-of-two factor 2^e
 * (e = 0 when it lies in [2^-10, 2^15) or is 0, else the e that puts it
 * in [2^14, 2^15)); the row is stored as f16(x * 2^-e), rs = 2^e. With
 * VEC the row moves in 16-byte chunks of 8 values, up to CPL chunks per
 * lane held in registers between the two passes (rows 16-byte aligned,
 * K % 8 == 0, K <= 512 * CPL); otherwise values are read one at a time,
 * twice. */
/* One row of K values (16-byte chunks of 8, up to CPL per lane) to f16
 * with its row factor, by one wave: every load first, then the row's
 * largest |value|, then the stores. */
template <bool BF16, int CPL>
__device__ __forceinline__ void cast_row_vec(const char *xrow, uint16_t *y, float *rsp, int K,
					     int lane)
{
	constexpr int L = BF16 ? 1 : 2;
	const int chunks = K / 8;
	const uint4 *x = (const uint4 *)xrow;
	uint4 v[CPL][L];
#pragma unroll
	for (int u = 0; u < CPL; ++u) {
		const int c = lane + 64 * u;
#pragma unroll
		for (int l = 0; l < L; ++l)
			v[u][l] = c < chunks ? x[c * L + l] : make_uint4(0, 0, 0, 0);
	}
	float f[CPL][8];
	float amax = 0.0f;
#pragma unroll
	for (int u = 0; u < CPL; ++u) {
		if constexpr (BF16) {
			const uint32_t w[4] = {v[u][0].x, v[u][0].y, v[u][0].z, v[u][0].w};
#pragma unroll
			for (int e = 0; e < 4; ++e) {
				f[u][2 * e] = bf16_to_f32(w[e] & 0xFFFFu);
				f[u][2 * e + 1] = bf16_to_f32(w[e] >> 16);
			}
		} else {
#pragma unroll
			for (int l = 0; l < 2; ++l) {
				f[u][4 * l] = __uint_as_float(v[u][l].x);
				f[u][4 * l + 1] = __uint_as_float(v[u][l].y);
				f[u][4 * l + 2] = __uint_as_float(v[u][l].z);
				f[u][4 * l + 3] = __uint_as_float(v[u][l].w);
			}
		}
#pragma unroll
		for (int e = 0; e < 8; ++e)
			amax = fmaxf(amax, finite_abs(f[u][e]));
	}
	const int ex = row_scale_exp(amax);
	const float inv = pow2f(-ex);
#pragma unroll
	for (int u = 0; u < CPL; ++u) {
		const int c = lane + 64 * u;
		if (c < chunks)
			((uint4 *)y)[c] = make_uint4(pack_f16x2(f[u][0] * inv, f[u][1] * inv),
						     pack_f16x2(f[u][2] * inv, f[u][3] * inv),
						     pack_f16x2(f[u][4] * inv, f[u][5] * inv),
						     pack_f16x2(f[u][6] * inv, f[u][7] * inv));
	}
	if (lane == 0)
		*rsp = pow2f(ex);
}

/* One row per wave, four rows per workgroup. With VEC the row moves in
 * 16-byte chunks (cast_row_vec); otherwise values are read one at a
 * time, twice. */
template <bool BF16, bool VEC, int CPL>
__global__ void __launch_bounds__(256) cast_f16_rows_k(const char *src, long long lda_b,
						       long long sa_b, uint16_t *dst, float *rs,
						       int M, int K)
{
	const int lane = threadIdx.x & 63;
	const int m = blockIdx.x * 4 + (threadIdx.x >> 6);
	if (m >= M)
		return;
	const char *x = src + (long long)blockIdx.y * sa_b + (long long)m * lda_b;
	const long long row = (long long)blockIdx.y * M + m;
	uint16_t *y = dst + row * K;
	if constexpr (VEC) {
		cast_row_vec<BF16, CPL>(x, y, rs + row, K, lane);
	} else {
		float amax = 0.0f;
		for (int k = lane; k < K; k += 64)
			amax = fmaxf(amax, finite_abs(BF16 ? bf16_to_f32(((const uint16_t *)x)[k])
							: ((const float *)x)[k]));
		const int ex = row_scale_exp(amax);
		const float inv = pow2f(-ex);
		for (int k = lane; k < K; k += 64)
			y[k] = (uint16_t)f32_to_f16((BF16 ? bf16_to_f32(((const uint16_t *)x)[k])
						     : ((const float *)x)[k]) * inv);
		if (lane == 0)
			rs[row] = pow2f(ex);
	}
}

/* The row cast of A and the expansion of a Q8_0 weight in one launch:
 * workgroups [0, row_wgs) cast four rows of A each, the rest expand four
 * weight rows each (expand_row, with their factors). The two are
 * independent and short, so one launch lets them overlap instead of
 * paying two dispatch ramps. */
template <bool BF16, int CPL>
__global__ void __launch_bounds__(256) cast_expand_k(const char *src, long long lda_b,
						     uint16_t *dst, float *rs, int M, int K,
						     const char *blk, uint16_t *wout, float *cs, int N,
						     int row_wgs)
{
	if ((int)blockIdx.x < row_wgs) {
		const int m = blockIdx.x * 4 + (threadIdx.x >> 6);
		if (m < M)
			cast_row_vec<BF16, CPL>(src + (long long)m * lda_b, dst + (long long)m * K, rs + m,
						K, threadIdx.x & 63);
	} else {
		const int n = (blockIdx.x - row_wgs) * 4 + (threadIdx.x >> 6);
		if (n < N)
			expand_row<CPL>(blk, wout, cs, K, n, threadIdx.x & 63);
	}
}

/* CAST between f32, f16 and bf16 (cpu_cast.c:26-145): one element per
 * thread and step. HW = false converts by integer arithmetic, bit-exact
 * with half.h; HW = true uses the conversion instructions the GEMM
 * epilogues use (v_cvt_pk_bf16_f32, v_cvt_f16_f32, v_cvt_f32_f16). */
template <int SRC, int DST, bool HW>
__global__ void __launch_bounds__(256) cast_k(const void *src, void *dst, long long n)
{
	const long long stride = (long long)gridDim.x * 256;
	for (long long i = (long long)blockIdx.x * 256 + threadIdx.x; i < n; i += stride) {
		float v;
		if constexpr (SRC == S3K_F32) {
			v = ((const float *)src)[i];
		} else {
			const uint32_t h = ((const uint16_t *)src)[i];
			if constexpr (SRC == S3K_BF16)
				v = bf16_to_f32(h);
			else
				v = HW ? f16_to_f32(h) : f16_to_f32_sw(h);
		}
		if constexpr (DST == S3K_F32)
			((float *)dst)[i] = v;
		else if constexpr (DST == S3K_BF16)
			((uint16_t *)dst)[i] = (uint16_t)(HW ? pack_bf16x2(v, 0.0f) & 0xFFFFu : f32_to_bf16(v));
		else
			((uint16_t *)dst)[i] = (uint16_t)(HW ? f32_to_f16(v) : f32_to_f16_sw(v));
	}
}

template <int KIND>
__global__ void __launch_bounds__(256) bias_add_k(const void *x, const void *bias, void *out,
						  long long rows, int n)
{
	const long long i = (long long)blockIdx.x * 256 + threadIdx.x;
	if (i >= rows * n)
		return;
	const float v = add_rn(load_as_f32(x, i, KIND), load_as_f32(bias, i % n, KIND));
	store_from_f32(out, i, KIND, v);
}

template <int KIND>
__global__ void __launch_bounds__(256) add_same_k(const void *x, const void *y, void *out, long long n)
{
	const long long i = (long long)blockIdx.x * 256 + threadIdx.x;
	if (i >= n)
		return;
	store_from_f32(out, i, KIND, add_rn(load_as_f32(x, i, KIND), load_as_f32(y, i, KIND)));
}

template <int KIND>
__global__ void __launch_bounds__(256) gelu_k(const void *x, void *out, long long n)
{
	const long long i = (long long)blockIdx.x * 256 + threadIdx.x;
	if (i >= n)
		return;
	store_from_f32(out, i, KIND, gelu_tanh(load_as_f32(x, i, KIND)));
}

/* 32x32 tiles through LDS; blockIdx.z walks the [rows, cols] slices. */
template <typename T>
__global__ void __launch_bounds__(256) transpose_k(const T *src, T *dst, int rows, int cols)
{
	__shared__ T tile[32][33];
	const int c0 = blockIdx.x * 32, r0 = blockIdx.y * 32;
	src += (long long)blockIdx.z * rows * cols;
	dst += (long long)blockIdx.z * rows * cols;
	const int tx = threadIdx.x & 31, ty = threadIdx.x >> 5;
	for (int y = ty; y < 32; y += 8) {
		const int r = r0 + y, c = c0 + tx;
		if (r < rows && c < cols)
			tile[y][tx] = src[(long long)r * cols + c];
	}
	__syncthreads();
	for (int y = ty; y < 32; y += 8) {
		const int c = c0 + y, r = r0 + tx;
		if (r < rows && c < cols)
			dst[(long long)c * rows + r] = tile[tx][y];
	}
}

} /* namespace s3k */

using namespace s3k;

static dim3 grid1(long long n)
{
	return dim3((unsigned)((n + 255) / 256));
}

extern "C" int s3k_rowflag_check(int n, unsigned *const *flags, const int *rows, unsigned tag,
				 unsigned *ovf, void *stream)
{
	if (n <= 0)
		return 0;
	if (n > 32 || !ovf)
		return (int)hipErrorInvalidValue;
	RowFlagSet s = {};
	int most = 0;
	for (int i = 0; i < n; ++i) {
		if (!flags[i] || rows[i] < 0)
			return (int)hipErrorInvalidValue;
		s.f[i] = flags[i];
		s.rows[i] = rows[i];
		most = rows[i] > most ? rows[i] : most;
	}
	if (most == 0)
		return 0;
	hipLaunchKernelGGL(rowflag_check_k, dim3((unsigned)((most + 255) / 256), (unsigned)n),
			   dim3(256), 0, (hipStream_t)stream, s, tag, ovf);
	return (int)hipGetLastError();
}

extern "C" int s3k_q8_wfactors(const void *blocks, float *cs, int K, int N, int nt, int batch,
			       long long stride_b, void *stream)
{
	if (K <= 0 || N <= 0 || batch <= 0 || !cs || ((uintptr_t)blocks & 3u) || (!nt && batch != 1) ||
	    batch > 65535)
		return (int)hipErrorInvalidValue;
	if (nt)
		hipLaunchKernelGGL(q8_wfac_nk_k, dim3((unsigned)((N + 3) / 4), (unsigned)batch),
				   dim3(256), 0, (hipStream_t)stream, (const char *)blocks, cs, K, N,
				   stride_b);
	else
		hipLaunchKernelGGL(q8_wfac_kn_k, dim3((unsigned)((N + 63) / 64)), dim3(256), 0,
				   (hipStream_t)stream, (const char *)blocks, cs, K, N);
	return (int)hipGetLastError();
}

extern "C" int s3k_q8_kn_to_f16_nk(const void *blocks, void *out, const float *cs, int K, int N,
				   void *stream)
{
	const long long tot = (long long)K * N;
	if (tot <= 0)
		return 0;
	if (!cs)
		return (int)hipErrorInvalidValue;
	hipLaunchKernelGGL(q8_to_f16_nk<true>, grid1(tot), dim3(256), 0, (hipStream_t)stream,
			   (const char *)blocks, (uint16_t *)out, cs, K, N);
	return (int)hipGetLastError();
}

extern "C" int s3k_q8_nk_to_f16_nk(const void *blocks, void *out, float *cs, int K, int N,
				   void *stream)
{
	const long long tot = (long long)K * N;
	if (tot <= 0)
		return 0;
	if (!cs)
		return (int)hipErrorInvalidValue;
	hipStream_t st = (hipStream_t)stream;
	if (K % 32 == 0 && K <= 4096 && !((uintptr_t)blocks & 3u) && !((uintptr_t)out & 15u)) {
		const int cpl = (K / 8 + 63) / 64;
		const dim3 grid((unsigned)((N + 3) / 4));
		const char *b = (const char *)blocks;
		uint16_t *o = (uint16_t *)out;
		if (cpl <= 2)
			hipLaunchKernelGGL(q8_expand_rows_k<2>, grid, dim3(256), 0, st, b, o, cs, K, N);
		else if (cpl <= 4)
			hipLaunchKernelGGL(q8_expand_rows_k<4>, grid, dim3(256), 0, st, b, o, cs, K, N);
		else
			hipLaunchKernelGGL(q8_expand_rows_k<8>, grid, dim3(256), 0, st, b, o, cs, K, N);
		return (int)hipGetLastError();
	}
	const int e = s3k_q8_wfactors(blocks, cs, K, N, 1, 1, 0, stream);
	if (e)
		return e;
	hipLaunchKernelGGL(q8_to_f16_nk<false>, grid1(tot), dim3(256), 0, st, (const char *)blocks,
			   (uint16_t *)out, cs, K, N);
	return (int)hipGetLastError();
}

extern "C" int s3k_q8_quantize(const void *src, void *dst, int n, void *stream)
{
	if (n <= 0)
		return 0;
	const long long lanes = ((long long)n + 31) / 32 * 8;
	hipLaunchKernelGGL(q8_quantize_k, grid1(lanes), dim3(256), 0, (hipStream_t)stream,
			   (const float *)src, (char *)dst, n);
	return (int)hipGetLastError();
}

extern "C" int s3k_q8_dequantize(const void *src, void *dst, int n, void *stream)
{
	if (n <= 0)
		return 0;
	const long long lanes = ((long long)n + 31) / 32 * 8;
	hipLaunchKernelGGL(q8_dequantize_k, grid1(lanes), dim3(256), 0, (hipStream_t)stream,
			   (const char *)src, (float *)dst, n);
	return (int)hipGetLastError();
}

/* f32 rows [rows, K] (row pitch ld elements) -> bf16 rows [rows, 3K] of
 * hi = bf16(x) and lo = bf16(x - hi) in the order [hi, lo, hi] (order 0)
 * or [hi, hi, lo] (order 1): a bf16 GEMM of one against the other over
 * 3K sums hi*hi + lo*hi + hi*lo. One thread per 8 values of a row. */
__global__ void __launch_bounds__(256) split3_bf16_k(const float *src, uint16_t *dst, int rows,
						     int K, long long ld, int order)
{
	const int per_row = K / 8;
	const long long t = (long long)blockIdx.x * 256 + threadIdx.x;
	if (t >= (long long)rows * per_row)
		return;
	const long long r = t / per_row;
	const int k0 = (int)(t % per_row) * 8;
	const float4 a = *(const float4 *)(src + r * ld + k0);
	const float4 b = *(const float4 *)(src + r * ld + k0 + 4);
	uint4 H, L;
	split_bf16x2(a.x, a.y, H.x, L.x);
	split_bf16x2(a.z, a.w, H.y, L.y);
	split_bf16x2(b.x, b.y, H.z, L.z);
	split_bf16x2(b.z, b.w, H.w, L.w);
	uint16_t *d = dst + r * 3LL * K + k0;
	*(uint4 *)d = H;
	if (order == 0) {
		*(uint4 *)(d + K) = L;
		*(uint4 *)(d + 2LL * K) = H;
	} else {
		*(uint4 *)(d + K) = H;
		*(uint4 *)(d + 2LL * K) = L;
	}
}

extern "C" int s3k_split3_bf16(const float *src, void *dst, int rows, int K, long long ld,
			       int order, void *stream)
{
	if (rows < 0 || K <= 0 || K % 8 || ld < K || ld % 4 || (((uintptr_t)src | (uintptr_t)dst) & 15u))
		return (int)hipErrorInvalidValue;
	const long long n = (long long)rows * (K / 8);
	if (n == 0)
		return 0;
	hipLaunchKernelGGL(split3_bf16_k, dim3((unsigned)((n + 255) / 256)), dim3(256), 0,
			   (hipStream_t)stream, src, (uint16_t *)dst, rows, K, ld, order);
	return (int)hipGetLastError();
}

extern "C" int s3k_cast_f16(int kind, const void *src, void *dst, long long n, void *stream)
{
	if (n <= 0)
		return 0;
	if (((uintptr_t)src | (uintptr_t)dst) & 15u)
		return (int)hipErrorInvalidValue;
	/* U chunks of 8 values per thread: 4 for bf16 (64 bytes in flight per
	 * lane), 2 for f32 (64 bytes) */
	const long long chunks = n / 8 > 0 ? n / 8 : 1;
	if (kind == S3K_BF16)
		hipLaunchKernelGGL((cast_f16_k<true, 4>), dim3((unsigned)((chunks + 1023) / 1024)), dim3(256),
				   0, (hipStream_t)stream, src, (uint16_t *)dst, n);
	else if (kind == S3K_F32)
		hipLaunchKernelGGL((cast_f16_k<false, 2>), dim3((unsigned)((chunks + 511) / 512)), dim3(256),
				   0, (hipStream_t)stream, src, (uint16_t *)dst, n);
	else
		return (int)hipErrorInvalidValue;
	return (int)hipGetLastError();
}

/* One row per wave. Several rows per wave (more loads in flight per
 * lane) measured slower at M = 5184, K = 1024: 6.1 us against 4.7 us for
 * bf16, 8.6 against 5.0 for f32, as fewer waves leave less overlap of
 * one wave's loads with another's stores. */
template <bool BF16>
static int cast_rows_launch(const char *src, long long lda_b, long long sa_b, uint16_t *dst,
			    float *rs, int batch, int M, int K, bool vec, hipStream_t st)
{
	const int cpl = (K / 8 + 63) / 64;
	const dim3 grid((unsigned)((M + 3) / 4), (unsigned)batch);
	if (!vec || cpl > 8)
		hipLaunchKernelGGL((cast_f16_rows_k<BF16, false, 1>), grid, dim3(256), 0, st, src,
				   lda_b, sa_b, dst, rs, M, K);
	else if (cpl <= 2)
		hipLaunchKernelGGL((cast_f16_rows_k<BF16, true, 2>), grid, dim3(256), 0, st, src,
				   lda_b, sa_b, dst, rs, M, K);
	else if (cpl <= 4)
		hipLaunchKernelGGL((cast_f16_rows_k<BF16, true, 4>), grid, dim3(256), 0, st, src,
				   lda_b, sa_b, dst, rs, M, K);
	else
		hipLaunchKernelGGL((cast_f16_rows_k<BF16, true, 8>), grid, dim3(256), 0, st, src,
				   lda_b, sa_b, dst, rs, M, K);
	return (int)hipGetLastError();
}

template <bool BF16>
static int cast_expand_launch(const char *src, long long lda_b, uint16_t *dst, float *rs, int M,
			      int K, const char *blk, uint16_t *wout, float *cs, int N, hipStream_t st)
{
	const int cpl = (K / 8 + 63) / 64;
	const int row_wgs = (M + 3) / 4;
	const dim3 grid((unsigned)(row_wgs + (N + 3) / 4));
	if (cpl <= 2)
		hipLaunchKernelGGL((cast_expand_k<BF16, 2>), grid, dim3(256), 0, st, src, lda_b, dst, rs,
				   M, K, blk, wout, cs, N, row_wgs);
	else if (cpl <= 4)
		hipLaunchKernelGGL((cast_expand_k<BF16, 4>), grid, dim3(256), 0, st, src, lda_b, dst, rs,
				   M, K, blk, wout, cs, N, row_wgs);
	else
		hipLaunchKernelGGL((cast_expand_k<BF16, 8>), grid, dim3(256), 0, st, src, lda_b, dst, rs,
				   M, K, blk, wout, cs, N, row_wgs);
	return (int)hipGetLastError();
}

/* A (f32 or bf16 [M, K], pitch lda elements) to row-scaled f16 rows plus
 * factors (as s3k_cast_f16_rows, one batch), and W (Q8_0 [N, K]) to f16
 * [N, K] with its factors cs (as s3k_q8_nk_to_f16_nk), in one launch.
 * hipErrorInvalidValue when the shapes or alignments do not allow it
 * (K % 32, K > 4096, 16-byte rows): the caller then uses the two
 * separate launches. */
extern "C" int s3k_cast_rows_expand(int kind, const void *src, long long lda, void *dst, float *rs,
				    int M, int K, const void *wblk, void *wout, float *cs, int N,
				    void *stream)
{
	const int es = kind == S3K_F32 ? 4 : 2;
	if ((kind != S3K_F32 && kind != S3K_BF16) || M <= 0 || N <= 0 || K <= 0 || K % 32 ||
	    K > 4096 || M > (1 << 28) || N > (1 << 28) || (lda * es) % 16 || lda < K ||
	    (((uintptr_t)src | (uintptr_t)dst | (uintptr_t)wout) & 15u) || ((uintptr_t)wblk & 3u) ||
	    !rs || !cs)
		return (int)hipErrorInvalidValue;
	hipStream_t st = (hipStream_t)stream;
	return kind == S3K_BF16
		? cast_expand_launch<true>((const char *)src, lda * es, (uint16_t *)dst, rs, M, K,
					   (const char *)wblk, (uint16_t *)wout, cs, N, st)
		: cast_expand_launch<false>((const char *)src, lda * es, (uint16_t *)dst, rs, M, K,
					    (const char *)wblk, (uint16_t *)wout, cs, N, st);
}

extern "C" int s3k_cast_f16_rows(int kind, const void *src, long long lda, long long sa, void *dst,
				 float *rs, int batch, int M, int K, void *stream)
{
	if (batch <= 0 || M <= 0 || K <= 0)
		return 0;
	if ((kind != S3K_F32 && kind != S3K_BF16) || !src || !dst || !rs || M > (1 << 30) ||
	    batch > 65535)
		return (int)hipErrorInvalidValue;
	const int es = kind == S3K_F32 ? 4 : 2;
	const bool vec = K % 8 == 0 && !(((uintptr_t)src | (uintptr_t)dst) & 15u) &&
			 (lda * es) % 16 == 0 && (sa * es) % 16 == 0;
	hipStream_t st = (hipStream_t)stream;
	return kind == S3K_BF16
		? cast_rows_launch<true>((const char *)src, lda * es, sa * es, (uint16_t *)dst, rs,
					 batch, M, K, vec, st)
		: cast_rows_launch<false>((const char *)src, lda * es, sa * es, (uint16_t *)dst, rs,
					  batch, M, K, vec, st);
}

template <int SRC, int DST>
static void cast_launch(const void *src, void *dst, long long n, bool hw, hipStream_t st)
{
	const long long blocks = (n + 255) / 256;
	const dim3 grid((unsigned)(blocks < 16384 ? blocks : 16384));
	if (hw)
		hipLaunchKernelGGL((cast_k<SRC, DST, true>), grid, dim3(256), 0, st, src, dst, n);
	else
		hipLaunchKernelGGL((cast_k<SRC, DST, false>), grid, dim3(256), 0, st, src, dst, n);
}

extern "C" int s3k_cast(int src_kind, int dst_kind, const void *src, void *dst, long long n, int hw,
			void *stream)
{
	if (n <= 0)
		return 0;
	const hipStream_t st = (hipStream_t)stream;
	switch (src_kind * 8 + dst_kind) {
	case S3K_F32 * 8 + S3K_F16:  cast_launch<S3K_F32, S3K_F16>(src, dst, n, hw, st); break;
	case S3K_F32 * 8 + S3K_BF16: cast_launch<S3K_F32, S3K_BF16>(src, dst, n, hw, st); break;
	case S3K_F16 * 8 + S3K_F32:  cast_launch<S3K_F16, S3K_F32>(src, dst, n, hw, st); break;
	case S3K_F16 * 8 + S3K_BF16: cast_launch<S3K_F16, S3K_BF16>(src, dst, n, hw, st); break;
	case S3K_BF16 * 8 + S3K_F32: cast_launch<S3K_BF16, S3K_F32>(src, dst, n, hw, st); break;
	case S3K_BF16 * 8 + S3K_F16: cast_launch<S3K_BF16, S3K_F16>(src, dst, n, hw, st); break;
	default: return (int)hipErrorInvalidValue;
	}
	return (int)hipGetLastError();
}

extern "C" int s3k_bias_add(int kind, const void *x, const void *bias, void *out,
			    long long rows, int n, void *stream)
{
	hipStream_t st = (hipStream_t)stream;
	const long long tot = rows * n;
	if (tot <= 0)
		return 0;
	if (kind == S3K_F32)
		hipLaunchKernelGGL(bias_add_k<0>, grid1(tot), dim3(256), 0, st, x, bias, out, rows, n);
	else if (kind == S3K_F16)
		hipLaunchKernelGGL(bias_add_k<1>, grid1(tot), dim3(256), 0, st, x, bias, out, rows, n);
	else if (kind == S3K_BF16)
		hipLaunchKernelGGL(bias_add_k<2>, grid1(tot), dim3(256), 0, st, x, bias, out, rows, n);
	else
		return (int)hipErrorInvalidValue;
	return (int)hipGetLastError();
}

extern "C" int s3k_add_same(int kind, const void *x, const void *y, void *out, long long n,
			    void *stream)
{
	hipStream_t st = (hipStream_t)stream;
	if (n <= 0)
		return 0;
	if (kind == S3K_F32)
		hipLaunchKernelGGL(add_same_k<0>, grid1(n), dim3(256), 0, st, x, y, out, n);
	else if (kind == S3K_F16)
		hipLaunchKernelGGL(add_same_k<1>, grid1(n), dim3(256), 0, st, x, y, out, n);
	else if (kind == S3K_BF16)
		hipLaunchKernelGGL(add_same_k<2>, grid1(n), dim3(256), 0, st, x, y, out, n);
	else
		return (int)hipErrorInvalidValue;
	return (int)hipGetLastError();
}

extern "C" int s3k_gelu(int kind, const void *x, void *out, long long n, void *stream)
{
	hipStream_t st = (hipStream_t)stream;
	if (n <= 0)
		return 0;
	if (kind == S3K_F32)
		hipLaunchKernelGGL(gelu_k<0>, grid1(n), dim3(256), 0, st, x, out, n);
	else if (kind == S3K_F16)
		hipLaunchKernelGGL(gelu_k<1>, grid1(n), dim3(256), 0, st, x, out, n);
	else if (kind == S3K_BF16)
		hipLaunchKernelGGL(gelu_k<2>, grid1(n), dim3(256), 0, st, x, out, n);
	else
		return (int)hipErrorInvalidValue;
	return (int)hipGetLastError();
}

extern "C" int s3k_transpose2d(int esize, const void *src, void *dst, int batch, int rows,
			       int cols, void *stream)
{
	hipStream_t st = (hipStream_t)stream;
	if (rows <= 0 || cols <= 0 || batch <= 0)
		return 0;
	dim3 grid((cols + 31) / 32, (rows + 31) / 32, batch);
	if (esize == 4)
		hipLaunchKernelGGL(transpose_k<uint32_t>, grid, dim3(256), 0, st,
				   (const uint32_t *)src, (uint32_t *)dst, rows, cols);
	else if (esize == 2)
		hipLaunchKernelGGL(transpose_k<uint16_t>, grid, dim3(256), 0, st,
				   (const uint16_t *)src, (uint16_t *)dst, rows, cols);
	else if (esize == 1)
		hipLaunchKernelGGL(transpose_k<uint8_t>, grid, dim3(256), 0, st,
				   (const uint8_t *)src, (uint8_t *)dst, rows, cols);
	else
		return (int)hipErrorInvalidValue;
	return (int)hipGetLastError();
}
