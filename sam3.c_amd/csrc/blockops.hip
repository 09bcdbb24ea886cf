/*
 * blockops.hip - the non-matmul ops of a ViT block on gfx950, so that a
 * block's activations stay in HBM between its matmuls and attention:
 *
 *   - LayerNorm over the last dim (src/backend/cpu/kernels/cpu_layernorm.c:
 *     28-55, 198-254; bf16/f16 twins cpu_layernorm_bf16.c:88-115 and
 *     cpu_layernorm_f16.c:99-127): one wave per row, the row held in
 *     registers, mean and variance by wave reductions in f32 (a different
 *     summation order from the reference's left-to-right loop), then
 *     (x - mean) * inv_std, * gamma, + beta with one rounding each, as
 *     there.
 *   - RoPE on interleaved pairs (cpu_rope.c:88-104, cpu_rope_bf16.c:100-121,
 *     cpu_rope_f16.c:100-121): one lane per pair, y0 = x0*c - x1*s and
 *     y1 = x0*s + x1*c with each product rounded (no contraction), which is
 *     bit-identical to the reference's f32 arithmetic.
 *   - Permutation of up to 4 axes (cpu_transpose.c:313-387): one lane per
 *     output element, or per 16/8/4-byte chunk of it when the last axis
 *     stays last.
 */
#include "gemm_common.h"

namespace s3k {

template <int DT>
__device__ __forceinline__ float bo_ld(const void *p, long long i)
{
	if constexpr (DT == S3K_F32)
		return ((const float *)p)[i];
	else if constexpr (DT == S3K_BF16)
		return bf16_to_f32(((const uint16_t *)p)[i]);
	else
		return f16_to_f32(((const uint16_t *)p)[i]);
}

template <int DT>
__device__ __forceinline__ void bo_st(void *p, long long i, float v)
{
	if constexpr (DT == S3K_F32)
		((float *)p)[i] = v;
	else if constexpr (DT == S3K_BF16)
		((uint16_t *)p)[i] = (uint16_t)f32_to_bf16(v);
	else
		((uint16_t *)p)[i] = (uint16_t)f32_to_f16(v);
}

__device__ __forceinline__ float bo_wave_sum(float v)
{
	return wave_xor_sum(v);
}

/* One wave per row; element j of the row is held by lane j % 64 in slot
 * j / 64 (EPL slots cover cols <= 64 * EPL). EPL = 0: rows of any length,
 * re-read from memory in each pass. */
/* Output row map of a LayerNorm (g 0: identity): row m is stored at
 * ((a*d2 + c)*d1 + b)*g + m % g, m / g = (a*d1 + b)*d2 + c, i.e. the
 * permute (0,2,1,3) of [., d1, d2, g*cols] applied to the output (the
 * ViT window partition written by the LN that precedes it). */
struct LnMap {
	int g, d1, d2;
	unsigned *ovf;    /* S3K_LN_F16: range flag, tag stored when a row's  */
	unsigned tag;     /* largest |y| is >= 2^15 or below 2^-10 (nonzero)  */
};

/* The f16 operand's range check of one row (rmax: the wave's largest
 * finite |y|, every lane holding it): a row the f16 copy cannot hold to
 * f16 precision stores the tag. */
__device__ __forceinline__ void ln_range_flag(const LnMap &rm, float rmax, int lane)
{
	if (rm.ovf && lane == 0 && (rmax >= 32768.0f || (rmax > 0.0f && rmax < 0x1p-10f)))
		*rm.ovf = rm.tag;
}

__device__ __forceinline__ float bo_finite_abs(float x)
{
	const float a = __builtin_fabsf(x);
	return a <= 3.402823466e38f ? a : 0.0f;
}

__device__ __forceinline__ long long ln_out_row(const LnMap &rm, long long m)
{
	if (!rm.g)
		return m;
	const long long gi = m / rm.g, w = m - gi * rm.g;
	const long long c = gi % rm.d2, t = gi / rm.d2;
	const long long b = t % rm.d1, a = t / rm.d1;
	return ((a * rm.d2 + c) * rm.d1 + b) * rm.g + w;
}

template <int DT, int EPL, int OUTF>
__global__ void __launch_bounds__(256) layernorm_k(const void *x, const void *gamma,
						   const void *beta, void *out, int rows, int cols,
						   LnMap rm)
{
	static_assert(OUTF == S3K_LN_SAME || DT == S3K_F32, "operand formats are made from f32");
	const int lane = threadIdx.x & 63;
	const long long row = (long long)blockIdx.x * 4 + (threadIdx.x >> 6);
	if (row >= rows)
		return;
	const long long base = row * cols;
	const long long orow = ln_out_row(rm, row), obase = orow * cols;
	constexpr int N = EPL > 0 ? EPL : 1;
	float v[N];
	float sum = 0.0f;
	if constexpr (EPL > 0) {
#pragma unroll
		for (int i = 0; i < EPL; ++i) {
			const int j = lane + 64 * i;
			v[i] = j < cols ? bo_ld<DT>(x, base + j) : 0.0f;
			sum += v[i];
		}
	} else {
		for (int j = lane; j < cols; j += 64)
			sum += bo_ld<DT>(x, base + j);
	}
	const float mean = bo_wave_sum(sum) / (float)cols;
	float var = 0.0f;
	if constexpr (EPL > 0) {
#pragma unroll
		for (int i = 0; i < EPL; ++i) {
			const float d = sub_rn(v[i], mean);
			if (lane + 64 * i < cols)
				var = fmaf(d, d, var);
		}
	} else {
		for (int j = lane; j < cols; j += 64) {
			const float d = sub_rn(bo_ld<DT>(x, base + j), mean);
			var = fmaf(d, d, var);
		}
	}
	const float inv_std = 1.0f / sqrtf(bo_wave_sum(var) / (float)cols + 1e-5f);
	float ymax = 0.0f;
	auto finish = [&](int j, float xj) {
		float val = mul_rn(sub_rn(xj, mean), inv_std);
		if (gamma)
			val = mul_rn(val, bo_ld<DT>(gamma, j));
		if (beta)
			val = add_rn(val, bo_ld<DT>(beta, j));
		if constexpr (OUTF == S3K_LN_F16)
			ymax = fmaxf(ymax, bo_finite_abs(val));
		if constexpr (OUTF == S3K_LN_SAME) {
			bo_st<DT>(out, obase + j, val);
		} else if constexpr (OUTF == S3K_LN_PLANES) {
			uint32_t hi, lo;
			split_bf16x2(val, 0.0f, hi, lo);
			uint16_t *d = (uint16_t *)out + orow * 3LL * cols + j;
			d[0] = (uint16_t)hi;
			d[cols] = (uint16_t)lo;
			d[2LL * cols] = (uint16_t)hi;
		} else {
			((uint16_t *)out)[obase + j] = (uint16_t)f32_to_f16(val);
		}
	};
	if constexpr (EPL > 0) {
#pragma unroll
		for (int i = 0; i < EPL; ++i) {
			const int j = lane + 64 * i;
			if (j < cols)
				finish(j, v[i]);
		}
	} else {
		for (int j = lane; j < cols; j += 64)
			finish(j, bo_ld<DT>(x, base + j));
	}
	if constexpr (OUTF == S3K_LN_F16)
		ln_range_flag(rm, wave_max_f32(ymax), lane);
}

/* 16 bytes of a row as f32: 4 f32 or 8 bf16/f16 values. */
template <int DT>
__device__ __forceinline__ void bo_ld16(const void *p, long long i, float *v)
{
	if constexpr (DT == S3K_F32) {
		const float4 a = *(const float4 *)((const float *)p + i);
		v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
	} else {
		const uint4 a = *(const uint4 *)((const uint16_t *)p + i);
		const uint32_t w[4] = {a.x, a.y, a.z, a.w};
#pragma unroll
		for (int e = 0; e < 4; ++e) {
			v[2 * e] = DT == S3K_BF16 ? bf16_to_f32(w[e] & 0xFFFFu) : f16_to_f32(w[e] & 0xFFFFu);
			v[2 * e + 1] = DT == S3K_BF16 ? bf16_to_f32(w[e] >> 16) : f16_to_f32(w[e] >> 16);
		}
	}
}

template <int DT>
__device__ __forceinline__ void bo_st16(void *p, long long i, const float *v)
{
	if constexpr (DT == S3K_F32) {
		*(float4 *)((float *)p + i) = make_float4(v[0], v[1], v[2], v[3]);
	} else {
		uint32_t h[8];
#pragma unroll
		for (int e = 0; e < 8; ++e)
			h[e] = DT == S3K_BF16 ? f32_to_bf16(v[e]) : f32_to_f16(v[e]);
		*(uint4 *)((uint16_t *)p + i) = make_uint4(h[0] | (h[1] << 16), h[2] | (h[3] << 16),
							   h[4] | (h[5] << 16), h[6] | (h[7] << 16));
	}
}

/* The same LayerNorm with 16-byte accesses: rows of cols = SLOTS * 64 * VEC
 * elements, lane l holding elements (64 s + l) * VEC .. + VEC - 1 of each
 * slot s; the sums are taken in the same per-lane-then-wave order. */
template <int DT, int SLOTS, int OUTF>
__global__ void __launch_bounds__(256) layernorm_v(const void *x, const void *gamma,
						   const void *beta, void *out, int rows, int cols,
						   LnMap rm)
{
	static_assert(OUTF == S3K_LN_SAME || DT == S3K_F32, "operand formats are made from f32");
	constexpr int VEC = DT == S3K_F32 ? 4 : 8;
	const int lane = threadIdx.x & 63;
	const long long row = (long long)blockIdx.x * 4 + (threadIdx.x >> 6);
	if (row >= rows)
		return;
	const long long base = row * cols;
	const long long orow = ln_out_row(rm, row), obase = orow * cols;
	float v[SLOTS][VEC];
	float sum = 0.0f;
#pragma unroll
	for (int i = 0; i < SLOTS; ++i) {
		bo_ld16<DT>(x, base + (long long)(i * 64 + lane) * VEC, v[i]);
#pragma unroll
		for (int e = 0; e < VEC; ++e)
			sum += v[i][e];
	}
	const float mean = bo_wave_sum(sum) / (float)cols;
	float var = 0.0f;
#pragma unroll
	for (int i = 0; i < SLOTS; ++i)
#pragma unroll
		for (int e = 0; e < VEC; ++e) {
			const float d = sub_rn(v[i][e], mean);
			var = fmaf(d, d, var);
		}
	const float inv_std = 1.0f / sqrtf(bo_wave_sum(var) / (float)cols + 1e-5f);
	float ymax = 0.0f;
#pragma unroll
	for (int i = 0; i < SLOTS; ++i) {
		const int j0 = (i * 64 + lane) * VEC;
		float g[VEC], b[VEC];
		if (gamma)
			bo_ld16<DT>(gamma, j0, g);
		if (beta)
			bo_ld16<DT>(beta, j0, b);
#pragma unroll
		for (int e = 0; e < VEC; ++e) {
			float val = mul_rn(sub_rn(v[i][e], mean), inv_std);
			if (gamma)
				val = mul_rn(val, g[e]);
			if (beta)
				val = add_rn(val, b[e]);
			v[i][e] = val;
			if constexpr (OUTF == S3K_LN_F16)
				ymax = fmaxf(ymax, bo_finite_abs(val));
		}
		if constexpr (OUTF == S3K_LN_SAME) {
			bo_st16<DT>(out, obase + j0, v[i]);
		} else if constexpr (OUTF == S3K_LN_PLANES) {
			uint32_t hi[2], lo[2];
			split_bf16x2(v[i][0], v[i][1], hi[0], lo[0]);
			split_bf16x2(v[i][2], v[i][3], hi[1], lo[1]);
			uint16_t *d = (uint16_t *)out + orow * 3LL * cols + j0;
			*(uint2 *)d = make_uint2(hi[0], hi[1]);
			*(uint2 *)(d + cols) = make_uint2(lo[0], lo[1]);
			*(uint2 *)(d + 2LL * cols) = make_uint2(hi[0], hi[1]);
		} else {
			*(uint2 *)((uint16_t *)out + obase + j0) =
				make_uint2(pack_f16x2(v[i][0], v[i][1]), pack_f16x2(v[i][2], v[i][3]));
		}
	}
	if constexpr (OUTF == S3K_LN_F16)
		ln_range_flag(rm, wave_max_f32(ymax), lane);
}

/* pair p covers elements 2p, 2p+1 of x; its position s and frequency d
 * index the [seq, half] tables */
template <int DT>
__global__ void __launch_bounds__(256) rope_k(const void *x, const float *cos_t,
					      const float *sin_t, void *out, long long pairs,
					      int seq, int heads, int half)
{
	const long long p = (long long)blockIdx.x * 256 + threadIdx.x;
	if (p >= pairs)
		return;
	const int d = (int)(p % half);
	const long long rest = p / half;
	const int s = (int)((rest / heads) % seq);
	const float c = cos_t[(long long)s * half + d], sn = sin_t[(long long)s * half + d];
	const float x0 = bo_ld<DT>(x, 2 * p), x1 = bo_ld<DT>(x, 2 * p + 1);
	bo_st<DT>(out, 2 * p, sub_rn(mul_rn(x0, c), mul_rn(x1, sn)));
	bo_st<DT>(out, 2 * p + 1, add_rn(mul_rn(x0, sn), mul_rn(x1, c)));
}

/* Head-split operands of attention straight from the fused qkv
 * projection: x holds rows of `pitch` f32 values; element (b, s, h, d)
 * of the [B, S, H, D] view of operand y is
 * x[(b*S + s)*pitch + col0[y] + h*D + d]. The output is [B, H, S, D]
 * (permute 0,2,1,3). With RoPE it is applied on the way exactly as
 * rope_k does it (pair (d, d+1), cos/sin [S, D/2], products and sums
 * rounded separately). Four values per thread. Up to three operands
 * from the same qkv rows in one launch (blockIdx.y picks the operand):
 * out[y] takes columns col0[y] onward, with RoPE when bit y of rope_mask
 * is set. */
struct Split3Args {
	const float *x;
	long long pitch;
	long long col0[3];
	float *out[3];
	const float *cos_t, *sin_t;
	int rope_mask;
	int B, S, H, D;
};

__global__ void __launch_bounds__(256) rope_split3_k(Split3Args a)
{
	const int y = blockIdx.y;
	const long long q = (long long)blockIdx.x * 256 + threadIdx.x;
	const int D4 = a.D / 4;
	if (q >= (long long)a.B * a.S * a.H * D4)
		return;
	const int d = (int)(q % D4) * 4;
	long long r = q / D4;
	const int h = (int)(r % a.H);
	r /= a.H;
	const int s = (int)(r % a.S);
	const int b = (int)(r / a.S);
	float4 v = *(const float4 *)(a.x + ((long long)b * a.S + s) * a.pitch + a.col0[y] +
				     (long long)h * a.D + d);
	if ((a.rope_mask >> y) & 1) {
		const int half = a.D / 2;
		const long long t = (long long)s * half + d / 2;
		const float c0 = a.cos_t[t], s0 = a.sin_t[t], c1 = a.cos_t[t + 1], s1 = a.sin_t[t + 1];
		const float4 u = v;
		v.x = sub_rn(mul_rn(u.x, c0), mul_rn(u.y, s0));
		v.y = add_rn(mul_rn(u.x, s0), mul_rn(u.y, c0));
		v.z = sub_rn(mul_rn(u.z, c1), mul_rn(u.w, s1));
		v.w = add_rn(mul_rn(u.z, s1), mul_rn(u.w, c1));
	}
	*(float4 *)(a.out[y] + (((long long)b * a.H + h) * a.S + s) * a.D + d) = v;
}

struct PermArgs {
	const char *src;
	char *dst;
	unsigned od1, od2, od3;          /* output dims 1..3 (dim 0 implied) */
	long long st0, st1, st2, st3;    /* input stride (elements) of output axis k */
	long long total;
	unsigned *ovf;                   /* f16 operand range flag (or NULL) */
	unsigned tag;
};

/* I: index type, 32-bit when the element count allows it */
template <typename T, typename I>
__global__ void __launch_bounds__(256) permute_k(PermArgs a)
{
	const I stride = (I)gridDim.x * 256, total = (I)a.total;
	const I od1 = a.od1, od2 = a.od2, od3 = a.od3;
	for (I i = (I)blockIdx.x * 256 + threadIdx.x; i < total; i += stride) {
		I t = i;
		const I o3 = t % od3;
		t /= od3;
		const I o2 = t % od2;
		t /= od2;
		const I o1 = t % od1;
		const I o0 = t / od1;
		const long long src = (long long)o0 * a.st0 + (long long)o1 * a.st1 +
				      (long long)o2 * a.st2 + (long long)o3 * a.st3;
		((T *)a.dst)[i] = ((const T *)a.src)[src];
	}
}

/* f32 permute whose last axis stays last, written as a GEMM operand: the
 * output, read as rows of K values, becomes bf16 planes [hi|lo|hi] with
 * row pitch 3K (PLANES) or f16 (else), the split / cast a GEMM applies
 * to f32 A. One thread per 4 values (one 16-byte source chunk). */
template <bool PLANES, typename I>
__global__ void __launch_bounds__(256) permute_op_k(PermArgs a, unsigned K)
{
	const I stride = (I)gridDim.x * 256, total = (I)a.total;
	const I od1 = a.od1, od2 = a.od2, od3 = a.od3;
	for (I i = (I)blockIdx.x * 256 + threadIdx.x; i < total; i += stride) {
		I t = i;
		const I o3 = t % od3;
		t /= od3;
		const I o2 = t % od2;
		t /= od2;
		const I o1 = t % od1;
		const I o0 = t / od1;
		const long long src = (long long)o0 * a.st0 + (long long)o1 * a.st1 +
				      (long long)o2 * a.st2 + (long long)o3 * a.st3;
		const float4 v = ((const float4 *)a.src)[src];
		const long long e = (long long)i * 4;
		if (PLANES) {
			uint32_t hi[2], lo[2];
			split_bf16x2(v.x, v.y, hi[0], lo[0]);
			split_bf16x2(v.z, v.w, hi[1], lo[1]);
			uint16_t *d = (uint16_t *)a.dst + (e / K) * 3LL * K + e % K;
			*(uint2 *)d = make_uint2(hi[0], hi[1]);
			*(uint2 *)(d + K) = make_uint2(lo[0], lo[1]);
			*(uint2 *)(d + 2LL * K) = make_uint2(hi[0], hi[1]);
		} else {
			/* a value past 2^15, or four nonzero values all below 2^-10:
			 * the f16 copy would not hold them to f16 precision */
			const float ax = __builtin_fabsf(v.x), ay = __builtin_fabsf(v.y);
			const float az = __builtin_fabsf(v.z), aw = __builtin_fabsf(v.w);
			const float mx = fmaxf(fmaxf(ax, ay), fmaxf(az, aw));
			const bool big = (ax >= 32768.0f && ax <= 3.402823466e38f) ||
					 (ay >= 32768.0f && ay <= 3.402823466e38f) ||
					 (az >= 32768.0f && az <= 3.402823466e38f) ||
					 (aw >= 32768.0f && aw <= 3.402823466e38f);
			if (a.ovf && (big || (mx > 0.0f && mx < 0x1p-10f)))
				*a.ovf = a.tag;
			*(uint2 *)((uint16_t *)a.dst + e) = make_uint2(pack_f16x2(v.x, v.y), pack_f16x2(v.z, v.w));
		}
	}
}

template <typename T>
static void launch_perm(const PermArgs &a, dim3 grid, hipStream_t st)
{
	if (a.total + (long long)grid.x * 256 < (1LL << 32))
		hipLaunchKernelGGL((permute_k<T, unsigned>), grid, dim3(256), 0, st, a);
	else
		hipLaunchKernelGGL((permute_k<T, long long>), grid, dim3(256), 0, st, a);
}

template <int DT, int OUTF>
static void launch_ln(const void *x, const void *g, const void *b, void *o, int rows, int cols,
		      hipStream_t st, LnMap rm = LnMap{0, 0, 0, nullptr, 0})
{
	const dim3 grid((unsigned)((rows + 3) / 4)), block(256);
	constexpr int VEC = DT == S3K_F32 ? 4 : 8;
	const bool vec = cols % (64 * VEC) == 0 && cols / (64 * VEC) <= 8 &&
			 !(((uintptr_t)x | (uintptr_t)g | (uintptr_t)b | (uintptr_t)o) & 15u);
	if (vec) {
		switch (cols / (64 * VEC)) {
		case 1: hipLaunchKernelGGL((layernorm_v<DT, 1, OUTF>), grid, block, 0, st, x, g, b, o, rows, cols, rm); return;
		case 2: hipLaunchKernelGGL((layernorm_v<DT, 2, OUTF>), grid, block, 0, st, x, g, b, o, rows, cols, rm); return;
		case 3: hipLaunchKernelGGL((layernorm_v<DT, 3, OUTF>), grid, block, 0, st, x, g, b, o, rows, cols, rm); return;
		case 4: hipLaunchKernelGGL((layernorm_v<DT, 4, OUTF>), grid, block, 0, st, x, g, b, o, rows, cols, rm); return;
		case 6: hipLaunchKernelGGL((layernorm_v<DT, 6, OUTF>), grid, block, 0, st, x, g, b, o, rows, cols, rm); return;
		case 8: hipLaunchKernelGGL((layernorm_v<DT, 8, OUTF>), grid, block, 0, st, x, g, b, o, rows, cols, rm); return;
		default: break;
		}
	}
	if (cols <= 256)
		hipLaunchKernelGGL((layernorm_k<DT, 4, OUTF>), grid, block, 0, st, x, g, b, o, rows, cols, rm);
	else if (cols <= 512)
		hipLaunchKernelGGL((layernorm_k<DT, 8, OUTF>), grid, block, 0, st, x, g, b, o, rows, cols, rm);
	else if (cols <= 1024)
		hipLaunchKernelGGL((layernorm_k<DT, 16, OUTF>), grid, block, 0, st, x, g, b, o, rows, cols, rm);
	else if (cols <= 2048)
		hipLaunchKernelGGL((layernorm_k<DT, 32, OUTF>), grid, block, 0, st, x, g, b, o, rows, cols, rm);
	else
		hipLaunchKernelGGL((layernorm_k<DT, 0, OUTF>), grid, block, 0, st, x, g, b, o, rows, cols, rm);
}

} /* namespace s3k */

using namespace s3k;

extern "C" int s3k_layernorm(int kind, const void *x, const void *gamma, const void *beta,
			     void *out, long long rows, int cols, void *stream)
{
	if (rows < 0 || cols <= 0 || rows > 0x7FFFFFFFLL)
		return (int)hipErrorInvalidValue;
	if (rows == 0)
		return (int)hipSuccess;
	const hipStream_t st = (hipStream_t)stream;
	if (kind == S3K_F32)
		launch_ln<S3K_F32, S3K_LN_SAME>(x, gamma, beta, out, (int)rows, cols, st);
	else if (kind == S3K_BF16)
		launch_ln<S3K_BF16, S3K_LN_SAME>(x, gamma, beta, out, (int)rows, cols, st);
	else if (kind == S3K_F16)
		launch_ln<S3K_F16, S3K_LN_SAME>(x, gamma, beta, out, (int)rows, cols, st);
	else
		return (int)hipErrorInvalidValue;
	return (int)hipGetLastError();
}

extern "C" int s3k_layernorm_to_map(int fmt, const float *x, const float *gamma,
				    const float *beta, void *out, long long rows, int cols, int rm_g,
				    int rm_d1, int rm_d2, unsigned *ovf, unsigned ovf_tag, void *stream)
{
	if (rows < 0 || cols <= 0 || rows > 0x7FFFFFFFLL || (fmt == S3K_LN_PLANES && cols % 8))
		return (int)hipErrorInvalidValue;
	if (rm_g && (rm_g < 0 || rm_d1 <= 0 || rm_d2 <= 0 || rows % ((long long)rm_g * rm_d1 * rm_d2)))
		return (int)hipErrorInvalidValue;
	if (rows == 0)
		return (int)hipSuccess;
	const hipStream_t st = (hipStream_t)stream;
	const LnMap rm{rm_g, rm_d1, rm_d2, fmt == S3K_LN_F16 ? ovf : nullptr, ovf_tag};
	if (fmt == S3K_LN_PLANES)
		launch_ln<S3K_F32, S3K_LN_PLANES>(x, gamma, beta, out, (int)rows, cols, st, rm);
	else if (fmt == S3K_LN_F16)
		launch_ln<S3K_F32, S3K_LN_F16>(x, gamma, beta, out, (int)rows, cols, st, rm);
	else
		return (int)hipErrorInvalidValue;
	return (int)hipGetLastError();
}

extern "C" int s3k_layernorm_to(int fmt, const float *x, const float *gamma, const float *beta,
				void *out, long long rows, int cols, unsigned *ovf, unsigned ovf_tag,
				void *stream)
{
	return s3k_layernorm_to_map(fmt, x, gamma, beta, out, rows, cols, 0, 0, 0, ovf, ovf_tag,
				    stream);
}

extern "C" int s3k_rope(int kind, const void *x, const float *cos_t, const float *sin_t,
			void *out, int batch, int seq, int heads, int hd, void *stream)
{
	if (batch < 0 || seq < 0 || heads < 0 || hd <= 0 || (hd & 1))
		return (int)hipErrorInvalidValue;
	const long long pairs = (long long)batch * seq * heads * (hd / 2);
	if (pairs == 0)
		return (int)hipSuccess;
	const hipStream_t st = (hipStream_t)stream;
	const dim3 grid((unsigned)((pairs + 255) / 256)), block(256);
	if (kind == S3K_F32)
		hipLaunchKernelGGL(rope_k<S3K_F32>, grid, block, 0, st, x, cos_t, sin_t, out, pairs,
				   seq, heads, hd / 2);
	else if (kind == S3K_BF16)
		hipLaunchKernelGGL(rope_k<S3K_BF16>, grid, block, 0, st, x, cos_t, sin_t, out, pairs,
				   seq, heads, hd / 2);
	else if (kind == S3K_F16)
		hipLaunchKernelGGL(rope_k<S3K_F16>, grid, block, 0, st, x, cos_t, sin_t, out, pairs,
				   seq, heads, hd / 2);
	else
		return (int)hipErrorInvalidValue;
	return (int)hipGetLastError();
}

extern "C" int s3k_rope_split3(const float *x, long long pitch, const long long *col0,
			       const float *cos_t, const float *sin_t, int rope_mask, float *const *out,
			       int n_out, int B, int S, int H, int D, void *stream)
{
	if (n_out < 1 || n_out > 3 || B < 0 || S < 0 || H < 0 || D <= 0 || D % 4 || pitch % 4 ||
	    (rope_mask && (!cos_t || !sin_t)) || (rope_mask >> n_out) || (((uintptr_t)x) & 15u))
		return (int)hipErrorInvalidValue;
	Split3Args a;
	a.x = x;
	a.pitch = pitch;
	for (int y = 0; y < 3; ++y) {
		const int k = y < n_out ? y : 0;
		if (col0[k] % 4 || col0[k] < 0 || col0[k] + (long long)H * D > pitch || !out[k] ||
		    ((uintptr_t)out[k] & 15u))
			return (int)hipErrorInvalidValue;
		a.col0[y] = col0[k];
		a.out[y] = out[k];
	}
	a.cos_t = cos_t;
	a.sin_t = sin_t;
	a.rope_mask = rope_mask;
	a.B = B;
	a.S = S;
	a.H = H;
	a.D = D;
	const long long n = (long long)B * S * H * (D / 4);
	if (n == 0)
		return (int)hipSuccess;
	hipLaunchKernelGGL(rope_split3_k, dim3((unsigned)((n + 255) / 256), (unsigned)n_out), dim3(256),
			   0, (hipStream_t)stream, a);
	return (int)hipGetLastError();
}

/* dst = src permuted: output axis k is input axis axes[k]; ndim <= 4,
 * esize bytes per element. */
extern "C" int s3k_permute_to(int fmt, const float *src, void *dst, int ndim, const int *in_dims,
			      const int *axes, int K, unsigned *ovf, unsigned ovf_tag, void *stream)
{
	if (ndim < 1 || ndim > 4 || K <= 0 || K % 4 || (fmt != S3K_LN_PLANES && fmt != S3K_LN_F16) ||
	    axes[ndim - 1] != ndim - 1 || in_dims[ndim - 1] % 4 ||
	    (((uintptr_t)src | (uintptr_t)dst) & 15u))
		return (int)hipErrorInvalidValue;
	long long d[4] = {1, 1, 1, 1};
	int ax[4] = {0, 1, 2, 3};
	const int pad = 4 - ndim;
	int seen = 0;
	for (int k = 0; k < ndim; ++k) {
		if (in_dims[k] < 0 || axes[k] < 0 || axes[k] >= ndim || (seen >> axes[k]) & 1)
			return (int)hipErrorInvalidValue;
		seen |= 1 << axes[k];
		d[pad + k] = in_dims[k];
		ax[pad + k] = pad + axes[k];
	}
	d[3] /= 4; /* 16-byte chunks of 4 values */
	const long long ist[4] = {d[1] * d[2] * d[3], d[2] * d[3], d[3], 1};
	PermArgs a;
	a.src = (const char *)src;
	a.dst = (char *)dst;
	a.od1 = (unsigned)d[ax[1]];
	a.od2 = (unsigned)d[ax[2]];
	a.od3 = (unsigned)d[ax[3]];
	a.st0 = ist[ax[0]];
	a.st1 = ist[ax[1]];
	a.st2 = ist[ax[2]];
	a.st3 = ist[ax[3]];
	a.total = d[0] * d[1] * d[2] * d[3];
	a.ovf = fmt == S3K_LN_F16 ? ovf : nullptr;
	a.tag = ovf_tag;
	if (a.total == 0 || a.od1 == 0 || a.od2 == 0 || a.od3 == 0)
		return (int)hipSuccess;
	const long long blocks = (a.total + 255) / 256;
	const dim3 grid((unsigned)(blocks < 65536 ? blocks : 65536)), block(256);
	const hipStream_t st = (hipStream_t)stream;
	const bool small = a.total * 4 + (long long)grid.x * 256 * 4 < (1LL << 32);
	if (fmt == S3K_LN_PLANES) {
		if (small)
			hipLaunchKernelGGL((permute_op_k<true, unsigned>), grid, block, 0, st, a, (unsigned)K);
		else
			hipLaunchKernelGGL((permute_op_k<true, long long>), grid, block, 0, st, a, (unsigned)K);
	} else {
		if (small)
			hipLaunchKernelGGL((permute_op_k<false, unsigned>), grid, block, 0, st, a, (unsigned)K);
		else
			hipLaunchKernelGGL((permute_op_k<false, long long>), grid, block, 0, st, a, (unsigned)K);
	}
	return (int)hipGetLastError();
}

extern "C" int s3k_permute(int esize, const void *src, void *dst, int ndim, const int *in_dims,
			   const int *axes, void *stream)
{
	if (ndim < 1 || ndim > 4 || esize <= 0)
		return (int)hipErrorInvalidValue;
	/* pad to 4 axes with leading size-1 axes */
	long long d[4] = {1, 1, 1, 1};
	int ax[4] = {0, 1, 2, 3};
	const int pad = 4 - ndim;
	int seen = 0;
	for (int k = 0; k < ndim; ++k) {
		if (in_dims[k] < 0 || axes[k] < 0 || axes[k] >= ndim || (seen >> axes[k]) & 1)
			return (int)hipErrorInvalidValue;
		seen |= 1 << axes[k];
		d[pad + k] = in_dims[k];
		ax[pad + k] = pad + axes[k];
	}
	long long es = esize;
	/* the last axis stays last: move it in chunks of up to 16 bytes */
	if (ax[3] == 3) {
		long long row = d[3] * es;
		long long chunk = 1;
		for (long long c = 16; c > 1; c >>= 1)
			if (c <= row && row % c == 0 && ((uintptr_t)src % c) == 0 && ((uintptr_t)dst % c) == 0) {
				chunk = c;
				break;
			}
		if (chunk > 1 && chunk >= es) {
			d[3] = row / chunk;
			es = chunk;
		}
	}
	const long long ist[4] = {d[1] * d[2] * d[3], d[2] * d[3], d[3], 1};
	PermArgs a;
	a.src = (const char *)src;
	a.dst = (char *)dst;
	a.od1 = (unsigned)d[ax[1]];
	a.od2 = (unsigned)d[ax[2]];
	a.od3 = (unsigned)d[ax[3]];
	a.st0 = ist[ax[0]];
	a.st1 = ist[ax[1]];
	a.st2 = ist[ax[2]];
	a.st3 = ist[ax[3]];
	a.total = d[0] * d[1] * d[2] * d[3];
	if (a.total == 0)
		return (int)hipSuccess;
	if (a.od1 == 0 || a.od2 == 0 || a.od3 == 0)
		return (int)hipSuccess;
	const hipStream_t st = (hipStream_t)stream;
	const long long blocks = (a.total + 255) / 256;
	const dim3 grid((unsigned)(blocks < 65536 ? blocks : 65536)), block(256);
	(void)block;
	switch (es) {
	case 1:  launch_perm<uint8_t>(a, grid, st); break;
	case 2:  launch_perm<uint16_t>(a, grid, st); break;
	case 4:  launch_perm<uint32_t>(a, grid, st); break;
	case 8:  launch_perm<uint2>(a, grid, st); break;
	case 16: launch_perm<uint4>(a, grid, st); break;
	default: return (int)hipErrorInvalidValue;
	}
	return (int)hipGetLastError();
}
