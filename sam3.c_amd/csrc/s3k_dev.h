/*
 * s3k_dev.h - device-side helpers shared by the gfx950 kernels.
 *
 * Conversions follow the rounding the reference CPU path uses
 * (src/core/half.h:58-210 of sam3.c): f32 -> bf16 and f32 -> f16 round
 * to nearest even; a NaN converted to bf16 stays a quiet NaN. The GELU
 * is the tanh form of the reference CPU kernel (cpu_gelu.c:23-38).
 */
#ifndef SAM3_S3K_DEV_H
#define SAM3_S3K_DEV_H

#include <hip/hip_runtime.h>
#include <stdint.h>

typedef __attribute__((ext_vector_type(8))) __bf16 s3k_bf16x8;
typedef __attribute__((ext_vector_type(8))) _Float16 s3k_f16x8;
typedef __attribute__((ext_vector_type(16))) float s3k_f32x16;
typedef __attribute__((ext_vector_type(4))) float s3k_f32x4;
typedef __attribute__((ext_vector_type(4))) unsigned s3k_u32x4;

namespace s3k {

/* One rounded f32 multiply / add that the compiler may not fuse into an
 * FMA (clang's __fmul_rn/__fadd_rn are plain, contractable operators). */
__device__ __forceinline__ float mul_rn(float a, float b)
{
#pragma clang fp contract(off)
	return a * b;
}

__device__ __forceinline__ float add_rn(float a, float b)
{
#pragma clang fp contract(off)
	return a + b;
}

__device__ __forceinline__ float sub_rn(float a, float b)
{
#pragma clang fp contract(off)
	return a - b;
}

/* Largest v over the 64 lanes of the wave. */
__device__ __forceinline__ float wave_max_f32(float v)
{
#pragma unroll
	for (int off = 32; off > 0; off >>= 1)
		v = fmaxf(v, __shfl_xor(v, off));
	return v;
}

/* 2^e as a float, -126 <= e <= 127 */
__device__ __forceinline__ float pow2f(int e)
{
	return __uint_as_float((uint32_t)(e + 127) << 23);
}

/* Sum over the wave as the xor butterfly computes it: v += v[lane ^ off]
 * for off = 32, 16, 8, 4, 2, 1, so every lane ends with the same value
 * (each step adds the same two operands on both lanes of a pair). The
 * partner values come from v_permlane32_swap (32), ds_swizzle in its
 * xor mode (16, 8, 4) and DPP quad permutes (2, 1) instead of
 * ds_bpermute: the same sums, fewer LDS-pipe round trips. */
__device__ __forceinline__ float wave_xor_sum(float v)
{
	{
		const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v),
								 false, false);
		v = __uint_as_float(r[0]) + __uint_as_float(r[1]);
	}
	v += __int_as_float(__builtin_amdgcn_ds_swizzle(__float_as_int(v), 0x401F)); /* ^16 */
	v += __int_as_float(__builtin_amdgcn_ds_swizzle(__float_as_int(v), 0x201F)); /* ^8  */
	v += __int_as_float(__builtin_amdgcn_ds_swizzle(__float_as_int(v), 0x101F)); /* ^4  */
	v += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x4E, 0xF, 0xF, true)); /* ^2 */
	v += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0xB1, 0xF, 0xF, true)); /* ^1 */
	return v;
}

/* |x| for the row scale; inf and NaN count as 0 (they do not set it) */
__device__ __forceinline__ float finite_abs(float x)
{
	const float a = __builtin_fabsf(x);
	return a <= 3.402823466e38f ? a : 0.0f;
}

/* The exponent e of the power-of-two factor of an f16 copy of a row
 * whose largest finite |value| is amax (already reduced over the row):
 * 0 when amax lies in [2^-10, 2^15) or is 0, else the e that puts amax
 * in [2^14, 2^15), clamped to [-100, 113]. The row is stored as
 * f16(x * 2^-e) and the product scaled back by 2^e. */
__device__ __forceinline__ int scale_exp_of(float amax)
{
	if (amax == 0.0f || (amax >= 0x1p-10f && amax < 0x1p15f))
		return 0;
	int e = (int)((__float_as_uint(amax) >> 23) & 0xFFu) - 127 - 14;
	return e < -100 ? -100 : e > 113 ? 113 : e;
}

/* The exponent e of the weight-row factor 2^e of a Q8_0 weight row
 * whose values |q*scale| are at most m (inf and NaN counted as 0): 0
 * when m lies in [2^-6, 2^15) or is 0, else the e that brings m into
 * [2^14, 2^15), clamped to [-100, 113]. For a row of whole blocks m is
 * 127 * its largest |scale|, so at e = 0 that scale, at least 2^-6 / 127,
 * is an f16 normal (2^-14 and up), and so is every nonzero q times it.
 * The row's weights go to f16 as f16(q * scale * 2^-e); output column n
 * is multiplied by 2^e in the f32 epilogue. */
__device__ __forceinline__ int wscale_exp_of(float m)
{
	if (!(m > 0.0f) || m > 3.402823466e38f || (m >= 0x1p-6f && m < 0x1p15f))
		return 0;
	int e = (int)((__float_as_uint(m) >> 23) & 0xFFu) - 127 - 14;
	return e < -100 ? -100 : e > 113 ? 113 : e;
}

/* 1 / f for f = 2^e, -126 <= e <= 126 (exact) */
__device__ __forceinline__ float inv_pow2(float f)
{
	return __uint_as_float((254u - ((__float_as_uint(f) >> 23) & 0xFFu)) << 23);
}

/* scale_exp_of the largest amax over the wave */
__device__ __forceinline__ int row_scale_exp(float amax)
{
	return scale_exp_of(wave_max_f32(amax));
}

__device__ __forceinline__ float bf16_to_f32(uint32_t b)
{
	return __uint_as_float(b << 16);
}

/* Round to nearest even; NaN -> quiet NaN with the sign kept. */
__device__ __forceinline__ uint32_t f32_to_bf16(float f)
{
	uint32_t u = __float_as_uint(f);
	if ((u & 0x7F800000u) == 0x7F800000u && (u & 0x7FFFFFu))
		return ((u >> 16) | 0x40u) & 0xFFFFu;
	u += 0x7FFFu + ((u >> 16) & 1u);
	return u >> 16;
}

__device__ __forceinline__ float f16_to_f32(uint32_t h)
{
	return (float)__builtin_bit_cast(_Float16, (uint16_t)h);
}

/* Hardware conversion: round to nearest even, f16 subnormals kept. */
__device__ __forceinline__ uint32_t f32_to_f16(float f)
{
	return (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)f);
}

/* IEEE binary16 <-> binary32 by integer arithmetic, bit-exact with
 * sam3.c's scalar converters (src/core/half.h:58-161): RNE (for f16
 * subnormals after the reference's truncating pre-shift); f32 NaN -> f16
 * keeps the top mantissa bits and sets bit 0;
 * f16 NaN -> f32 keeps the payload as is (no quieting). The hardware
 * conversions (f32_to_f16 / f16_to_f32 above) agree on every finite
 * value and infinity; NaN payloads may differ. */
__device__ __forceinline__ uint32_t f32_to_f16_sw(float f)
{
	const uint32_t u = __float_as_uint(f);
	const uint32_t sign = (u >> 16) & 0x8000u;
	const uint32_t e8 = (u >> 23) & 0xFFu;
	uint32_t m = u & 0x7FFFFFu;
	if (e8 == 0xFFu)
		return sign | 0x7C00u | (m ? (m >> 13) | 1u : 0u);
	const int e = (int)e8 - 112; /* f16 biased exponent */
	if (e >= 31)
		return sign | 0x7C00u;
	if (e <= 0) {
		if (e < -10)
			return sign;
		/* subnormal: the mantissa with its leading one is first shifted
		 * down by 1 - e (those bits are dropped, as the reference does),
		 * then rounded to nearest even on its low 13 bits */
		m = (m | 0x800000u) >> (1 - e);
	}
	const uint32_t rest = m & 0x1FFFu;
	uint32_t q = m >> 13;
	if (rest > 0x1000u || (rest == 0x1000u && (q & 1u)))
		++q;
	/* a carry out of the mantissa moves into the exponent (and from the
	 * largest finite value to infinity) by itself */
	return sign | (e > 0 ? (((uint32_t)e << 10) + q) : q);
}

__device__ __forceinline__ float f16_to_f32_sw(uint32_t h)
{
	const uint32_t sign = (h & 0x8000u) << 16;
	const uint32_t e = (h >> 10) & 0x1Fu, m = h & 0x3FFu;
	if (e == 0x1Fu)
		return __uint_as_float(sign | 0x7F800000u | (m << 13));
	if (e)
		return __uint_as_float(sign | ((e + 112u) << 23) | (m << 13));
	if (!m)
		return __uint_as_float(sign);
	/* subnormal: m * 2^-24, normalized by the leading one's position */
	const int lz = __builtin_clz(m) - 21; /* shifts that bring its top bit to bit 10 */
	return __uint_as_float(sign | ((uint32_t)(113 - lz) << 23) | (((m << lz) & 0x3FFu) << 13));
}

__device__ __forceinline__ float round_bf16(float f)
{
	return bf16_to_f32(f32_to_bf16(f));
}

/* The same rounding by the hardware conversion (v_cvt_pk_bf16_f32, round
 * to nearest even) for the epilogue's intermediate roundings; NaN stays a
 * NaN. Defined after pack_bf16x2. */
__device__ __forceinline__ float round_bf16_hw(float f);

__device__ __forceinline__ float round_f16(float f)
{
	return (float)(_Float16)f;
}

/* The reference's GELU, 0.5*x*(1 + tanh(u)) with
 * u = 0.7978845608*(x + 0.044715*x^3) (cpu_gelu.c:30-38), evaluated as
 * x / (1 + exp(-2u)), the same function (0.5*(1 + tanh(u)) is the
 * logistic of 2u), with the hardware exp2 and reciprocal:
 * 2u*log2(e) = x*(a + b*x^2), a = 2*0.7978845608*log2(e), b = 0.044715*a.
 * Five VALU operations and two transcendentals; relative error near 1e-7.
 * exp2 overflows to +inf for large negative x, giving x * 0 = -0, the
 * reference's limit; for large positive x it gives x. */
__device__ __forceinline__ float gelu_tanh(float x)
{
	const float p = fmaf(0.10294324f, x * x, 2.3022082f);
	const float e = __builtin_amdgcn_exp2f(-(x * p));
	return x * __builtin_amdgcn_rcpf(1.0f + e);
}

typedef __bf16 s3k_bf16x2 __attribute__((ext_vector_type(2)));
typedef float s3k_f32x2 __attribute__((ext_vector_type(2)));

/* Pack two f32 as two bf16 (RNE, NaN stays NaN) in one dword, lo first:
 * one v_cvt_pk_bf16_f32 on gfx950. */
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi)
{
	const s3k_f32x2 v = {lo, hi};
	return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, s3k_bf16x2));
}

/* Two f32 split into bf16 hi = bf16(x) and lo = bf16(x - hi), each pair
 * packed lo element first: the operand planes of the split f32 GEMM. */
__device__ __forceinline__ void split_bf16x2(float a, float b, uint32_t &hi, uint32_t &lo)
{
	hi = pack_bf16x2(a, b);
	lo = pack_bf16x2(a - __uint_as_float(hi << 16), b - __uint_as_float(hi & 0xFFFF0000u));
}

__device__ __forceinline__ float round_bf16_hw(float f)
{
	return __uint_as_float(pack_bf16x2(f, 0.0f) << 16);
}

/* Pack two f32 as two f16 (RNE) in one dword, lo first. */
__device__ __forceinline__ uint32_t pack_f16x2(float lo, float hi)
{
	return f32_to_f16(lo) | (f32_to_f16(hi) << 16);
}

/* Four signed bytes of w, each times s, as four f16 in two dwords. The
 * product q*s is formed in f32 (exact rounding of the true product) and
 * rounded once to f16. */
__device__ __forceinline__ uint2 dequant4_f16(uint32_t w, float s)
{
	float f0 = (float)(int)(int8_t)(w & 0xFFu);
	float f1 = (float)(int)(int8_t)((w >> 8) & 0xFFu);
	float f2 = (float)(int)(int8_t)((w >> 16) & 0xFFu);
	float f3 = (float)(int)(int8_t)(w >> 24);
	uint2 r;
	r.x = pack_f16x2(f0 * s, f1 * s);
	r.y = pack_f16x2(f2 * s, f3 * s);
	return r;
}

/* Output epilogue with the reference's rounding points: the matmul
 * result, the bias add and the GELU each round to the output type, as
 * MATMUL -> ADD -> GELU nodes do on the CPU backend. */
template <int CK>
__device__ __forceinline__ float epilogue(float acc, float bias, int flags)
{
	float v = acc;
	if (CK == 2) { /* BF16 */
		v = round_bf16_hw(v);
		if (flags & 1)
			v = round_bf16_hw(add_rn(v, bias));
		if (flags & 2)
			v = round_bf16_hw(gelu_tanh(v));
	} else if (CK == 1) { /* F16 */
		v = round_f16(v);
		if (flags & 1)
			v = round_f16(add_rn(v, bias));
		if (flags & 2)
			v = round_f16(gelu_tanh(v));
	} else {
		if (flags & 1)
			v = add_rn(v, bias);
		if (flags & 2)
			v = gelu_tanh(v);
	}
	return v;
}

__device__ __forceinline__ float load_as_f32(const void *p, long long i, int kind)
{
	if (kind == 0)
		return ((const float *)p)[i];
	uint32_t h = ((const uint16_t *)p)[i];
	return kind == 2 ? bf16_to_f32(h) : f16_to_f32(h);
}

__device__ __forceinline__ void store_from_f32(void *p, long long i, int kind, float v)
{
	if (kind == 0)
		((float *)p)[i] = v;
	else if (kind == 2)
		((uint16_t *)p)[i] = (uint16_t)f32_to_bf16(v);
	else
		((uint16_t *)p)[i] = (uint16_t)f32_to_f16(v);
}

} /* namespace s3k */

#endif /* SAM3_S3K_DEV_H */
