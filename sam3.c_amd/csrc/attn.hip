/*
 * attn.hip - fused scaled dot-product attention (flash-attention forward)
 * for gfx950: out = softmax(Q K^T / sqrt(D) + mask) V per head, without
 * materializing the [Sq, Sk] score matrix. Replaces cpu_kernel_sdpa
 * (src/backend/cpu/kernels/cpu_sdpa.c:216-288), whose per-row online
 * softmax (sdpa_row_f32, :49-159) this follows one 64-key tile at a time.
 *
 * Layout: Q [BH, Sq, D], K and V [BH, Sk, D], out [BH, Sq, D], all of one
 * dtype (f32, bf16 or f16); the optional additive mask is f32 [Sq, Sk],
 * shared by all heads (cpu_sdpa.c:193-196).
 *
 * attn_fwd (D = 64, 16-byte aligned tensors): a workgroup (4 waves) owns
 * 128 queries of one head; wave w owns 32. The scores are computed
 * transposed, S^T = K Q^T, with v_mfma_f32_32x32x16: a lane then holds one
 * query (lane & 31) and 32 of the tile's 64 keys, so the row max and row
 * sum are in-lane reductions plus one exchange with lane ^ 32. The output
 * is accumulated transposed too, O^T = V^T P^T: the P^T operand is exactly
 * the lane's own probabilities (the MFMA's k index is permuted the same
 * way for both operands, which leaves the product unchanged), and the
 * per-query rescale exp(m_old - m_new) is a per-lane scalar.
 *   - bf16/f16: K tiles arrive in LDS by direct-to-LDS loads
 *     (XOR-swizzled rows); V tiles are staged through registers and
 *     written transposed, V^T [D][64 keys], row pitch 136 bytes;
 *   - f32: every operand is split into two bf16 planes, x = hi + lo with
 *     hi = bf16(x), lo = bf16(x - hi), and each product is formed as
 *     hi*hi + lo*hi + hi*lo (the dropped lo*lo term is below 2^-16 of the
 *     product), so f32 inputs keep about 16 significant bits per product at
 *     three bf16 MFMAs per tile step. K and V are split while they are
 *     staged into LDS through registers;
 *   - keys past Sk get a -inf score, queries past Sq are not stored;
 *   - scores are scaled into base 2 (exp2 = v_exp_f32).
 *
 * attn_generic: any D up to 512 and any element alignment, one wave per
 * query row, f32 arithmetic with expf: the path for the reference's other
 * head sizes (the mask decoder's 32, the prompt encoder's 16).
 */
#include "gemm_common.h"
#include "lds_dma.h"

namespace s3k {

struct AttnArgs {
	const char *q, *k, *v;
	const float *mask;
	char *out;
	int Sq, Sk;
	long long hq, hk;       /* per-head strides, elements */
	float scale_log2;       /* log2(e) / sqrt(D) */
	unsigned k_extent;      /* bytes of one head's K (16-bit inputs) */
};

constexpr int AT_D = 64, AT_BQ = 128, AT_BKV = 64;
constexpr int AT_VT_PITCH = AT_BKV * 2 + 8;          /* bytes per V^T row */
constexpr int AT_K_BYTES = AT_BKV * AT_D * 2;        /* 8 KiB per plane */
constexpr int AT_VT_BYTES = AT_D * AT_VT_PITCH;      /* 8.5 KiB per plane */

template <int DT>
struct AtCfg {
	static constexpr bool SPLIT = DT == S3K_F32;
	static constexpr int NPL = SPLIT ? 2 : 1;        /* bf16 planes */
	static constexpr int VT_OFF = NPL * AT_K_BYTES;
	static constexpr int STAGE = NPL * (AT_K_BYTES + AT_VT_BYTES);
	static constexpr int FAM = DT == S3K_F16 ? FAM_F16 : FAM_BF16;
};

template <int DT>
__device__ __forceinline__ uint32_t at_pack2(float lo, float hi)
{
	if constexpr (DT == S3K_F16)
		return pack_f16x2(lo, hi);
	else
		return pack_bf16x2(lo, hi);
}

/* hi/lo bf16 planes of two f32 values, one dword each */
__device__ __forceinline__ void at_split2(float a, float b, uint32_t &hi, uint32_t &lo)
{
	hi = pack_bf16x2(a, b);
	lo = pack_bf16x2(a - __uint_as_float(hi << 16), b - __uint_as_float(hi & 0xFFFF0000u));
}

__device__ __forceinline__ void at_split8(const float4 &x, const float4 &y, uint4 &hi, uint4 &lo)
{
	at_split2(x.x, x.y, hi.x, lo.x);
	at_split2(x.z, x.w, hi.y, lo.y);
	at_split2(y.x, y.y, hi.z, lo.z);
	at_split2(y.z, y.w, hi.w, lo.w);
}

template <int DT>
__global__ void __launch_bounds__(256, 2) attn_fwd(AttnArgs p)
{
	using C = AtCfg<DT>;
	__shared__ __attribute__((aligned(1024))) char smem[2 * C::STAGE];
	const int lane = threadIdx.x & 63;
	const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
	const int h = lane >> 5, l32 = lane & 31;
	const long long head = blockIdx.y;
	const int q = blockIdx.x * AT_BQ + wave * 32 + l32;   /* this lane's query */
	const unsigned lds0 = lds_addr_of(smem);

	/* Q^T operand: query row q, d chunk 16c + 8h (hi and lo planes for f32) */
	uint4 qh[4], ql[4];
#pragma unroll
	for (int c = 0; c < 4; ++c) {
		qh[c] = ql[c] = make_uint4(0, 0, 0, 0);
		if (q < p.Sq) {
			if constexpr (C::SPLIT) {
				const float *Q = (const float *)p.q + head * p.hq + (long long)q * AT_D + 16 * c + 8 * h;
				at_split8(*(const float4 *)Q, *(const float4 *)(Q + 4), qh[c], ql[c]);
			} else {
				const uint16_t *Q = (const uint16_t *)p.q + head * p.hq;
				qh[c] = *(const uint4 *)(Q + (long long)q * AT_D + 16 * c + 8 * h);
			}
		}
	}

	/* 16-bit K tile loads: 8 KiB = 8 instructions, 2 per wave; slot s of
	 * load j holds row s/8, chunk (s%8) ^ swz(row) */
	const s3k_i32x4 rk = buf_rsrc(p.k + head * p.hk * 2, p.k_extent);
	unsigned k_off[2];
#pragma unroll
	for (int t = 0; t < 2; ++t) {
		const int s = (t * 4 + wave) * 64 + lane;
		const int row = s / 8, c = (s % 8) ^ lds_swz<8>(row);
		k_off[t] = (unsigned)(row * AT_D * 2 + c * 16);
	}
	auto issue_k = [&](int kt) {
		const unsigned st = lds0 + (unsigned)((kt & 1) * C::STAGE);
		const int rows_left = p.Sk - kt * AT_BKV;
#pragma unroll
		for (int t = 0; t < 2; ++t) {
			const int row = ((t * 4 + wave) * 64 + lane) / 8;
			const unsigned o = row < rows_left ? k_off[t] : S3K_OOB;
			dma16s(st + (t * 4 + wave) * 1024, rk, o, (unsigned)(kt * AT_BKV * AT_D * 2));
		}
	};

	/* f32 K tile: thread t stages row t/4, d 16*(t%4)..+15 */
	const int kr0 = threadIdx.x >> 2, kd0 = 16 * (threadIdx.x & 3);
	/* V tile: thread t stages keys 4*(t/16)..+3, d 4*(t%16)..+3 */
	const int vk0 = 4 * (threadIdx.x >> 4), vd0 = 4 * (threadIdx.x & 15);

	/* registers carrying tile kt+1 from global memory to LDS */
	uint2 vr[4];
	float4 vf[4], kf[4];
	auto load_tile = [&](int kt) {
		if constexpr (C::SPLIT) {
			const float *K = (const float *)p.k + head * p.hk;
			const float *V = (const float *)p.v + head * p.hk;
			const int krow = kt * AT_BKV + kr0;
#pragma unroll
			for (int i = 0; i < 4; ++i)
				kf[i] = krow < p.Sk ? *(const float4 *)(K + (long long)krow * AT_D + kd0 + 4 * i)
						    : make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
			for (int i = 0; i < 4; ++i) {
				const int key = kt * AT_BKV + vk0 + i;
				vf[i] = key < p.Sk ? *(const float4 *)(V + (long long)key * AT_D + vd0)
						   : make_float4(0.f, 0.f, 0.f, 0.f);
			}
		} else {
			const uint16_t *V = (const uint16_t *)p.v + head * p.hk;
#pragma unroll
			for (int i = 0; i < 4; ++i) {
				const int key = kt * AT_BKV + vk0 + i;
				vr[i] = key < p.Sk ? *(const uint2 *)(V + (long long)key * AT_D + vd0)
						   : make_uint2(0, 0);
			}
		}
	};
	auto store_tile = [&](int kt) {
		char *st = smem + (kt & 1) * C::STAGE;
		char *vt = st + C::VT_OFF;
		if constexpr (C::SPLIT) {
			/* K hi/lo planes: logical chunks kd0/8 and kd0/8 + 1 of row kr0 */
#pragma unroll
			for (int u = 0; u < 2; ++u) {
				uint4 hi, lo;
				at_split8(kf[2 * u], kf[2 * u + 1], hi, lo);
				const int off = (kr0 * 8 + ((kd0 / 8 + u) ^ lds_swz<8>(kr0))) << 4;
				*(uint4 *)(st + off) = hi;
				*(uint4 *)(st + AT_K_BYTES + off) = lo;
			}
			/* V^T hi/lo planes: row d = vd0 + j holds keys vk0..vk0+3 */
			const float e[4][4] = {{vf[0].x, vf[1].x, vf[2].x, vf[3].x},
					       {vf[0].y, vf[1].y, vf[2].y, vf[3].y},
					       {vf[0].z, vf[1].z, vf[2].z, vf[3].z},
					       {vf[0].w, vf[1].w, vf[2].w, vf[3].w}};
#pragma unroll
			for (int j = 0; j < 4; ++j) {
				uint32_t h0, l0, h1, l1;
				at_split2(e[j][0], e[j][1], h0, l0);
				at_split2(e[j][2], e[j][3], h1, l1);
				const int off = (vd0 + j) * AT_VT_PITCH + vk0 * 2;
				*(uint2 *)(vt + off) = make_uint2(h0, h1);
				*(uint2 *)(vt + AT_VT_BYTES + off) = make_uint2(l0, l1);
			}
		} else {
			/* 4x4 transpose of 16-bit values: row j of the result is d vd0+j */
#pragma unroll
			for (int j = 0; j < 4; ++j) {
				const int sh = (j & 1) * 16;
				uint32_t e[4];
#pragma unroll
				for (int i = 0; i < 4; ++i)
					e[i] = ((j < 2 ? vr[i].x : vr[i].y) >> sh) & 0xFFFFu;
				*(uint2 *)(vt + (vd0 + j) * AT_VT_PITCH + vk0 * 2) =
					make_uint2(e[0] | (e[1] << 16), e[2] | (e[3] << 16));
			}
		}
	};

	s3k_f32x16 o[2];
#pragma unroll
	for (int md = 0; md < 2; ++md)
#pragma unroll
		for (int r = 0; r < 16; ++r)
			o[md][r] = 0.0f;
	float m_run = -3.402823466e38f, l_run = 0.0f;

	const int nkt = (p.Sk + AT_BKV - 1) / AT_BKV;
	if constexpr (!C::SPLIT)
		issue_k(0);
	load_tile(0);
	store_tile(0);

	for (int kt = 0; kt < nkt; ++kt) {
		const bool more = kt + 1 < nkt;
		/* K(kt) landed and V^T(kt) stored; every wave is past tile kt-1,
		 * whose slots are refilled below */
		wait_vm<0>();
		__syncthreads();
		if (more) {
			if constexpr (!C::SPLIT)
				issue_k(kt + 1);
			load_tile(kt + 1);
		}

		const char *Ks = smem + (kt & 1) * C::STAGE;
		const char *Vt = Ks + C::VT_OFF;

		/* S^T = K Q^T for keys 32*mb + (row), this lane's query */
		s3k_f32x16 s[2];
#pragma unroll
		for (int mb = 0; mb < 2; ++mb) {
#pragma unroll
			for (int r = 0; r < 16; ++r)
				s[mb][r] = 0.0f;
			const int row = 32 * mb + l32;
#pragma unroll
			for (int c = 0; c < 4; ++c) {
				const int off = (row * 8 + ((2 * c + h) ^ lds_swz<8>(row))) << 4;
				const uint4 kh = *(const uint4 *)(Ks + off);
				if constexpr (C::SPLIT) {
					const uint4 kl = *(const uint4 *)(Ks + AT_K_BYTES + off);
					mfma_chunk<C::FAM>(s[mb], kl, qh[c]);
					mfma_chunk<C::FAM>(s[mb], kh, ql[c]);
				}
				mfma_chunk<C::FAM>(s[mb], kh, qh[c]);
			}
		}

		/* scale into base 2, mask, -inf past Sk; running max */
		float mt = -3.402823466e38f;
		const int kbase = kt * AT_BKV;
#pragma unroll
		for (int mb = 0; mb < 2; ++mb)
#pragma unroll
			for (int g = 0; g < 4; ++g) {
				const int key0 = kbase + 32 * mb + 8 * g + 4 * h;
				float4 mk = make_float4(0.f, 0.f, 0.f, 0.f);
				if (p.mask && q < p.Sq) {
					const float *mrow = p.mask + (long long)q * p.Sk;
					if (key0 + 4 <= p.Sk && (p.Sk & 3) == 0 && ((uintptr_t)p.mask & 15u) == 0)
						mk = *(const float4 *)(mrow + key0);
					else {
						mk.x = key0 < p.Sk ? mrow[key0] : 0.f;
						mk.y = key0 + 1 < p.Sk ? mrow[key0 + 1] : 0.f;
						mk.z = key0 + 2 < p.Sk ? mrow[key0 + 2] : 0.f;
						mk.w = key0 + 3 < p.Sk ? mrow[key0 + 3] : 0.f;
					}
				}
				const float mv[4] = {mk.x, mk.y, mk.z, mk.w};
#pragma unroll
				for (int e = 0; e < 4; ++e) {
					float v = s[mb][4 * g + e] * p.scale_log2 + mv[e] * 1.44269504088896341f;
					if (key0 + e >= p.Sk)
						v = -__builtin_inff();
					s[mb][4 * g + e] = v;
					mt = fmaxf(mt, v);
				}
			}
		mt = fmaxf(mt, __shfl_xor(mt, 32));
		const float m_new = fmaxf(m_run, mt);
		const float alpha = __builtin_amdgcn_exp2f(m_run - m_new);
		m_run = m_new;

		/* probabilities, packed as the P^T operand of each 16-key chunk */
		uint4 ph[4], pl[4];
		float lsum = 0.0f;
#pragma unroll
		for (int mb = 0; mb < 2; ++mb)
#pragma unroll
			for (int sub = 0; sub < 2; ++sub) {
				float pv[8];
#pragma unroll
				for (int e = 0; e < 8; ++e) {
					pv[e] = __builtin_amdgcn_exp2f(s[mb][8 * sub + e] - m_new);
					lsum += pv[e];
				}
				const int cc = 2 * mb + sub;
				if constexpr (C::SPLIT) {
					at_split8(make_float4(pv[0], pv[1], pv[2], pv[3]),
						  make_float4(pv[4], pv[5], pv[6], pv[7]), ph[cc], pl[cc]);
				} else {
					ph[cc] = make_uint4(at_pack2<DT>(pv[0], pv[1]), at_pack2<DT>(pv[2], pv[3]),
							    at_pack2<DT>(pv[4], pv[5]), at_pack2<DT>(pv[6], pv[7]));
				}
			}
		l_run = l_run * alpha + lsum;
#pragma unroll
		for (int md = 0; md < 2; ++md)
#pragma unroll
			for (int r = 0; r < 16; ++r)
				o[md][r] *= alpha;

		/* O^T += V^T P^T: A = V^T rows d, keys in the same permuted order */
#pragma unroll
		for (int md = 0; md < 2; ++md) {
			const char *vrow = Vt + (32 * md + l32) * AT_VT_PITCH;
#pragma unroll
			for (int cc = 0; cc < 4; ++cc) {
				const int key = 16 * cc + 4 * h;   /* = 32*mb + 16*sub + 4h */
				const uint2 lo = *(const uint2 *)(vrow + key * 2);
				const uint2 hi = *(const uint2 *)(vrow + (key + 8) * 2);
				const uint4 vh = make_uint4(lo.x, lo.y, hi.x, hi.y);
				if constexpr (C::SPLIT) {
					const uint2 llo = *(const uint2 *)(vrow + AT_VT_BYTES + key * 2);
					const uint2 lhi = *(const uint2 *)(vrow + AT_VT_BYTES + (key + 8) * 2);
					mfma_chunk<C::FAM>(o[md], make_uint4(llo.x, llo.y, lhi.x, lhi.y), ph[cc]);
					mfma_chunk<C::FAM>(o[md], vh, pl[cc]);
				}
				mfma_chunk<C::FAM>(o[md], vh, ph[cc]);
			}
		}

		if (more)
			store_tile(kt + 1);
	}

	/* normalize (a query with no finite score keeps zeros, as the
	 * reference's row_sum > 0 test leaves it) and store out[q][d] */
	const float l_tot = l_run + __shfl_xor(l_run, 32);
	const float inv = l_tot > 0.0f ? 1.0f / l_tot : 0.0f;
	if (q < p.Sq) {
#pragma unroll
		for (int md = 0; md < 2; ++md)
#pragma unroll
			for (int g = 0; g < 4; ++g) {
				const int d0 = 32 * md + 8 * g + 4 * h;
				const float x0 = o[md][4 * g] * inv, x1 = o[md][4 * g + 1] * inv;
				const float x2 = o[md][4 * g + 2] * inv, x3 = o[md][4 * g + 3] * inv;
				if constexpr (C::SPLIT) {
					float *O = (float *)p.out + head * p.hq + (long long)q * AT_D;
					*(float4 *)(O + d0) = make_float4(x0, x1, x2, x3);
				} else {
					uint16_t *O = (uint16_t *)p.out + head * p.hq + (long long)q * AT_D;
					*(uint2 *)(O + d0) = make_uint2(at_pack2<DT>(x0, x1), at_pack2<DT>(x2, x3));
				}
			}
	}
}

/* ------------------------------------------------------------------ */
/* Any head size: one wave per query row                                */
/* ------------------------------------------------------------------ */
struct AttnGArgs {
	const char *q, *k, *v;
	const float *mask;
	char *out;
	int BH, Sq, Sk, D;
	float scale;
};

template <int DT>
__device__ __forceinline__ float at_ld(const char *base, long long i)
{
	if constexpr (DT == S3K_F32)
		return ((const float *)base)[i];
	else if constexpr (DT == S3K_BF16)
		return bf16_to_f32(((const uint16_t *)base)[i]);
	else
		return f16_to_f32(((const uint16_t *)base)[i]);
}

template <int DT>
__device__ __forceinline__ void at_st(char *base, long long i, float v)
{
	if constexpr (DT == S3K_F32)
		((float *)base)[i] = v;
	else if constexpr (DT == S3K_BF16)
		((uint16_t *)base)[i] = (uint16_t)f32_to_bf16(v);
	else
		((uint16_t *)base)[i] = (uint16_t)f32_to_f16(v);
}

template <int DT, int NACC>
__global__ void __launch_bounds__(256) attn_generic(AttnGArgs p)
{
	__shared__ float qs[4][NACC * 64];
	__shared__ float ps[4][64];
	const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
	const long long rows = (long long)p.BH * p.Sq;
	long long row = (long long)blockIdx.x * 4 + wave;
	/* every wave runs the same tiles (the barriers are block-wide); a
	 * wave past the last row recomputes it and stores nothing */
	const bool live = row < rows;
	if (!live)
		row = rows - 1;
	const long long head = row / p.Sq;
	const int qi = (int)(row - head * p.Sq);
	const long long kv0 = head * p.Sk * p.D;
	for (int d = lane; d < p.D; d += 64)
		qs[wave][d] = at_ld<DT>(p.q, row * p.D + d);
	__syncthreads();

	float acc[NACC];
#pragma unroll
	for (int i = 0; i < NACC; ++i)
		acc[i] = 0.0f;
	float m_run = -3.402823466e38f, l_run = 0.0f;
	const float *mrow = p.mask ? p.mask + (long long)qi * p.Sk : nullptr;

	for (int t = 0; t < p.Sk; t += 64) {
		const int key = t + lane;
		float s = -__builtin_inff();
		if (key < p.Sk) {
			const long long ko = kv0 + (long long)key * p.D;
			float dot = 0.0f;
			for (int d = 0; d < p.D; ++d)
				dot = fmaf(qs[wave][d], at_ld<DT>(p.k, ko + d), dot);
			s = dot * p.scale;
			if (mrow)
				s += mrow[key];
		}
		float mt = s;
#pragma unroll
		for (int off = 32; off; off >>= 1)
			mt = fmaxf(mt, __shfl_xor(mt, off));
		const float m_new = fmaxf(m_run, mt);
		const float alpha = expf(m_run - m_new);
		const float pj = expf(s - m_new);
		float ls = pj;
#pragma unroll
		for (int off = 32; off; off >>= 1)
			ls += __shfl_xor(ls, off);
		l_run = l_run * alpha + ls;
		m_run = m_new;
		ps[wave][lane] = pj;
		__syncthreads();
#pragma unroll
		for (int i = 0; i < NACC; ++i)
			acc[i] *= alpha;
		const int nk = min(64, p.Sk - t);
		for (int j = 0; j < nk; ++j) {
			const float w = ps[wave][j];
			const long long vo = kv0 + (long long)(t + j) * p.D;
#pragma unroll
			for (int i = 0; i < NACC; ++i) {
				const int d = lane + 64 * i;
				if (d < p.D)
					acc[i] = fmaf(w, at_ld<DT>(p.v, vo + d), acc[i]);
			}
		}
		__syncthreads();
	}
	if (live) {
		const float inv = l_run > 0.0f ? 1.0f / l_run : 0.0f;
#pragma unroll
		for (int i = 0; i < NACC; ++i) {
			const int d = lane + 64 * i;
			if (d < p.D)
				at_st<DT>(p.out, row * p.D + d, acc[i] * inv);
		}
	}
}

template <int DT>
static void launch_generic(const AttnGArgs &g, hipStream_t st)
{
	const long long rows = (long long)g.BH * g.Sq;
	const dim3 grid((unsigned)((rows + 3) / 4));
	if (g.D <= 64)
		hipLaunchKernelGGL((attn_generic<DT, 1>), grid, dim3(256), 0, st, g);
	else if (g.D <= 128)
		hipLaunchKernelGGL((attn_generic<DT, 2>), grid, dim3(256), 0, st, g);
	else if (g.D <= 256)
		hipLaunchKernelGGL((attn_generic<DT, 4>), grid, dim3(256), 0, st, g);
	else
		hipLaunchKernelGGL((attn_generic<DT, 8>), grid, dim3(256), 0, st, g);
}

} /* namespace s3k */

using namespace s3k;

static int attn_kind_ok(int kind)
{
	return kind == S3K_F32 || kind == S3K_BF16 || kind == S3K_F16;
}

/* Which kernel runs the problem: S3K_ATTN_MFMA, S3K_ATTN_GENERIC or 0. */
extern "C" int s3k_attn_path(int kind, const void *q, const void *k, const void *v, void *out,
			     int BH, int Sq, int Sk, int D)
{
	if (!attn_kind_ok(kind) || BH < 0 || Sq < 0 || Sk < 0 || D <= 0)
		return 0;
	const long long es = kind == S3K_F32 ? 4 : 2;
	if (((uintptr_t)q | (uintptr_t)k | (uintptr_t)v | (uintptr_t)out) & (uintptr_t)(es - 1))
		return 0;
	if (D == AT_D && BH >= 1 && BH <= 65535 && Sq >= 1 && Sk >= 1 &&
	    !(((uintptr_t)q | (uintptr_t)k | (uintptr_t)v | (uintptr_t)out) & 15u) &&
	    (long long)Sk * AT_D * es <= 0x7FFFFFF0LL)
		return S3K_ATTN_MFMA;
	if (D <= 512 && (long long)BH * Sq / 4 < 0x7FFFFFFFLL)
		return S3K_ATTN_GENERIC;
	return 0;
}

extern "C" int s3k_attn(int path, int kind, const void *q, const void *k, const void *v,
			const float *mask, void *out, int BH, int Sq, int Sk, int D, void *stream)
{
	const int best = s3k_attn_path(kind, q, k, v, out, BH, Sq, Sk, D);
	if (!best || (path == S3K_ATTN_MFMA && best != S3K_ATTN_MFMA) ||
	    (path != 0 && path != S3K_ATTN_MFMA && path != S3K_ATTN_GENERIC))
		return (int)hipErrorInvalidValue;
	if ((long long)BH * Sq == 0)
		return (int)hipSuccess;
	const hipStream_t st = (hipStream_t)stream;
	if (path == 0)
		path = best;
	if (path == S3K_ATTN_GENERIC) {
		AttnGArgs g;
		g.q = (const char *)q;
		g.k = (const char *)k;
		g.v = (const char *)v;
		g.mask = mask;
		g.out = (char *)out;
		g.BH = BH;
		g.Sq = Sq;
		g.Sk = Sk;
		g.D = D;
		g.scale = 1.0f / sqrtf((float)D);
		if (kind == S3K_F32)
			launch_generic<S3K_F32>(g, st);
		else if (kind == S3K_BF16)
			launch_generic<S3K_BF16>(g, st);
		else
			launch_generic<S3K_F16>(g, st);
		return (int)hipGetLastError();
	}
	AttnArgs p;
	p.q = (const char *)q;
	p.k = (const char *)k;
	p.v = (const char *)v;
	p.mask = mask;
	p.out = (char *)out;
	p.Sq = Sq;
	p.Sk = Sk;
	p.hq = (long long)Sq * D;
	p.hk = (long long)Sk * D;
	p.scale_log2 = 1.44269504088896341f / sqrtf((float)D);
	p.k_extent = (unsigned)((long long)Sk * D * 2);
	const dim3 grid((Sq + AT_BQ - 1) / AT_BQ, BH);
	if (kind == S3K_BF16)
		hipLaunchKernelGGL(attn_fwd<S3K_BF16>, grid, dim3(256), 0, st, p);
	else if (kind == S3K_F16)
		hipLaunchKernelGGL(attn_fwd<S3K_F16>, grid, dim3(256), 0, st, p);
	else
		hipLaunchKernelGGL(attn_fwd<S3K_F32>, grid, dim3(256), 0, st, p);
	return (int)hipGetLastError();
}
