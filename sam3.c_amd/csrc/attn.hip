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
	int BH, nqb;            /* heads, query blocks per head */
	int mask_vec;           /* mask rows 16-byte aligned: float4 loads */
	int oh;                 /* > 0: output head-merged (at_out_row)      */
	int ofmt;               /* merged f32 rows written as a GEMM operand:
				 * 0 f32, 1 bf16 planes [hi|lo|hi] (row pitch
				 * 3*oh*D), 2 f16 with the range flag        */
	unsigned *ovf;          /* ofmt 2: range flag (or NULL) and its tag  */
	unsigned ovf_tag;
};

/* Element offset of output row q of head hh: [BH, Sq, D] rows, or with
 * oh > 0 heads merged, hh = b*oh + h stored as row b*Sq + q, columns
 * h*D.. of [B*Sq, oh*D] (the permute (0,2,1,3) of [B, oh, Sq, D]). */
__device__ __forceinline__ long long at_out_row(int oh, long long hh, int Sq, int q, int D)
{
	if (oh <= 0)
		return (hh * Sq + q) * (long long)D;
	const long long b = hh / oh, h = hh - b * oh;
	return ((b * Sq + q) * oh + h) * (long long)D;
}

constexpr int AT_D = 64, AT_BKV = 64;
constexpr int AT_VT_PITCH = AT_BKV * 2 + 8;          /* bytes per V^T row */
constexpr int AT_K_BYTES = AT_BKV * AT_D * 2;        /* 8 KiB per plane */
constexpr int AT_VT_BYTES = AT_D * AT_VT_PITCH;      /* 8.5 KiB per plane */

/* VD: V tiles by direct-to-LDS loads, row-major [key][d], read as the
 * V^T operand with transposing LDS reads (16-bit inputs); else staged
 * through registers into a V^T tile */
template <int DT, int NW, bool VD = false>
struct AtCfg {
	static constexpr bool SPLIT = DT == S3K_F32;
	static constexpr int NPL = SPLIT ? 2 : 1;        /* bf16 planes */
	static constexpr int KS = NPL * AT_K_BYTES;      /* one K slot */
	static constexpr int VS = VD ? AT_K_BYTES : NPL * AT_VT_BYTES; /* one V slot */
	static constexpr int LDS = 2 * KS + 2 * VS;      /* two of each */
	static constexpr int FAM = DT == S3K_F16 ? FAM_F16 : FAM_BF16;
	static constexpr int BQ = 32 * NW;                /* queries per workgroup */
	static constexpr int KJ = (8 + NW - 1) / NW;      /* K loads per wave */
};

template <int DT>
__device__ __forceinline__ uint32_t at_pack2(float lo, float hi)
{
	if constexpr (DT == S3K_F16)
		return pack_f16x2(lo, hi);
	else
		return pack_bf16x2(lo, hi);
}

/* f32 sum of the two 16-bit values of w, added to acc (v_dot2 with 1, 1) */
template <int DT>
__device__ __forceinline__ float at_sum2(uint32_t w, float acc)
{
	if constexpr (DT == S3K_F16) {
		typedef _Float16 h2 __attribute__((ext_vector_type(2)));
		const h2 one = {(_Float16)1.0f, (_Float16)1.0f};
		return __builtin_amdgcn_fdot2(__builtin_bit_cast(h2, w), one, acc, false);
	} else {
		const s3k_bf16x2 one = {(__bf16)1.0f, (__bf16)1.0f};
		return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(s3k_bf16x2, w), one, acc, false);
	}
}

/* Chunk swizzle of a direct-to-LDS V tile row: it depends on the key's
 * low four bits only, so the transposed reads of the four 16-key chunks
 * of a tile differ by a constant offset. */
__device__ __forceinline__ int at_vswz(int key)
{
	const int r = key & 15;
	return (r ^ (r >> 3)) & 7;
}

typedef short at_v4i16 __attribute__((ext_vector_type(4)));

/* ds_read_b64_tr_b16: within each group of 16 lanes, lane i receives
 * element i % 4 of the 8 bytes addressed by lanes i / 4, 4 + i / 4,
 * 8 + i / 4 and 12 + i / 4 (measured on gfx950). */
__device__ __forceinline__ uint2 at_read_tr(const char *smem, unsigned off)
{
	const at_v4i16 r = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
		(__attribute__((address_space(3))) at_v4i16 *)((__attribute__((address_space(3))) char *)
								       smem + off));
	return __builtin_bit_cast(uint2, r);
}

/* x combined with the value of lane ^ 32 (v_permlane32_swap) */
__device__ __forceinline__ float at_max_pair(float x)
{
	const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
	return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}

__device__ __forceinline__ float at_sum_pair(float x)
{
	const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
	return __uint_as_float(r[0]) + __uint_as_float(r[1]);
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

/* workgroups per CU the registers are budgeted for, chosen so that no
 * variant spills: three (12 waves, 168 VGPRs) for the 16-bit kernel
 * without a mask, two for f32 or a mask, one for f32 with a mask (its
 * mask tile, score halves and hi/lo operand planes need 256+ VGPRs) */
template <int DT, int NW, bool MASK, bool VD = false>
constexpr int at_minb()
{
	return NW != 4 ? 1 : (DT == S3K_F32 && MASK) ? 1 : (DT == S3K_F32 || MASK) ? 2 : 3;
}

template <int N>
struct at_int {
	static constexpr int value = N;
};

/* The probabilities of a tile are formed against the running max m
 * without first taking the tile's max: they are only recomputed (after
 * moving m to the tile's max and rescaling the accumulators) when some
 * lane's 32 probabilities sum past 2^15, which also catches the first
 * tile (m = -FLT_MAX gives +inf). Every probability the MFMA sees is
 * then below 2^15, inside the f16 range. */
constexpr float AT_PSUM_MAX = 32768.0f;

template <int DT, int NW, bool MASK, bool VD>
__global__ void __launch_bounds__(64 * NW, (at_minb<DT, NW, MASK, VD>())) attn_fwd(AttnArgs p)
{
	using C = AtCfg<DT, NW, VD>;
	static_assert(!VD || !C::SPLIT, "V by direct-to-LDS loads for 16-bit inputs");
	__shared__ __attribute__((aligned(1024))) char smem[C::LDS];
	const int lane = threadIdx.x & 63;
	const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
	const int h = lane >> 5, l32 = lane & 31;

	/* workgroup -> (head, query block): workgroups are dispatched to the 8
	 * XCDs round-robin, so the nqb blocks of a head are given ids with
	 * one residue mod 8 and run on one XCD, whose L2 then serves the
	 * head's K and V to all of them (the heads past the last whole group
	 * of 8 are laid out plainly) */
	const unsigned L = blockIdx.x, nqb = (unsigned)p.nqb;
	const unsigned g8 = (unsigned)(p.BH / 8) * 8u * nqb;
	unsigned hh, qb;
	if (L < g8) {
		const unsigned sl = L >> 3;
		hh = sl / nqb * 8u + (L & 7u);
		qb = sl % nqb;
	} else {
		hh = (unsigned)(p.BH / 8) * 8u + (L - g8) / nqb;
		qb = (L - g8) % nqb;
	}
	const long long head = hh;
	const int q0w = (int)qb * C::BQ + wave * 32;         /* the wave's first query */
	const int q = q0w + l32;                             /* this lane's query */
	const bool wave_live = q0w < p.Sq;                   /* wave-uniform */
	const bool stager = wave < 4;                        /* threads 0..255 stage K, V */
	const unsigned lds0 = lds_addr_of(smem);
	constexpr int ES = C::SPLIT ? 4 : 2;                 /* input element bytes */

	/* Q^T operand, pre-multiplied by 1/sqrt(64) = 2^-3 (exact): query row
	 * q, d chunk 16c + 8h (hi and lo planes for f32) */
	uint4 qh[4], ql[4];
#pragma unroll
	for (int c = 0; c < 4; ++c) {
		qh[c] = ql[c] = make_uint4(0, 0, 0, 0);
		if (q < p.Sq) {
			if constexpr (C::SPLIT) {
				const float *Q = (const float *)p.q + head * p.hq + (long long)q * AT_D + 16 * c + 8 * h;
				float4 x = *(const float4 *)Q, y = *(const float4 *)(Q + 4);
				x.x *= 0.125f, x.y *= 0.125f, x.z *= 0.125f, x.w *= 0.125f;
				y.x *= 0.125f, y.y *= 0.125f, y.z *= 0.125f, y.w *= 0.125f;
				at_split8(x, y, qh[c], ql[c]);
			} else {
				const uint16_t *Q = (const uint16_t *)p.q + head * p.hq;
				const uint4 r = *(const uint4 *)(Q + (long long)q * AT_D + 16 * c + 8 * h);
				const uint32_t w[4] = {r.x, r.y, r.z, r.w};
				uint32_t o4[4];
#pragma unroll
				for (int i = 0; i < 4; ++i) {
					float lo, hi;
					if constexpr (DT == S3K_F16) {
						lo = f16_to_f32(w[i] & 0xFFFFu), hi = f16_to_f32(w[i] >> 16);
					} else {
						lo = bf16_to_f32(w[i] & 0xFFFFu), hi = bf16_to_f32(w[i] >> 16);
					}
					o4[i] = at_pack2<DT>(lo * 0.125f, hi * 0.125f);
				}
				qh[c] = make_uint4(o4[0], o4[1], o4[2], o4[3]);
			}
		}
	}

	/* the head's K and V as buffers: loads past Sk rows return zeros */
	const unsigned kv_bytes = (unsigned)((long long)p.Sk * AT_D * ES);
	const s3k_i32x4 rk = buf_rsrc(p.k + head * p.hk * ES, kv_bytes);
	const __amdgpu_buffer_rsrc_t bk = __builtin_amdgcn_make_buffer_rsrc(
		(void *)(p.k + head * p.hk * ES), (short)0, (int)kv_bytes, 0x00020000);
	const __amdgpu_buffer_rsrc_t bv = __builtin_amdgcn_make_buffer_rsrc(
		(void *)(p.v + head * p.hk * ES), (short)0, (int)kv_bytes, 0x00020000);
	constexpr unsigned TILE_BYTES = AT_BKV * AT_D * ES;  /* one K or V tile in memory */

	/* 16-bit K tile: 8 KiB = 8 direct-to-LDS instructions of 64 x 16
	 * bytes; wave w issues instructions w, w + NW, ...; slot s of
	 * instruction j holds row s/8, chunk (s%8) ^ swz(row). Rows past Sk
	 * are given an offset past the buffer and read as zeros. */
	unsigned k_off[C::KJ];
#pragma unroll
	for (int t = 0; t < C::KJ; ++t) {
		const int s = (wave + t * NW) * 64 + lane;
		const int row = s / 8, c = (s % 8) ^ lds_swz<8>(row);
		k_off[t] = (unsigned)(row * AT_D * 2 + c * 16);
	}
	auto issue_k = [&](int kt, unsigned slot) {
		const int rows_left = p.Sk - kt * AT_BKV;
#pragma unroll
		for (int t = 0; t < C::KJ; ++t) {
			const int j = wave + t * NW;
			if (j < 8) {
				const int row = (j * 64 + lane) / 8;
				const unsigned o = row < rows_left ? k_off[t] : S3K_OOB;
				dma16s(lds0 + slot + j * 1024, rk, o, (unsigned)kt * TILE_BYTES);
			}
		}
	};

	/* 16-bit V tile (VD): like K, 8 direct-to-LDS instructions, slot s of
	 * instruction j holding key row s/8, chunk (s%8) ^ at_vswz(row) */
	const s3k_i32x4 rv = buf_rsrc(p.v + head * p.hk * ES, kv_bytes);
	unsigned v_off[VD ? C::KJ : 1];
	if constexpr (VD) {
#pragma unroll
		for (int t = 0; t < C::KJ; ++t) {
			const int s = (wave + t * NW) * 64 + lane;
			const int row = s / 8, c = (s % 8) ^ at_vswz(row);
			v_off[t] = (unsigned)(row * AT_D * 2 + c * 16);
		}
	}
	auto issue_v = [&](int kt, unsigned slot) {
		const int rows_left = p.Sk - kt * AT_BKV;
#pragma unroll
		for (int t = 0; t < C::KJ; ++t) {
			const int j = wave + t * NW;
			if (j < 8) {
				const int row = (j * 64 + lane) / 8;
				const unsigned o = row < rows_left ? v_off[t] : S3K_OOB;
				dma16s(lds0 + slot + j * 1024, rv, o, (unsigned)kt * TILE_BYTES);
			}
		}
	};

	/* staging through registers (threads 0..255): f32 K row t/4, d
	 * 16*(t%4)..+15; V keys 4*(t/16)..+3, d 4*(t%16)..+3 */
	const int kr0 = (threadIdx.x & 255) >> 2, kd0 = 16 * (threadIdx.x & 3);
	const int vk0 = 4 * ((threadIdx.x & 255) >> 4), vd0 = 4 * (threadIdx.x & 15);
	const unsigned kst_off = (unsigned)((kr0 * AT_D + kd0) * ES);
	const unsigned vst_off = (unsigned)((vk0 * AT_D + vd0) * ES);
	uint2 vr[4];
	float4 vf[4], kf[4];
	auto load_kv = [&](int kt) {
		const int so = kt * (int)TILE_BYTES;
		if constexpr (C::SPLIT) {
#pragma unroll
			for (int i = 0; i < 4; ++i)
				kf[i] = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(
					bk, kst_off + 16 * i, so, 0));
#pragma unroll
			for (int i = 0; i < 4; ++i)
				vf[i] = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(
					bv, vst_off + i * AT_D * 4, so, 0));
		} else {
#pragma unroll
			for (int i = 0; i < 4; ++i)
				vr[i] = __builtin_bit_cast(uint2, __builtin_amdgcn_raw_buffer_load_b64(
					bv, vst_off + i * AT_D * 2, so, 0));
		}
	};
	auto store_kv = [&](unsigned kslot, unsigned vslot) {
		char *vt = smem + vslot;
		if constexpr (C::SPLIT) {
			/* K hi/lo planes: logical chunks kd0/8 and kd0/8 + 1 of row kr0 */
			char *st = smem + kslot;
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

	/* LDS read addresses: K fragment (c, mb) of row 32mb + l32, chunk
	 * (2c + h) ^ swz(row); V^T row 32md + l32 at key 4h */
	unsigned ka[4][2];
#pragma unroll
	for (int c = 0; c < 4; ++c)
#pragma unroll
		for (int mb = 0; mb < 2; ++mb) {
			const int row = 32 * mb + l32;
			ka[c][mb] = lds0 + (unsigned)((row * 8 + ((2 * c + h) ^ lds_swz<8>(row))) << 4);
		}
	const unsigned va = lds0 + (unsigned)(l32 * AT_VT_PITCH + 8 * h);
	/* VD: the V^T operand of O^T += V^T P^T for row d = 32 md + l32 and keys
	 * 16 cc + 4h + {0..3} (lo) / {8..11} (hi) by transposed reads: lane q of
	 * a 16-lane group G addresses key 4 (G >> 1) + q / 4 (+ 8 for hi), d
	 * 32 md + 16 (G & 1) + 4 (q % 4); chunk cc adds 16 rows (2 KiB) */
	unsigned vtr[2][2];
	if constexpr (VD) {
		const int G = lane >> 4, q = lane & 15;
#pragma unroll
		for (int md = 0; md < 2; ++md)
#pragma unroll
			for (int hl = 0; hl < 2; ++hl) {
				const int key = 4 * (G >> 1) + (q >> 2) + 8 * hl;
				const int d = 32 * md + 16 * (G & 1) + 4 * (q & 3);
				vtr[md][hl] = (unsigned)(key * AT_D * 2 +
							 (((d >> 3) ^ at_vswz(key)) << 4) + ((d >> 2) & 1) * 8);
			}
	}

	const float *mrow = MASK ? p.mask + (long long)(q < p.Sq ? q : p.Sq - 1) * p.Sk : nullptr;

	s3k_f32x16 o[2];
#pragma unroll
	for (int md = 0; md < 2; ++md)
#pragma unroll
		for (int r = 0; r < 16; ++r)
			o[md][r] = 0.0f;
	/* running max (base-2 exponent units) and running sum of this lane's
	 * half of the query's keys */
	float m_run = -3.402823466e38f, l_run = 0.0f;
	constexpr float LOG2E = 1.44269504088896341f;
	const int nkt = (p.Sk + AT_BKV - 1) / AT_BKV;

	/* One 64-key tile. P = stage parity (kt & 1), known at compile time so
	 * that every LDS address is a register plus a constant. */
	auto step = [&](auto par, int kt) {
		constexpr int P = decltype(par)::value;
		constexpr unsigned KSLOT = P * C::KS, VSLOT = 2 * C::KS + P * C::VS;
		constexpr unsigned KNEXT = (1 - P) * C::KS, VNEXT = 2 * C::KS + (1 - P) * C::VS;
		const bool more = kt + 1 < nkt;
		/* K(kt) landed and V^T(kt) stored; every wave is past tile kt-1,
		 * whose slots are refilled below */
		wait_vm<0>();
		__syncthreads();
		if (more) {
			if constexpr (!C::SPLIT)
				issue_k(kt + 1, KNEXT);
			if constexpr (VD)
				issue_v(kt + 1, VNEXT);
			else if (stager)
				load_kv(kt + 1);
		}

		if (wave_live) {
			const int kbase = kt * AT_BKV;
			/* mask of this tile: element 4g+e of block mb is key
			 * kbase + 32mb + 8g + 4h + e */
			float4 mk[2][4];
			if constexpr (MASK) {
#pragma unroll
				for (int mb = 0; mb < 2; ++mb)
#pragma unroll
					for (int g = 0; g < 4; ++g) {
						const int key0 = kbase + 32 * mb + 8 * g + 4 * h;
						if (p.mask_vec) {
							mk[mb][g] = key0 < p.Sk ? *(const float4 *)(mrow + key0)
										: make_float4(0.f, 0.f, 0.f, 0.f);
						} else {
							const int last = p.Sk - 1;
							mk[mb][g] = make_float4(mrow[min(key0, last)], mrow[min(key0 + 1, last)],
										mrow[min(key0 + 2, last)], mrow[min(key0 + 3, last)]);
						}
					}
			}

			/* S^T = K Q^T / 8 for keys 32*mb + (row), this lane's query. The
			 * tile is worked in two 32-key halves mb so that the matrix
			 * cores and the VALU overlap inside the wave: scores of half 1
			 * run while the probabilities of half 0 are formed, and P V of
			 * half 0 while those of half 1 are. */
			s3k_f32x16 s[2];
			auto scores_half = [&](int mb) {
#pragma unroll
				for (int r = 0; r < 16; ++r)
					s[mb][r] = 0.0f;
#pragma unroll
				for (int c = 0; c < 4; ++c) {
					const uint4 kh = *(const uint4 *)(smem + (ka[c][mb] - lds0) + KSLOT);
					if constexpr (C::SPLIT) {
						const uint4 kl = *(const uint4 *)(smem + (ka[c][mb] - lds0) + KSLOT + AT_K_BYTES);
						mfma_chunk<C::FAM>(s[mb], kl, qh[c]);
						mfma_chunk<C::FAM>(s[mb], kh, ql[c]);
					}
					mfma_chunk<C::FAM>(s[mb], kh, qh[c]);
				}
			};
			/* mask and keys past Sk (last tile only) for half mb */
			auto finish_half = [&](int mb) {
				if constexpr (MASK) {
#pragma unroll
					for (int g = 0; g < 4; ++g) {
						s[mb][4 * g] += mk[mb][g].x, s[mb][4 * g + 1] += mk[mb][g].y;
						s[mb][4 * g + 2] += mk[mb][g].z, s[mb][4 * g + 3] += mk[mb][g].w;
					}
				}
				if (kbase + AT_BKV > p.Sk) {
#pragma unroll
					for (int r = 0; r < 16; ++r)
						if (kbase + 32 * mb + 8 * (r >> 2) + 4 * h + (r & 3) >= p.Sk)
							s[mb][r] = -__builtin_inff();
				}
			};

			/* probabilities exp2(s*log2(e) - m) of half mb, packed as the
			 * P^T operand of its two 16-key chunks, and their sum */
			uint4 ph[4], pl[4];
			auto probs = [&](int mb) {
				const float nm = -m_run;
				float ts = 0.0f;
#pragma unroll
				for (int sub = 0; sub < 2; ++sub) {
					float pv[8];
#pragma unroll
					for (int e = 0; e < 8; ++e)
						pv[e] = __builtin_amdgcn_exp2f(fmaf(s[mb][8 * sub + e], LOG2E, nm));
					const int cc = 2 * mb + sub;
					if constexpr (C::SPLIT) {
#pragma unroll
						for (int e = 0; e < 8; ++e)
							ts += pv[e];
						at_split8(make_float4(pv[0], pv[1], pv[2], pv[3]),
							  make_float4(pv[4], pv[5], pv[6], pv[7]), ph[cc], pl[cc]);
					} else {
						/* the sum is of the rounded values the MFMA uses */
						ph[cc] = make_uint4(at_pack2<DT>(pv[0], pv[1]), at_pack2<DT>(pv[2], pv[3]),
								    at_pack2<DT>(pv[4], pv[5]), at_pack2<DT>(pv[6], pv[7]));
						ts = at_sum2<DT>(ph[cc].x, ts);
						ts = at_sum2<DT>(ph[cc].y, ts);
						ts = at_sum2<DT>(ph[cc].z, ts);
						ts = at_sum2<DT>(ph[cc].w, ts);
					}
				}
				return ts;
			};
			/* if some lane's sum passed the bound: move the max to the
			 * tile's, rescale what is accumulated, redo half mb (rare) */
			auto settle = [&](int mb, float ts) {
				if (__builtin_amdgcn_ballot_w64(!(ts <= AT_PSUM_MAX))) {
					float mt = s[0][0];
#pragma unroll
					for (int b = 0; b < 2; ++b)
#pragma unroll
						for (int r = 0; r < 16; ++r)
							mt = fmaxf(mt, s[b][r]);
					const float m_new = fmaxf(m_run, at_max_pair(mt) * LOG2E);
					const float alpha = __builtin_amdgcn_exp2f(m_run - m_new);
					m_run = m_new;
					l_run *= alpha;
#pragma unroll
					for (int md = 0; md < 2; ++md)
#pragma unroll
						for (int r = 0; r < 16; ++r)
							o[md][r] *= alpha;
					ts = probs(mb);
				}
				l_run += ts;
			};
			/* O^T += V^T P^T over the chunks of half mb: A = V^T rows d,
			 * keys 16cc + 4h + {0..3, 8..11}, as P^T holds them */
			auto pv_half = [&](int mb) {
#pragma unroll
				for (int md = 0; md < 2; ++md) {
					const char *vrow = smem + (va - lds0) + VSLOT + md * 32 * AT_VT_PITCH;
#pragma unroll
					for (int cc = 2 * mb; cc < 2 * mb + 2; ++cc) {
						uint2 lo, hi;
						if constexpr (VD) {
							lo = at_read_tr(smem, VSLOT + cc * 2048 + vtr[md][0]);
							hi = at_read_tr(smem, VSLOT + cc * 2048 + vtr[md][1]);
						} else {
							lo = *(const uint2 *)(vrow + 32 * cc);
							hi = *(const uint2 *)(vrow + 32 * cc + 16);
						}
						const uint4 vh = make_uint4(lo.x, lo.y, hi.x, hi.y);
						if constexpr (C::SPLIT) {
							const uint2 llo = *(const uint2 *)(vrow + AT_VT_BYTES + 32 * cc);
							const uint2 lhi = *(const uint2 *)(vrow + AT_VT_BYTES + 32 * cc + 16);
							mfma_chunk<C::FAM>(o[md], make_uint4(llo.x, llo.y, lhi.x, lhi.y), ph[cc]);
							mfma_chunk<C::FAM>(o[md], vh, pl[cc]);
						}
						mfma_chunk<C::FAM>(o[md], vh, ph[cc]);
					}
				}
			};

			scores_half(0);
			finish_half(0);
			scores_half(1);
			const float ts0 = probs(0);
			settle(0, ts0);
			finish_half(1);
			pv_half(0);
			const float ts1 = probs(1);
			settle(1, ts1);
			pv_half(1);
		}

		if constexpr (!VD) {
			if (more && stager)
				store_kv(KNEXT, VNEXT);
		}
	};

	/* prologue: tile 0 into slot 0 */
	if constexpr (!C::SPLIT)
		issue_k(0, 0);
	if constexpr (VD) {
		issue_v(0, 2 * C::KS);
	} else if (stager) {
		load_kv(0);
		store_kv(0, 2 * C::KS);
	}
	for (int kt = 0; kt < nkt; kt += 2) {
		step(at_int<0>{}, kt);
		if (kt + 1 < nkt)
			step(at_int<1>{}, kt + 1);
	}

	/* normalize (a query with no finite score keeps zeros, as the
	 * reference's row_sum > 0 test leaves it) and store out[q][d] */
	const float l_tot = at_sum_pair(l_run);
	const float inv = l_tot > 0.0f ? 1.0f / l_tot : 0.0f;
	if (q < p.Sq) {
#pragma unroll
		for (int md = 0; md < 2; ++md)
#pragma unroll
			for (int g = 0; g < 4; ++g) {
				const int d0 = 32 * md + 8 * g + 4 * h;
				const float x0 = o[md][4 * g] * inv, x1 = o[md][4 * g + 1] * inv;
				const float x2 = o[md][4 * g + 2] * inv, x3 = o[md][4 * g + 3] * inv;
				const long long orow = at_out_row(p.oh, head, p.Sq, q, AT_D);
				if constexpr (C::SPLIT) {
					if (p.ofmt == 1) {
						/* the merged row r = orow / K as bf16 planes,
						 * the split of split3 / the permute kernel */
						const long long K = (long long)p.oh * AT_D, r = orow / K;
						uint16_t *dp = (uint16_t *)p.out + r * 3 * K + (orow - r * K) + d0;
						uint32_t hi[2], lo[2];
						split_bf16x2(x0, x1, hi[0], lo[0]);
						split_bf16x2(x2, x3, hi[1], lo[1]);
						*(uint2 *)dp = make_uint2(hi[0], hi[1]);
						*(uint2 *)(dp + K) = make_uint2(lo[0], lo[1]);
						*(uint2 *)(dp + 2 * K) = make_uint2(hi[0], hi[1]);
					} else if (p.ofmt == 2) {
						/* f16, flagged as the permute kernel flags it: a
						 * value past 2^15, or four nonzero values all
						 * below 2^-10 */
						const float ax = __builtin_fabsf(x0), ay = __builtin_fabsf(x1);
						const float az = __builtin_fabsf(x2), aw = __builtin_fabsf(x3);
						const float mx = fmaxf(fmaxf(ax, ay), fmaxf(az, aw));
						const bool big = (ax >= 32768.0f && ax <= 3.402823466e38f) ||
								 (ay >= 32768.0f && ay <= 3.402823466e38f) ||
								 (az >= 32768.0f && az <= 3.402823466e38f) ||
								 (aw >= 32768.0f && aw <= 3.402823466e38f);
						if (p.ovf && (big || (mx > 0.0f && mx < 0x1p-10f)))
							*p.ovf = p.ovf_tag;
						*(uint2 *)((uint16_t *)p.out + orow + d0) =
							make_uint2(pack_f16x2(x0, x1), pack_f16x2(x2, x3));
					} else {
						float *O = (float *)p.out + orow;
						*(float4 *)(O + d0) = make_float4(x0, x1, x2, x3);
					}
				} else {
					uint16_t *O = (uint16_t *)p.out + orow;
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
	int oh;                 /* > 0: output head-merged (at_out_row) */
	int ofmt;               /* attn_small: AttnArgs' operand forms */
	unsigned *ovf;
	unsigned ovf_tag;
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
				at_st<DT>(p.out, at_out_row(p.oh, head, p.Sq, qi, p.D) + d, acc[i] * inv);
		}
	}
}

/*
 * Attention over few keys (Sk <= 128, D = 64, f32): the text encoder's
 * shapes (cpu_sdpa.c:49-159 per query row, softmax over all keys), where
 * a launch's time is its latency. One workgroup per 16 queries of a head:
 * every load (K, V, the queries, the mask entries) is issued before the
 * first use, so the kernel waits for memory once; K is stored transposed
 * in LDS so that lane j's key j reads are bank-distinct. Wave w owns
 * queries 4w..4w+3 in both phases, lane l keys l and l + 64 for the
 * scores, then output element l. Arithmetic: dot = fmaf over d in
 * order, s = dot * scale + mask, p = expf(s - max), l = butterfly sum,
 * out = (fmaf over keys in order of p * v) * (1 / l), 0 when every score
 * is -inf; for Sk <= 64 these are the steps (and bits) of attn_generic.
 */
constexpr int AS_QB = 16, AS_MAXK = 128, AS_KTP = AS_MAXK + 4;

__global__ void __launch_bounds__(256) attn_small(AttnGArgs p)
{
	__shared__ __attribute__((aligned(16))) float kt[AT_D][AS_KTP];
	__shared__ __attribute__((aligned(16))) float vs[AS_MAXK][AT_D];
	__shared__ __attribute__((aligned(16))) float qs[AS_QB][AT_D];
	__shared__ __attribute__((aligned(16))) float ps[AS_QB][AS_MAXK];
	const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
	const int nqb = (p.Sq + AS_QB - 1) / AS_QB;
	const long long head = blockIdx.x / nqb;
	const int q0 = (int)(blockIdx.x - head * nqb) * AS_QB;
	const int nq = min(AS_QB, p.Sq - q0);
	const float4 *K4 = (const float4 *)p.k + head * p.Sk * (AT_D / 4);
	const float4 *V4 = (const float4 *)p.v + head * p.Sk * (AT_D / 4);
	const float4 *Q4 = (const float4 *)p.q + (head * p.Sq + q0) * (AT_D / 4);
	const int n4 = p.Sk * (AT_D / 4);

	/* every load first */
	constexpr int NL = AS_MAXK * AT_D / 4 / 256; /* float4 of K (and of V) per thread */
	float4 kr[NL], vr[NL];
#pragma unroll
	for (int i = 0; i < NL; ++i) {
		const int idx = min(i * 256 + tid, n4 - 1); /* in bounds; the extra ones unused */
		kr[i] = K4[idx];
		vr[i] = V4[idx];
	}
	const float4 qr = tid < nq * (AT_D / 4) ? Q4[tid] : make_float4(0.f, 0.f, 0.f, 0.f);
	float mk[4][2];
#pragma unroll
	for (int j = 0; j < 4; ++j)
#pragma unroll
		for (int c = 0; c < 2; ++c) {
			const int q = q0 + 4 * wave + j, key = lane + 64 * c;
			mk[j][c] = p.mask && q < p.Sq && key < p.Sk ? p.mask[(long long)q * p.Sk + key]
								      : 0.0f;
		}
#pragma unroll
	for (int i = 0; i < NL; ++i) {
		const int idx = i * 256 + tid;
		if (idx < n4) {
			const int key = idx >> 4, d0 = (idx & 15) * 4;
			kt[d0][key] = kr[i].x;
			kt[d0 + 1][key] = kr[i].y;
			kt[d0 + 2][key] = kr[i].z;
			kt[d0 + 3][key] = kr[i].w;
			*(float4 *)&vs[key][d0] = vr[i];
		}
	}
	*(float4 *)&qs[tid >> 4][(tid & 15) * 4] = qr;
	__syncthreads();

	/* the wave's queries: nqw of 4 exist (wave-uniform); a wave without
	 * any is done (no barrier follows) */
	const int nqw = min(4, p.Sq - (q0 + 4 * wave));
	if (nqw <= 0)
		return;

	/* scores of this wave's queries against keys lane, lane + 64 (the
	 * second only when Sk > 64) */
	float sc[4][2];
#pragma unroll
	for (int j = 0; j < 4; ++j)
		sc[j][0] = sc[j][1] = 0.0f;
	const bool hi = p.Sk > 64;
	auto dots = [&](auto two) {
		constexpr bool TWO = decltype(two)::value != 0;
#pragma unroll 2
		for (int d = 0; d < AT_D; d += 4) {
			float k0[4], k1[4];
#pragma unroll
			for (int e = 0; e < 4; ++e) {
				k0[e] = kt[d + e][lane];
				k1[e] = TWO ? kt[d + e][lane + 64] : 0.0f;
			}
#pragma unroll
			for (int j = 0; j < 4; ++j) {
				const float4 q4 = *(const float4 *)&qs[4 * wave + j][d];
				const float qv[4] = {q4.x, q4.y, q4.z, q4.w};
#pragma unroll
				for (int e = 0; e < 4; ++e) {
					sc[j][0] = fmaf(qv[e], k0[e], sc[j][0]);
					if (TWO)
						sc[j][1] = fmaf(qv[e], k1[e], sc[j][1]);
				}
			}
		}
	};
	if (hi)
		dots(at_int<1>{});
	else
		dots(at_int<0>{});
	float inv[4];
#pragma unroll
	for (int j = 0; j < 4; ++j) {
		float s[2], m = -3.402823466e38f;
#pragma unroll
		for (int c = 0; c < 2; ++c) {
			s[c] = -__builtin_inff();
			if (lane + 64 * c < p.Sk) {
				s[c] = sc[j][c] * p.scale;
				if (p.mask)
					s[c] += mk[j][c];
			}
			m = fmaxf(m, s[c]);
		}
#pragma unroll
		for (int off = 32; off; off >>= 1)
			m = fmaxf(m, __shfl_xor(m, off));
		const float p0 = expf(s[0] - m), p1 = hi ? expf(s[1] - m) : 0.0f;
		float l = hi ? p0 + p1 : p0;
#pragma unroll
		for (int off = 32; off; off >>= 1)
			l += __shfl_xor(l, off);
		inv[j] = l > 0.0f ? 1.0f / l : 0.0f;
		ps[4 * wave + j][lane] = p0;
		ps[4 * wave + j][lane + 64] = p1;
	}
	/* the wave reads back only its own rows of ps: its LDS accesses run
	 * in order, so waiting for its writes is enough */
	__builtin_amdgcn_s_waitcnt(0xC07F); /* lgkmcnt(0) */
	__builtin_amdgcn_wave_barrier();

	/* out[q][lane] over the keys in order */
	float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
	int key = 0;
	for (; key + 4 <= p.Sk; key += 4) {
		float v[4];
#pragma unroll
		for (int e = 0; e < 4; ++e)
			v[e] = vs[key + e][lane];
#pragma unroll
		for (int j = 0; j < 4; ++j) {
			const float4 w4 = *(const float4 *)&ps[4 * wave + j][key];
			acc[j] = fmaf(w4.x, v[0], acc[j]);
			acc[j] = fmaf(w4.y, v[1], acc[j]);
			acc[j] = fmaf(w4.z, v[2], acc[j]);
			acc[j] = fmaf(w4.w, v[3], acc[j]);
		}
	}
	for (; key < p.Sk; ++key) {
		const float v = vs[key][lane];
#pragma unroll
		for (int j = 0; j < 4; ++j)
			acc[j] = fmaf(ps[4 * wave + j][key], v, acc[j]);
	}
#pragma unroll
	for (int j = 0; j < 4; ++j) {
		const int q = q0 + 4 * wave + j;
		const float x = acc[j] * inv[j];
		/* the neighbours of the operand forms' pairs and groups of four */
		const float x1 = __shfl_xor(x, 1);
		if (q >= p.Sq)
			continue;
		const long long orow = at_out_row(p.oh, head, p.Sq, q, AT_D);
		if (p.ofmt == 0) {
			((float *)p.out)[orow + lane] = x;
		} else if (p.ofmt == 1) {
			/* bf16 planes [hi|lo|hi] of the merged row, as attn_fwd */
			if (!(lane & 1)) {
				const long long K = (long long)p.oh * AT_D, r = orow / K;
				uint16_t *dp = (uint16_t *)p.out + r * 3 * K + (orow - r * K) + lane;
				uint32_t hi, lo;
				split_bf16x2(x, x1, hi, lo);
				*(uint32_t *)dp = hi;
				*(uint32_t *)(dp + K) = lo;
				*(uint32_t *)(dp + 2 * K) = hi;
			}
		} else {
			/* f16, flagged per four values as attn_fwd flags them */
			const float ax = __builtin_fabsf(x);
			float mx = fmaxf(ax, __shfl_xor(ax, 1));
			mx = fmaxf(mx, __shfl_xor(mx, 2));
			const bool big = ax >= 32768.0f && ax <= 3.402823466e38f;
			if (p.ovf && (big || (!(lane & 3) && mx > 0.0f && mx < 0x1p-10f)))
				*p.ovf = p.ovf_tag;
			if (!(lane & 1))
				*(uint32_t *)((uint16_t *)p.out + orow + lane) = pack_f16x2(x, x1);
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
	if (D == AT_D && BH >= 1 && Sq >= 1 && Sk >= 1 && (long long)BH * ((Sq + 127) / 128) < (1LL << 31) &&
	    !(((uintptr_t)q | (uintptr_t)k | (uintptr_t)v | (uintptr_t)out) & 15u) &&
	    (long long)Sk * AT_D * es <= 0x7FFFFFF0LL)
		return S3K_ATTN_MFMA;
	if (D <= 512 && (long long)BH * Sq / 4 < 0x7FFFFFFFLL)
		return S3K_ATTN_GENERIC;
	return 0;
}

/* The few-keys kernel's conditions (attn_small). */
static bool attn_small_ok(int kind, const void *q, const void *k, const void *v, void *out,
			  int BH, int Sq, int Sk, int D)
{
	return kind == S3K_F32 && D == AT_D && Sk >= 1 && Sk <= AS_MAXK && BH >= 1 && Sq >= 1 &&
	       (long long)BH * ((Sq + AS_QB - 1) / AS_QB) < (1LL << 31) &&
	       !(((uintptr_t)q | (uintptr_t)k | (uintptr_t)v | (uintptr_t)out) & 15u);
}

/* The kernel s3k_attn_heads(path, ...) runs for these arguments (0: it
 * refuses them). */
static int attn_heads_pick(int path, int kind, const void *q, const void *k, const void *v,
			   void *out, int BH, int Sq, int Sk, int D, int oh, int ofmt)
{
	const int best = s3k_attn_path(kind, q, k, v, out, BH, Sq, Sk, D);
	const bool small = attn_small_ok(kind, q, k, v, out, BH, Sq, Sk, D);
	const bool small_fmt = oh >= 0 && !(oh > 0 && BH % oh) && ofmt >= 0 && ofmt <= 2 &&
			       !(ofmt && oh <= 0);
	if (path == S3K_ATTN_SMALL)
		return small && small_fmt ? S3K_ATTN_SMALL : 0;
	if (path == 0 && small && small_fmt) {
		/* latency-bound sizes, by measured launch time (16 heads, f32,
		 * in a HIP graph): up to 64 scores per head the one-wave-per-row
		 * kernel (1 / 8 queries and keys: 3.3 / 4.4 us against 6.4 /
		 * 6.2 for attn_fwd), from 65 keys the few-keys kernel (77: 9.7
		 * against 11.0), attn_fwd in between (32: 6.5 against 8.5) */
		if ((long long)Sq * Sk <= 64 && !ofmt)
			return S3K_ATTN_GENERIC;
		if (Sk > 64)
			return S3K_ATTN_SMALL;
	}
	if (!best || (path == S3K_ATTN_MFMA && best != S3K_ATTN_MFMA) ||
	    (path != 0 && path != S3K_ATTN_MFMA && path != S3K_ATTN_GENERIC) || oh < 0 ||
	    (oh > 0 && BH % oh) || ofmt < 0 || ofmt > 2 ||
	    (ofmt && (oh <= 0 || kind != S3K_F32 || best != S3K_ATTN_MFMA || path == S3K_ATTN_GENERIC)))
		return 0;
	return path == 0 ? best : path;
}

extern "C" int s3k_attn_heads_path(int kind, const void *q, const void *k, const void *v,
				   void *out, int BH, int Sq, int Sk, int D, int oh, int ofmt)
{
	return attn_heads_pick(0, kind, q, k, v, out, BH, Sq, Sk, D, oh, ofmt);
}

extern "C" int s3k_attn_heads(int path, int kind, const void *q, const void *k, const void *v,
			      const float *mask, void *out, int BH, int Sq, int Sk, int D, int oh,
			      int ofmt, unsigned *ovf, unsigned ovf_tag, void *stream)
{
	path = attn_heads_pick(path, kind, q, k, v, out, BH, Sq, Sk, D, oh, ofmt);
	if (!path)
		return (int)hipErrorInvalidValue;
	if (path == S3K_ATTN_SMALL) {
		AttnGArgs g{};
		g.q = (const char *)q;
		g.k = (const char *)k;
		g.v = (const char *)v;
		g.mask = mask;
		g.out = (char *)out;
		g.BH = BH;
		g.Sq = Sq;
		g.Sk = Sk;
		g.D = D;
		g.oh = oh;
		g.ofmt = ofmt;
		g.ovf = ovf;
		g.ovf_tag = ovf_tag;
		g.scale = 1.0f / sqrtf((float)D);
		const dim3 grid((unsigned)((long long)BH * ((Sq + AS_QB - 1) / AS_QB)));
		hipLaunchKernelGGL(attn_small, grid, dim3(256), 0, (hipStream_t)stream, g);
		return (int)hipGetLastError();
	}
	if ((long long)BH * Sq == 0)
		return (int)hipSuccess;
	const hipStream_t st = (hipStream_t)stream;
	if (path == S3K_ATTN_GENERIC) {
		AttnGArgs g{};
		g.q = (const char *)q;
		g.k = (const char *)k;
		g.v = (const char *)v;
		g.mask = mask;
		g.out = (char *)out;
		g.BH = BH;
		g.Sq = Sq;
		g.Sk = Sk;
		g.D = D;
		g.oh = oh;
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
	p.mask_vec = mask && (Sk & 3) == 0 && ((uintptr_t)mask & 15u) == 0;
	/* waves per workgroup: 4 (128 queries); 6 and 8 for measurements */
	int nw = 4;
	if (kind != S3K_F32) {
		const int env = s3h_settings()->attn_nw;
		if (env == 4 || env == 6 || env == 8)
			nw = env;
	}
	p.BH = BH;
	p.oh = oh;
	p.ofmt = ofmt;
	p.ovf = ovf;
	p.ovf_tag = ovf_tag;
	p.nqb = (Sq + 32 * nw - 1) / (32 * nw);
	const dim3 grid((unsigned)((long long)p.nqb * BH));
	const dim3 block(64 * nw);
#define S3K_ATTN_GO(DT_, NW_, VD_)                                                          \
	do {                                                                                 \
		if (mask)                                                                    \
			hipLaunchKernelGGL((attn_fwd<DT_, NW_, true, VD_>), grid, block, 0, st, p);  \
		else                                                                         \
			hipLaunchKernelGGL((attn_fwd<DT_, NW_, false, VD_>), grid, block, 0, st, p); \
	} while (0)
	const bool vd = s3h_settings()->attn_vdma != 0;
	if (kind == S3K_F32)
		S3K_ATTN_GO(S3K_F32, 4, false);
	else if (kind == S3K_BF16) {
		if (nw == 4 && vd)
			S3K_ATTN_GO(S3K_BF16, 4, true);
		else if (nw == 4)
			S3K_ATTN_GO(S3K_BF16, 4, false);
		else if (nw == 6)
			S3K_ATTN_GO(S3K_BF16, 6, false);
		else
			S3K_ATTN_GO(S3K_BF16, 8, false);
	} else {
		if (nw == 4 && vd)
			S3K_ATTN_GO(S3K_F16, 4, true);
		else if (nw == 4)
			S3K_ATTN_GO(S3K_F16, 4, false);
		else if (nw == 6)
			S3K_ATTN_GO(S3K_F16, 6, false);
		else
			S3K_ATTN_GO(S3K_F16, 8, false);
	}
#undef S3K_ATTN_GO
	return (int)hipGetLastError();
}

extern "C" int s3k_attn(int path, int kind, const void *q, const void *k, const void *v,
			const float *mask, void *out, int BH, int Sq, int Sk, int D, void *stream)
{
	return s3k_attn_heads(path, kind, q, k, v, mask, out, BH, Sq, Sk, D, 0, 0, nullptr, 0, stream);
}
