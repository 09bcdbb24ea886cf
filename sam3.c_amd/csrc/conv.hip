/*
 * conv.hip - NHWC Conv2D for gfx950 (sam3.c's SAM3_OP_CONV2D,
 * cpu_conv2d.c:296-435 and its f16/bf16 twins): input x [N,H,W,C], weight
 * OHWI [OC,KH,KW,C/groups], output y [N,OH,OW,OC]; stride, padding per
 * axis, groups.
 *
 * The reference unrolls input patches into a column matrix
 * [OH*OW, KH*KW*C] (im2col, cpu_conv2d.c:46-88) and multiplies it by the
 * weight viewed as [OC, KH*KW*C] (:98-128). That product is the NT GEMM
 * of gemm_dl.hip, so:
 *
 *   conv_dl (implicit GEMM, groups 1, C % 64 == 0): gemm_dl's pipeline and
 *     epilogue with an A loader that gathers the rows of the column matrix
 *     straight from x. A k-step of 64 lies inside one tap (kh, kw), so the
 *     tap walk is wave-uniform; each 16-byte load adds the tap's offset to
 *     its pixel base and checks the tap lands inside the image. Taps in
 *     the padding get an out-of-range buffer offset and load zeros. The
 *     column matrix is never written.
 *     f32 tensors run on bf16 planes, as the split f32 GEMM does: x is
 *     split once into [hi|lo|hi] per pixel (pixel pitch 3C) and W into
 *     [hi|hi|lo] per row, and the virtual k' = 3K walks the three planes,
 *     so the accumulator sums hi*hi + lo*hi + hi*lo.
 *   conv_im2col_k + GEMM (groups 1, other C, e.g. the patch embedding's
 *     C = 3): the column matrix in 16-bit, or in the f32 planes, with K
 *     padded to a multiple of 8 for gemm_dl; conv_wprep_k pads (and
 *     splits) the weight to match.
 *   conv_direct_k: one output per thread, taps and channels in the
 *     reference's order with separately rounded products and sums, so f32
 *     results are bit-exact with cpu_conv2d.c; groups and small problems.
 */
#include "gemm_common.h"
#include "lds_dma.h"

namespace s3k {

struct ConvArgs {
	GemmArgs g;    /* a = x or its planes, b = W [OC, K'], c = y; M = N*OH*OW, N = OC, K = K' */
	int H, W, C, KH, KW, stride, ph, pw, OH, OW;
	int PP;        /* pixel pitch of the A source in elements (C, or 3C for f32 planes) */
};

template <int CPR>
__device__ __forceinline__ int cv_off(int row, int c)
{
	return (row * CPR + (c ^ lds_swz<CPR>(row))) << 4;
}

template <int BM, int BN, int BK, int WGM, int WGN, int STAGES, int FAM, int CK, int OCC>
__global__ void __launch_bounds__(64 * WGM * WGN, OCC) conv_dl(ConvArgs q)
{
	const GemmArgs &p = q.g;
	constexpr int NW = WGM * WGN;
	constexpr int CPR = BK / 8;
	constexpr int A_BYTES = BM * BK * 2, B_BYTES = BN * BK * 2;
	constexpr int SB = A_BYTES + B_BYTES;
	constexpr int A_INS = BM * CPR / 64, B_INS = BN * CPR / 64;
	static_assert(A_INS % NW == 0 && B_INS % NW == 0, "loads split evenly over waves");
	constexpr int A_PER = A_INS / NW, B_PER = B_INS / NW;
	constexpr int LOADS = A_PER + B_PER;
	constexpr int WTM = BM / WGM, WTN = BN / WGN;
	constexpr int FM = WTM / 32, FN = WTN / 32;
	constexpr int KS = BK / 16;
	static_assert(NW * 32 * (WTN + 8) * 4 <= STAGES * SB, "epilogue staging fits");
	__shared__ __attribute__((aligned(1024))) char smem[STAGES * SB];

	const int lane = threadIdx.x & 63;
	const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
	const int wm0 = (wave / WGN) * WTM, wn0 = (wave % WGN) * WTN;
	const unsigned lds0 = lds_addr_of(smem);
	int tm, tn;
	tile_of(blockIdx.x, p.tiles_m, p.tiles_n, tm, tn);

	const s3k_i32x4 ra = buf_rsrc(p.a, p.a_extent);
	const s3k_i32x4 rb = buf_rsrc(p.b, p.b_extent);

	/* A: each load's output pixel (fixed across k). ih/iw are the
	 * coordinates of tap (0, 0); rows past M get a coordinate no tap can
	 * bring inside the image. */
	int a_base[A_PER], a_ih[A_PER], a_iw[A_PER];
	const int ohw = q.OH * q.OW;
#pragma unroll
	for (int j = 0; j < A_PER; ++j) {
		const int s = (j * NW + wave) * 64 + lane;
		const int row = s / CPR, c = (s % CPR) ^ lds_swz<CPR>(row);
		const int m = tm * BM + row;
		if (m < p.M) {
			const int n = m / ohw, r = m - n * ohw;
			const int oh = r / q.OW, ow = r - oh * q.OW;
			a_ih[j] = oh * q.stride - q.ph;
			a_iw[j] = ow * q.stride - q.pw;
			a_base[j] = ((n * q.H + a_ih[j]) * q.W + a_iw[j]) * q.PP * 2 + c * 16;
		} else {
			a_ih[j] = -(1 << 29);
			a_iw[j] = 0;
			a_base[j] = 0;
		}
	}
	unsigned b_off[B_PER];
#pragma unroll
	for (int j = 0; j < B_PER; ++j) {
		const int s = (j * NW + wave) * 64 + lane;
		const int row = s / CPR, c = (s % CPR) ^ lds_swz<CPR>(row);
		const int g = tn * BN + row;
		b_off[j] = g < p.N ? (unsigned)(g * p.ldb_b + c * 16) : S3K_OOB;
	}

	/* Tap walk of the next k-step to issue (steps are issued in order):
	 * plane seg, tap (kh, kw), first channel ic. */
	int w_seg = 0, w_kh = 0, w_kw = 0, w_ic = 0;
	auto issue = [&](int kt) {
		const int k0 = kt * BK;
		const unsigned st = lds0 + (unsigned)((kt % STAGES) * SB) + (unsigned)wave * 1024u;
		const int toff = ((w_kh * q.W + w_kw) * q.PP + w_seg * q.C + w_ic) * 2;
#pragma unroll
		for (int j = 0; j < A_PER; ++j) {
			const int ih = a_ih[j] + w_kh, iw = a_iw[j] + w_kw;
			const bool in = (unsigned)ih < (unsigned)q.H && (unsigned)iw < (unsigned)q.W;
			dma16s(st + j * NW * 1024, ra, in ? (unsigned)a_base[j] + (unsigned)toff : S3K_OOB, 0u);
		}
#pragma unroll
		for (int j = 0; j < B_PER; ++j)
			dma16s(st + A_BYTES + j * NW * 1024, rb, b_off[j], 2u * k0);
		w_ic += BK;
		if (w_ic == q.C) {
			w_ic = 0;
			if (++w_kw == q.KW) {
				w_kw = 0;
				if (++w_kh == q.KH) {
					w_kh = 0;
					++w_seg;
				}
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

	const int nk = p.K / BK;
#pragma unroll
	for (int s = 0; s < STAGES - 1; ++s)
		if (s < nk)
			issue(s);

	for (int kt = 0; kt < nk; ++kt) {
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
		uint4 af[2][FM], bfr[2][FN];
#pragma unroll
		for (int i = 0; i < FM; ++i)
			af[0][i] = *(const uint4 *)(As + cv_off<CPR>(wm0 + i * 32 + (lane & 31), lane >> 5));
#pragma unroll
		for (int j = 0; j < FN; ++j)
			bfr[0][j] = *(const uint4 *)(Bs + cv_off<CPR>(wn0 + j * 32 + (lane & 31), lane >> 5));
#pragma unroll
		for (int ks = 0; ks < KS; ++ks) {
			const int cur = ks & 1;
			if (ks + 1 < KS) {
				const int c = 2 * (ks + 1) + (lane >> 5);
#pragma unroll
				for (int i = 0; i < FM; ++i)
					af[cur ^ 1][i] = *(const uint4 *)(As + cv_off<CPR>(wm0 + i * 32 + (lane & 31), c));
#pragma unroll
				for (int j = 0; j < FN; ++j)
					bfr[cur ^ 1][j] = *(const uint4 *)(Bs + cv_off<CPR>(wn0 + j * 32 + (lane & 31), c));
			}
			__builtin_amdgcn_s_setprio(1);
#pragma unroll
			for (int i = 0; i < FM; ++i)
#pragma unroll
				for (int j = 0; j < FN; ++j)
					/* the weights first: the MFMA forms C^T (the
					 * transposed layout the epilogue stages) */
					mfma_chunk<FAM>(acc[i][j], bfr[cur][j], af[cur][i]);
			__builtin_amdgcn_s_setprio(0);
		}
	}

	__syncthreads();
	write_tile_ck<FM, FN, WTN, CK, true>(p, acc, smem, wave, lane, tm * BM + wm0, tn * BN + wn0, 0);
}

/* Element k of row m of the column matrix (cpu_conv2d.c:46-88): k runs
 * over (kh, kw, ic) with ic fastest; 0 in the padding or past K. */
template <int DT>
__device__ __forceinline__ float col_value(const void *x, int m, int k, int K, int H, int W, int C,
					   int KW, int stride, int ph, int pw, int OH, int OW)
{
	if (k >= K)
		return 0.0f;
	const int ohw = OH * OW;
	const int n = m / ohw, r = m - n * ohw, oh = r / OW, ow = r - oh * OW;
	const int tap = k / C, ic = k - tap * C, kh = tap / KW, kw = tap - kh * KW;
	const int ih = oh * stride - ph + kh, iw = ow * stride - pw + kw;
	if ((unsigned)ih >= (unsigned)H || (unsigned)iw >= (unsigned)W)
		return 0.0f;
	return load_as_f32(x, ((long long)(n * H + ih) * W + iw) * C + ic, DT);
}

/* Column matrix [M, Kp] (16-bit x, one rounding-free copy) or f32 planes
 * [M, 3Kp] = [hi|lo|hi] (PLANES). One thread per 8 values of a row. */
template <int DT, bool PLANES>
__global__ void __launch_bounds__(256) conv_im2col_k(const void *x, uint16_t *col, int M, int K,
						     int Kp, int H, int W, int C, int KW, int stride,
						     int ph, int pw, int OH, int OW)
{
	const int per_row = Kp / 8;
	const long long t = (long long)blockIdx.x * 256 + threadIdx.x;
	if (t >= (long long)M * per_row)
		return;
	const int m = (int)(t / per_row), k0 = (int)(t % per_row) * 8;
	if (PLANES) {
		uint32_t hi[4], lo[4];
#pragma unroll
		for (int i = 0; i < 4; ++i) {
			const float a = col_value<DT>(x, m, k0 + 2 * i, K, H, W, C, KW, stride, ph, pw, OH, OW);
			const float b = col_value<DT>(x, m, k0 + 2 * i + 1, K, H, W, C, KW, stride, ph, pw, OH, OW);
			hi[i] = pack_bf16x2(a, b);
			lo[i] = pack_bf16x2(a - __uint_as_float(hi[i] << 16), b - __uint_as_float(hi[i] & 0xFFFF0000u));
		}
		uint16_t *d = col + (long long)m * 3 * Kp + k0;
		const uint4 Hv = make_uint4(hi[0], hi[1], hi[2], hi[3]);
		*(uint4 *)d = Hv;
		*(uint4 *)(d + Kp) = make_uint4(lo[0], lo[1], lo[2], lo[3]);
		*(uint4 *)(d + 2LL * Kp) = Hv;
	} else {
		const uint16_t *xs = (const uint16_t *)x;
		uint16_t v[8];
		const int ohw = OH * OW;
		const int n = m / ohw, r = m - n * ohw, oh = r / OW, ow = r - oh * OW;
#pragma unroll
		for (int i = 0; i < 8; ++i) {
			const int k = k0 + i;
			v[i] = 0;
			if (k < K) {
				const int tap = k / C, ic = k - tap * C, kh = tap / KW, kw = tap - kh * KW;
				const int ih = oh * stride - ph + kh, iw = ow * stride - pw + kw;
				if ((unsigned)ih < (unsigned)H && (unsigned)iw < (unsigned)W)
					v[i] = xs[((long long)(n * H + ih) * W + iw) * C + ic];
			}
		}
		*(uint4 *)(col + (long long)m * Kp + k0) =
			make_uint4(v[0] | (v[1] << 16), v[2] | (v[3] << 16), v[4] | (v[5] << 16), v[6] | (v[7] << 16));
	}
}

/* Weight [OC, K] -> [OC, Kp] (16-bit, zero padded) or f32 -> planes
 * [OC, 3Kp] = [hi|hi|lo] (PLANES). One thread per 8 values of a row. */
template <int DT, bool PLANES>
__global__ void __launch_bounds__(256) conv_wprep_k(const void *w, uint16_t *out, int OC, int K, int Kp)
{
	const int per_row = Kp / 8;
	const long long t = (long long)blockIdx.x * 256 + threadIdx.x;
	if (t >= (long long)OC * per_row)
		return;
	const int o = (int)(t / per_row), k0 = (int)(t % per_row) * 8;
	if (PLANES) {
		const float *ws = (const float *)w + (long long)o * K;
		uint32_t hi[4], lo[4];
#pragma unroll
		for (int i = 0; i < 4; ++i) {
			const float a = k0 + 2 * i < K ? ws[k0 + 2 * i] : 0.0f;
			const float b = k0 + 2 * i + 1 < K ? ws[k0 + 2 * i + 1] : 0.0f;
			hi[i] = pack_bf16x2(a, b);
			lo[i] = pack_bf16x2(a - __uint_as_float(hi[i] << 16), b - __uint_as_float(hi[i] & 0xFFFF0000u));
		}
		uint16_t *d = out + (long long)o * 3 * Kp + k0;
		const uint4 Hv = make_uint4(hi[0], hi[1], hi[2], hi[3]);
		*(uint4 *)d = Hv;
		*(uint4 *)(d + Kp) = Hv;
		*(uint4 *)(d + 2LL * Kp) = make_uint4(lo[0], lo[1], lo[2], lo[3]);
	} else {
		const uint16_t *ws = (const uint16_t *)w + (long long)o * K;
		uint16_t v[8];
#pragma unroll
		for (int i = 0; i < 8; ++i)
			v[i] = k0 + i < K ? ws[k0 + i] : 0;
		*(uint4 *)(out + (long long)o * Kp + k0) =
			make_uint4(v[0] | (v[1] << 16), v[2] | (v[3] << 16), v[4] | (v[5] << 16), v[6] | (v[7] << 16));
	}
}

/* One output y[n, oh, ow, oc] per thread: acc = 0, then for each tap
 * (kh, kw) inside the image and each channel of the group, in that order,
 * acc = acc + x*w with the product and the sum rounded separately (the
 * reference's im2col + matmul order, cpu_conv2d.c:115-127; a padded tap
 * adds x = 0 there, which leaves acc unchanged). One rounding to the
 * output type at the end (cpu_conv2d_bf16.c:197-212). */
template <int DT>
__global__ void __launch_bounds__(256) conv_direct_k(const void *x, const void *w, void *y, int N,
						     int H, int W, int C, int OC, int KH, int KW,
						     int stride, int ph, int pw, int groups, int OH, int OW)
{
	const long long t = (long long)blockIdx.x * 256 + threadIdx.x;
	const long long total = (long long)N * OH * OW * OC;
	if (t >= total)
		return;
	const int oc = (int)(t % OC);
	const long long pix = t / OC;
	const int ow = (int)(pix % OW), oh = (int)((pix / OW) % OH), n = (int)(pix / ((long long)OW * OH));
	const int cpg_in = C / groups, cpg_out = OC / groups, g = oc / cpg_out;
	const long long wrow = (long long)oc * KH * KW * cpg_in;
	float acc = 0.0f;
	for (int kh = 0; kh < KH; ++kh) {
		const int ih = oh * stride - ph + kh;
		if ((unsigned)ih >= (unsigned)H)
			continue;
		for (int kw = 0; kw < KW; ++kw) {
			const int iw = ow * stride - pw + kw;
			if ((unsigned)iw >= (unsigned)W)
				continue;
			const long long xo = ((long long)(n * H + ih) * W + iw) * C + (long long)g * cpg_in;
			const long long wo = wrow + (long long)(kh * KW + kw) * cpg_in;
			for (int ic = 0; ic < cpg_in; ++ic)
				acc = add_rn(acc, mul_rn(load_as_f32(x, xo + ic, DT), load_as_f32(w, wo + ic, DT)));
		}
	}
	store_from_f32(y, t, DT, acc);
}

template <int BM, int BN, int BK, int WGM, int WGN, int STAGES, int OCC>
static int launch_conv_cfg(ConvArgs q, int kind, hipStream_t st)
{
	q.g.tiles_m = (q.g.M + BM - 1) / BM;
	q.g.tiles_n = (q.g.N + BN - 1) / BN;
	const dim3 grid(q.g.tiles_m * q.g.tiles_n), block(64 * WGM * WGN);
	if (kind == S3K_F32)
		hipLaunchKernelGGL((conv_dl<BM, BN, BK, WGM, WGN, STAGES, FAM_BF16, S3K_F32, OCC>), grid, block, 0, st, q);
	else if (kind == S3K_BF16)
		hipLaunchKernelGGL((conv_dl<BM, BN, BK, WGM, WGN, STAGES, FAM_BF16, S3K_BF16, OCC>), grid, block, 0, st, q);
	else
		hipLaunchKernelGGL((conv_dl<BM, BN, BK, WGM, WGN, STAGES, FAM_F16, S3K_F16, OCC>), grid, block, 0, st, q);
	return (int)hipGetLastError();
}

static long long conv_tiles(int M, int N, int bm, int bn)
{
	return (long long)((M + bm - 1) / bm) * ((N + bn - 1) / bn);
}

} /* namespace s3k */

using namespace s3k;

static dim3 grid_for(long long threads)
{
	return dim3((unsigned)((threads + 255) / 256));
}

extern "C" int s3k_conv_implicit(const struct s3k_conv *c, const void *xa, const void *wb,
				 int pixel_pitch, void *stream)
{
	const int K1 = c->KH * c->KW * c->C;
	const int segs = c->kind == S3K_F32 ? 3 : 1;
	const long long M = (long long)c->N * c->OH * c->OW;
	const long long a_bytes = (long long)c->N * c->H * c->W * pixel_pitch * 2;
	if (c->groups != 1 || c->C % 64 || M <= 0 || M > INT32_MAX || c->OC <= 0 ||
	    a_bytes > 0x7FFFFFF0LL || (long long)c->OC * K1 * segs * 2 > 0x7FFFFFF0LL ||
	    (((uintptr_t)xa | (uintptr_t)wb) & 15u))
		return (int)hipErrorInvalidValue;
	ConvArgs q = {};
	q.g.a = (const char *)xa;
	q.g.b = (const char *)wb;
	q.g.c = (char *)c->y;
	q.g.bias = (const char *)c->bias;
	q.g.M = (int)M;
	q.g.N = c->OC;
	q.g.K = K1 * segs;
	q.g.ldb_b = (long long)K1 * segs * 2;
	q.g.ldc = c->OC;
	q.g.flags = c->flags & (S3K_EPI_BIAS | S3K_EPI_GELU);
	q.g.c_kind = c->kind;
	q.g.bias_kind = c->kind;
	q.g.vec_ok = (c->OC % 8 == 0) && (((uintptr_t)c->y & 15u) == 0);
	q.g.a_extent = (unsigned)a_bytes;
	q.g.b_extent = (unsigned)((long long)c->OC * K1 * segs * 2);
	q.H = c->H; q.W = c->W; q.C = c->C; q.KH = c->KH; q.KW = c->KW;
	q.stride = c->stride; q.ph = c->pad_h; q.pw = c->pad_w; q.OH = c->OH; q.OW = c->OW;
	q.PP = pixel_pitch;
	hipStream_t st = (hipStream_t)stream;
	int cfg = s3h_settings()->conv_cfg;
	/* Tiles (measured on the neck shapes): 64x64 when 128x128 tiles would
	 * not cover the 256 CUs (72x72 maps: 5184 x 256), else the GEMM's
	 * rule (256x256 for one nearly full round, 192x128 from 192 tiles). */
	if (cfg < 0) {
		const long long t9 = conv_tiles(q.g.M, q.g.N, 256, 256), t10 = conv_tiles(q.g.M, q.g.N, 192, 128);
		cfg = conv_tiles(q.g.M, q.g.N, 128, 128) < 256 ? 2 : (t9 >= 224 && t9 <= 256) ? 9 : t10 >= 192 ? 10 : 4;
	}
	switch (cfg) {
	case 2:  return launch_conv_cfg<64, 64, 64, 2, 2, 2, 2>(q, c->kind, st);
	case 4:  return launch_conv_cfg<128, 128, 64, 2, 2, 2, 2>(q, c->kind, st);
	case 5:  return launch_conv_cfg<128, 64, 64, 2, 2, 2, 2>(q, c->kind, st);
	case 9:  return launch_conv_cfg<256, 256, 64, 2, 4, 2, 1>(q, c->kind, st);
	case 10: return launch_conv_cfg<192, 128, 64, 2, 4, 2, 1>(q, c->kind, st);
	default: return (int)hipErrorInvalidValue;
	}
}

extern "C" int s3k_conv_im2col(const struct s3k_conv *c, void *col, int Kp, void *stream)
{
	const int K = c->KH * c->KW * c->C;
	const long long M = (long long)c->N * c->OH * c->OW;
	if (c->groups != 1 || Kp < K || Kp % 8 || M <= 0 || M > INT32_MAX || ((uintptr_t)col & 15u))
		return (int)hipErrorInvalidValue;
	const dim3 grid = grid_for(M * (Kp / 8));
	hipStream_t st = (hipStream_t)stream;
	const int m = (int)M;
	if (c->kind == S3K_F32)
		hipLaunchKernelGGL((conv_im2col_k<S3K_F32, true>), grid, dim3(256), 0, st, c->x, (uint16_t *)col, m, K, Kp,
				   c->H, c->W, c->C, c->KW, c->stride, c->pad_h, c->pad_w, c->OH, c->OW);
	else if (c->kind == S3K_BF16 || c->kind == S3K_F16)
		hipLaunchKernelGGL((conv_im2col_k<S3K_BF16, false>), grid, dim3(256), 0, st, c->x, (uint16_t *)col, m, K, Kp,
				   c->H, c->W, c->C, c->KW, c->stride, c->pad_h, c->pad_w, c->OH, c->OW);
	else
		return (int)hipErrorInvalidValue;
	return (int)hipGetLastError();
}

extern "C" int s3k_conv_wprep(int kind, const void *w, void *out, int OC, int K, int Kp, void *stream)
{
	if (OC <= 0 || K <= 0 || Kp < K || Kp % 8 || ((uintptr_t)out & 15u))
		return (int)hipErrorInvalidValue;
	const dim3 grid = grid_for((long long)OC * (Kp / 8));
	hipStream_t st = (hipStream_t)stream;
	if (kind == S3K_F32)
		hipLaunchKernelGGL((conv_wprep_k<S3K_F32, true>), grid, dim3(256), 0, st, w, (uint16_t *)out, OC, K, Kp);
	else if (kind == S3K_BF16 || kind == S3K_F16)
		hipLaunchKernelGGL((conv_wprep_k<S3K_BF16, false>), grid, dim3(256), 0, st, w, (uint16_t *)out, OC, K, Kp);
	else
		return (int)hipErrorInvalidValue;
	return (int)hipGetLastError();
}

extern "C" int s3k_conv_direct(const struct s3k_conv *c, void *stream)
{
	const long long total = (long long)c->N * c->OH * c->OW * c->OC;
	if (total <= 0)
		return 0;
	hipStream_t st = (hipStream_t)stream;
	const dim3 grid = grid_for(total);
#define S3K_CONV_DIRECT(DT)                                                                        \
	hipLaunchKernelGGL((conv_direct_k<DT>), grid, dim3(256), 0, st, c->x, c->w, c->y, c->N, c->H, \
			   c->W, c->C, c->OC, c->KH, c->KW, c->stride, c->pad_h, c->pad_w, c->groups,  \
			   c->OH, c->OW)
	if (c->kind == S3K_F32)
		S3K_CONV_DIRECT(S3K_F32);
	else if (c->kind == S3K_BF16)
		S3K_CONV_DIRECT(S3K_BF16);
	else if (c->kind == S3K_F16)
		S3K_CONV_DIRECT(S3K_F16);
	else
		return (int)hipErrorInvalidValue;
#undef S3K_CONV_DIRECT
	return (int)hipGetLastError();
}
