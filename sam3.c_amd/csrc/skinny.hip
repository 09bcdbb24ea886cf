/*
 * skinny.hip - bandwidth-bound Q8_0 matmul for small M (prompt-decoder and
 * text-encoder shapes: M <= 128 tokens), gfx950.
 *
 * Computes C[M,N] = A[M,K] * W^T with W[N,K] Q8_0 blocks along k
 * (K % 32 == 0), the layout sam3.c's converter writes (cli_convert.c:
 * 374-422), i.e. the weight of gh_linear after its transpose is fused.
 * Reference arithmetic: cpu_matmul_q8.c:124-131, c += (a*q)*scale.
 *
 * Layout of the work:
 *   - a workgroup owns 16*NTW weight rows (n) and WV waves; wave w walks
 *     the k-blocks w, w+WV, ..., so the WV waves of a workgroup read
 *     neighbouring 36-byte blocks of the same rows together;
 *   - per k-block a lane (n = l & 15, k-group g = l >> 4) reads the f32
 *     scale and 8 int8 of row n, turns them into exact f16 integers with
 *     one byte permute and one packed f16 subtract per pair (the bytes are
 *     biased by 128 and placed under the f16 exponent of 1024, then
 *     1152 is subtracted), and feeds v_mfma_f32_16x16x32_f16 against the
 *     A chunk of each 16-row m-tile (f32/bf16 -> f16 in registers);
 *   - the block's scale is applied in f32 to the MFMA result
 *     (acc += s * sum_k a*q), so q is exact and only A is rounded to f16;
 *   - the WV partial sums are reduced through LDS in a fixed order
 *     (deterministic), then bias/GELU are applied and C is written.
 * HBM traffic is the weight stream (36 bytes per 32 weights) plus A once
 * per workgroup (from L2) and C once.
 */
#include "s3k.h"
#include "s3k_dev.h"

namespace s3k {

typedef __attribute__((ext_vector_type(2))) _Float16 half2_t;

struct SkinnyArgs {
	const char *a;
	const char *w;
	char       *c;
	const char *bias;
	int M, N, K;
	long long lda, ldc;   /* elements */
	int a_kind, c_kind, flags;
};

/* Two int8 (selected by SEL from w ^ 0x80808080) -> exact f16 pair. */
__device__ __forceinline__ uint32_t q8pair_to_f16(uint32_t wx, uint32_t sel)
{
	uint32_t biased = __builtin_amdgcn_perm(0x64646464u, wx, sel);
	half2_t h = __builtin_bit_cast(half2_t, biased);
	h = h - (half2_t){(_Float16)1152.0f, (_Float16)1152.0f};
	return __builtin_bit_cast(uint32_t, h);
}

template <int AK>
__device__ __forceinline__ uint4 a_chunk_f16(const char *a, long long lda, int m, int M, int k)
{
	if (m >= M)
		return make_uint4(0, 0, 0, 0);
	if (AK == S3K_F32) {
		const uint4 *p = (const uint4 *)(a + ((long long)m * lda + k) * 4);
		const uint4 x = p[0], y = p[1];
		return make_uint4(pack_f16x2(__uint_as_float(x.x), __uint_as_float(x.y)),
				  pack_f16x2(__uint_as_float(x.z), __uint_as_float(x.w)),
				  pack_f16x2(__uint_as_float(y.x), __uint_as_float(y.y)),
				  pack_f16x2(__uint_as_float(y.z), __uint_as_float(y.w)));
	} else if (AK == S3K_BF16) {
		const uint4 x = *(const uint4 *)(a + ((long long)m * lda + k) * 2);
		return make_uint4(pack_f16x2(bf16_to_f32(x.x & 0xFFFF), bf16_to_f32(x.x >> 16)),
				  pack_f16x2(bf16_to_f32(x.y & 0xFFFF), bf16_to_f32(x.y >> 16)),
				  pack_f16x2(bf16_to_f32(x.z & 0xFFFF), bf16_to_f32(x.z >> 16)),
				  pack_f16x2(bf16_to_f32(x.w & 0xFFFF), bf16_to_f32(x.w >> 16)));
	} else {
		return *(const uint4 *)(a + ((long long)m * lda + k) * 2);
	}
}

template <int AK, int MT, int NTW, int WV>
__global__ void __launch_bounds__(WV * 64) q8_skinny(SkinnyArgs p)
{
	constexpr int NV = NTW * MT * 4; /* partial floats per lane */
	__shared__ float red[WV * NV * 64];

	const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
	const int nl = lane & 15, g = lane >> 4;
	const int n0 = blockIdx.x * (16 * NTW);
	const int KB = p.K / 32;
	const long long rowbytes = (long long)KB * 36;

	const char *wrow[NTW];
#pragma unroll
	for (int t = 0; t < NTW; ++t) {
		int n = n0 + t * 16 + nl;
		n = n < p.N ? n : p.N - 1;
		wrow[t] = p.w + (long long)n * rowbytes;
	}

	s3k_f32x4 acc[NTW][MT];
#pragma unroll
	for (int t = 0; t < NTW; ++t)
#pragma unroll
		for (int mt = 0; mt < MT; ++mt)
			acc[t][mt] = (s3k_f32x4){0.f, 0.f, 0.f, 0.f};

	for (int kb = wave; kb < KB; kb += WV) {
		uint4 af[MT];
#pragma unroll
		for (int mt = 0; mt < MT; ++mt)
			af[mt] = a_chunk_f16<AK>(p.a, p.lda, mt * 16 + nl, p.M, kb * 32 + 8 * g);
#pragma unroll
		for (int t = 0; t < NTW; ++t) {
			const char *blk = wrow[t] + (long long)kb * 36;
			const float s = __uint_as_float(*(const uint32_t *)blk);
			const uint32_t *q = (const uint32_t *)(blk + 4 + 8 * g);
			const uint32_t w0 = q[0] ^ 0x80808080u, w1 = q[1] ^ 0x80808080u;
			uint4 wf;
			wf.x = q8pair_to_f16(w0, 0x04010400u);
			wf.y = q8pair_to_f16(w0, 0x04030402u);
			wf.z = q8pair_to_f16(w1, 0x04010400u);
			wf.w = q8pair_to_f16(w1, 0x04030402u);
#pragma unroll
			for (int mt = 0; mt < MT; ++mt) {
				s3k_f32x4 part = __builtin_amdgcn_mfma_f32_16x16x32_f16(
					__builtin_bit_cast(s3k_f16x8, af[mt]),
					__builtin_bit_cast(s3k_f16x8, wf),
					(s3k_f32x4){0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
#pragma unroll
				for (int j = 0; j < 4; ++j)
					acc[t][mt][j] += part[j] * s;
			}
		}
	}

	/* Cross-wave reduction, fixed order. */
#pragma unroll
	for (int t = 0; t < NTW; ++t)
#pragma unroll
		for (int mt = 0; mt < MT; ++mt)
#pragma unroll
			for (int j = 0; j < 4; ++j)
				red[((wave * NV) + (t * MT + mt) * 4 + j) * 64 + lane] = acc[t][mt][j];
	__syncthreads();

	for (int v = threadIdx.x; v < NV * 64; v += WV * 64) {
		float s = 0.0f;
#pragma unroll
		for (int w = 0; w < WV; ++w)
			s += red[w * NV * 64 + v];
		const int ln = v & 63, slot = v >> 6;
		const int j = slot & 3, tm = slot >> 2;
		const int mt = tm % MT, t = tm / MT;
		const int m = mt * 16 + 4 * (ln >> 4) + j;
		const int n = n0 + t * 16 + (ln & 15);
		if (m >= p.M || n >= p.N)
			continue;
		float bv = 0.0f;
		if (p.flags & S3K_EPI_BIAS)
			bv = load_as_f32(p.bias, n, p.c_kind);
		float o;
		if (p.c_kind == S3K_BF16)
			o = epilogue<2>(s, bv, p.flags);
		else if (p.c_kind == S3K_F16)
			o = epilogue<1>(s, bv, p.flags);
		else
			o = epilogue<0>(s, bv, p.flags);
		store_from_f32(p.c, (long long)m * p.ldc + n, p.c_kind, o);
	}
}

} /* namespace s3k */

using namespace s3k;

extern "C" int s3k_skinny_ok(const struct s3k_gemm *g)
{
	if (g->b_kind != S3K_Q8 || !(g->flags & S3K_B_NT) || g->batch != 1)
		return 0;
	if (g->M < 1 || g->M > 128 || g->N < 1 || g->K < 32 || g->K % 32)
		return 0;
	if (g->a_kind != S3K_F32 && g->a_kind != S3K_BF16 && g->a_kind != S3K_F16)
		return 0;
	const int es = g->a_kind == S3K_F32 ? 4 : 2;
	if (((uintptr_t)g->a & 15u) || ((long long)g->lda * es) % 16 || ((uintptr_t)g->b & 3u))
		return 0;
	return 1;
}

template <int AK, int MT, int NTW, int WV>
static int launch_sk(const SkinnyArgs &p, hipStream_t st)
{
	dim3 grid((p.N + 16 * NTW - 1) / (16 * NTW));
	hipLaunchKernelGGL((q8_skinny<AK, MT, NTW, WV>), grid, dim3(WV * 64), 0, st, p);
	return (int)hipGetLastError();
}

/* Waves per workgroup: enough waves in flight to cover HBM latency, at
 * most one per k-block, and a reduction buffer of at most 64 KiB
 * (WV * NTW * MT * 4 floats per lane). */
template <int AK, int MT, int NTW, int WV>
static int launch_wv_at_most(int wv, const SkinnyArgs &p, hipStream_t st)
{
	if constexpr (WV > 1) {
		if (wv < WV)
			return launch_wv_at_most<AK, MT, NTW, WV / 2>(wv, p, st);
	}
	return launch_sk<AK, MT, NTW, WV>(p, st);
}

template <int AK, int MT, int NTW>
static int launch_wv(const SkinnyArgs &p, hipStream_t st)
{
	constexpr int NV = NTW * MT * 4;
	constexpr int WVMAX = (256 / NV) >= 16 ? 16 : (256 / NV) >= 8 ? 8 : (256 / NV) >= 4 ? 4 : 2;
	const int groups = (p.N + 16 * NTW - 1) / (16 * NTW);
	const int KB = p.K / 32;
	int wv = 16;
	while (wv > 4 && (long long)groups * wv > 2048)
		wv >>= 1;
	while (wv > 1 && wv > KB)
		wv >>= 1;
	return launch_wv_at_most<AK, MT, NTW, WVMAX>(wv, p, st);
}

template <int AK>
static int launch_mt(const SkinnyArgs &p, hipStream_t st)
{
	const int mt = (p.M + 15) / 16;
	switch (mt) {
	case 1:  return launch_wv<AK, 1, 1>(p, st);
	case 2:  return launch_wv<AK, 2, 2>(p, st);
	case 3:  return launch_wv<AK, 3, 2>(p, st);
	case 4:  return launch_wv<AK, 4, 2>(p, st);
	case 5:  return launch_wv<AK, 5, 2>(p, st);
	case 6:  return launch_wv<AK, 6, 1>(p, st);
	case 7:  return launch_wv<AK, 7, 1>(p, st);
	default: return launch_wv<AK, 8, 1>(p, st);
	}
}

extern "C" int s3k_skinny_launch(const struct s3k_gemm *g, void *stream)
{
	SkinnyArgs p;
	p.a = (const char *)g->a;
	p.w = (const char *)g->b;
	p.c = (char *)g->c;
	p.bias = (const char *)g->bias;
	p.M = g->M;
	p.N = g->N;
	p.K = g->K;
	p.lda = g->lda;
	p.ldc = g->ldc;
	p.a_kind = g->a_kind;
	p.c_kind = g->c_kind;
	p.flags = g->flags;
	hipStream_t st = (hipStream_t)stream;
	switch (g->a_kind) {
	case S3K_F32:  return launch_mt<S3K_F32>(p, st);
	case S3K_BF16: return launch_mt<S3K_BF16>(p, st);
	default:       return launch_mt<S3K_F16>(p, st);
	}
}
