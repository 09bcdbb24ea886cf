/*
 * skinny.hip - bandwidth-bound Q8_0 matmul for small M (prompt-decoder and
 * text-encoder shapes: M <= 128 tokens), gfx950.
 *
 * Computes C[M,N] = A[M,K] * W^T with W[N,K] Q8_0 blocks along k
 * (K % 32 == 0), the layout sam3.c's converter writes (cli_convert.c:
 * 374-422), i.e. the weight of gh_linear after its transpose is fused.
 * Reference arithmetic: cpu_matmul_q8.c:124-131, c += (a*q)*scale.
 *
 * Both kernels feed v_mfma_f32_16x16x32_f16 with exact integers: per
 * k-block a lane takes the f32 scale and 8 int8 of one weight row and
 * turns the bytes into f16 with one byte permute and one packed f16
 * subtract per pair (the bytes are biased by 128 and placed under the f16
 * exponent of 1024, then 1152 is subtracted). The block's scale is applied
 * in f32 to the MFMA result (acc += s * sum_k a*q), so q is exact and only
 * A is rounded to f16. Partial sums of the waves of a workgroup are reduced
 * through LDS in a fixed order, so results are deterministic.
 *
 * q8_stream (K % 256 == 0, 16-byte aligned W): the streaming kernel.
 *   - A workgroup owns NR = 16*NT weight rows and MR activation rows and
 *     walks k in chunks of KC = 8 or 16 blocks (256 or 512 k). Per chunk
 *     it moves the raw 36-byte blocks of its rows (KC * 36 contiguous
 *     bytes per row) and the A chunk (MR rows) straight into LDS with
 *     buffer_load ... lds, 16 bytes per lane, no VGPR staging; rows past
 *     N or M read zeros. The 16 waves of a workgroup share the loads and
 *     split the chunk's k-blocks; a wave issues all its MFMAs before the
 *     scale FMAs, so the blocks' latencies overlap.
 *   - A ring of ST chunks keeps the whole LDS budget in flight (waits are
 *     explicit vmcnt counts, so a wave only waits for its own oldest
 *     chunk).
 *   - The A image is XOR-swizzled per row (16-byte slot ^ (row & 15)), so
 *     the fragment reads of 16 rows hit 16 different bank groups.
 *   - M > MR is split over workgroups; the workgroups that share weight
 *     rows are given ids on the same XCD so the re-reads hit its L2.
 *   - The grid's y dimension walks a batch of independent problems
 *     (weights at a byte stride), which is how a stream of layers or heads
 *     runs in one launch.
 * q8_skinny (other K or alignment): per k-block global loads, one
 * workgroup per 16*NTW rows.
 */
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "s3k.h"
#include "s3k_dev.h"
#include "lds_dma.h"

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
	const float *rs;      /* S3K_EPI_ROWSCALE row factors */
	const float *res;     /* S3K_EPI_RES: f32 [M, N], pitch N, added last */
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
		if (p.flags & S3K_EPI_ROWSCALE)
			s *= p.rs[m];
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
		if (p.flags & S3K_EPI_RES)
			o += p.res[(long long)m * p.N + n];
		store_from_f32(p.c, (long long)m * p.ldc + n, p.c_kind, o);
	}
}


/* ------------------------------------------------------------------ */
/* q8_stream                                                            */
/* ------------------------------------------------------------------ */

struct StreamArgs {
	const char *a;
	const char *w;
	char       *c;
	const char *bias;
	int M, N, K;
	int lda_b;                 /* A row pitch, bytes                      */
	long long ldc;             /* C row pitch, elements                   */
	long long sa_b, sw_b, sc;  /* batch strides: bytes, bytes, elements   */
	unsigned w_ext;            /* bytes of one weight matrix (< 2 GiB)    */
	int flags;
	int groups;                /* weight-row groups: ceil(N / NR)         */
	int zsplit;                /* activation-row groups: ceil(M / MR)     */
	const float *rs;           /* S3K_EPI_ROWSCALE row factors ...        */
	long long rs_sb;           /* ... and their batch stride              */
	const float *res;          /* S3K_EPI_RES: f32 [M, N], pitch N (batch 1) */
	/* S3K_EPI_QKV without RoPE (struct s3k_gemm): the head-split stores */
	float *qkv_out[3];
	int qkv_S, qkv_H, qkv_dsh;
	/* S3K_A_LN (f32 A only): A's rows are a LayerNorm's input, normalized
	 * here with gamma ln_g and beta ln_b; ln bit 0 set, bits 1 and 2 when
	 * gamma and beta are given */
	int ln;
	const float *ln_g, *ln_b;
	/* S3K_A_ATT1 (q8_gemv): A is v of one-key attention heads of
	 * 1 << att_dsh elements, formed from q, k and the mask entry */
	int att, att_dsh;
	const float *att_q, *att_k, *att_mask;
	float att_scale;
	int nbatch;                /* q8_gemv_tasks: weight matrices        */
};

template <int AK, int MR, int NT, int KC, int RKB = 76>
struct StreamCfg {
	static constexpr int ES = AK == S3K_F32 ? 4 : 2;
	static constexpr int WV = 16;                    /* waves per workgroup      */
	static constexpr int CW = WV < KC ? WV : KC;     /* waves that multiply      */
	static constexpr int U = KC / CW;                /* k-blocks per wave, chunk */
	static constexpr int NR = 16 * NT;               /* weight rows              */
	static constexpr int MT = (MR + 15) / 16;        /* 16-row MFMA tiles of A   */
	static constexpr int GPRW = KC * 36 / 16;        /* 16-B slots of a W row    */
	static constexpr int PW = GPRW + 1;              /* LDS row pitch, slots     */
	static constexpr int GW = NR * PW;
	static constexpr int IW = (GW + 63) / 64;        /* KiB of W per chunk       */
	static constexpr int GAR = KC * 32 * ES / 16;    /* 16-B slots per A row     */
	static constexpr int GA = MR * GAR;
	static constexpr int IA = (GA + 63) / 64;        /* KiB of A per chunk       */
	static constexpr int I = IW + IA;
	static constexpr int NPW = (I + WV - 1) / WV;    /* loads per wave per chunk */
	static constexpr int SW = IW * 1024, SB = I * 1024;
	/* ring budget RKB KiB: 76 lets two workgroups share a CU, so one's
	 * start hides the other's drain (a deeper ring measured no faster
	 * for q8_stream and q8_gemv); q8_gemv_tasks, one workgroup per CU
	 * for the whole launch, takes 144 */
	static constexpr int ST0 = (RKB * 1024) / SB;
	static constexpr int ST1 = ST0 < 2 ? 2 : ST0 > 16 ? 16 : ST0;
	static constexpr int ST = (ST1 - 1) * NPW > 63 ? 63 / NPW + 1 : ST1; /* ring depth */
	static constexpr int RED = WV * NT * MT * 1024;
	static constexpr int LDS = ST * SB + 1024 > RED ? ST * SB + 1024 : RED;
	static_assert(KC == 8 || KC == 16, "chunk of 8 or 16 k-blocks");
	static_assert(GAR >= 16 && (GAR & (GAR - 1)) == 0, "A rows hold 2^n >= 16 slots");
	static_assert(LDS <= 160 * 1024, "LDS budget");
};

template <int AK, int MR, int NT, int KC>
__global__ void __launch_bounds__(1024) q8_stream(StreamArgs p)
{
	using C = StreamCfg<AK, MR, NT, KC>;
	constexpr int WV = C::WV;
	/* f32 / bf16 activations are rounded to f16 at the fragment read with
	 * a power-of-two factor per row (scale_exp_of, as the row-scaled f16
	 * copy uses): 2^-e before the rounding, 2^e in the epilogue */
	constexpr bool SCALE = AK != S3K_F16;
	/* S3K_A_LN (f32 A). Not built into the MR = 1, KC = 8 instance:
	 * hipcc (ROCm 7.2) fails instruction selection on it ("operand has
	 * incorrect register class"); stream_ln_ok keeps LN problems off it
	 * (K % 512 == 0 makes one-row workgroups take KC = 16). */
	constexpr bool LN = AK == S3K_F32 && !(MR == 1 && KC == 8);
	__shared__ __attribute__((aligned(1024))) char smem[C::LDS];
	__shared__ float rsc[SCALE ? 2 * MR : 1];
	__shared__ float rmx[SCALE ? C::WV * MR : 1];
	/* S3K_A_LN's LDS, allocated at launch (dynamic) only for it: gamma
	 * and beta f32 [K] (loaded once), then each row's mean and 1 / std */
	extern __shared__ __attribute__((aligned(16))) float lnsm[];
	float *const lng = lnsm, *const lnb = lnsm + p.K, *const lnst = lnsm + 2 * p.K;
	const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
	const int g16 = lane >> 4, l16 = lane & 15;

	/* workgroup -> (row group gi, activation group z); the zsplit
	 * workgroups of one row group get ids = x (mod 8), i.e. one XCD. */
	int gi, z;
	{
		const int id = blockIdx.x, Z = p.zsplit, G8 = (p.groups / 8) * 8;
		if (id < G8 * Z) {
			const int x = id % 8, r = id / 8;
			gi = (r / Z) * 8 + x;
			z = r % Z;
		} else {
			const int rem = id - G8 * Z;
			gi = G8 + rem / Z;
			z = rem % Z;
		}
	}
	const int n0 = gi * C::NR, m0 = z * MR;
	const int Mz = min(MR, p.M - m0);
	const int KB = p.K / 32;
	const unsigned rowbytes = (unsigned)KB * 36u;
	const char *abase = p.a + blockIdx.y * p.sa_b + (long long)m0 * p.lda_b;
	const s3k_i32x4 rw = buf_rsrc(p.w + blockIdx.y * p.sw_b, p.w_ext);
	const s3k_i32x4 ra = buf_rsrc(abase, (unsigned)((Mz - 1) * p.lda_b + p.K * C::ES));

	/* Source of each of this lane's loads for chunk 0. Load j of a chunk
	 * is wave j % WV's (j / WV)-th; j < IW moves W rows (PW slots each,
	 * the last one a zero pad that spreads the rows over the LDS banks),
	 * then A rows, then padding loads (zeros into a spare KiB) keep every
	 * wave at NPW loads per chunk. */
	unsigned off[C::NPW];
#pragma unroll
	for (int t = 0; t < C::NPW; ++t) {
		const int j = t * C::WV + wave;
		unsigned o = S3K_OOB;
		if (j < C::IW) {
			const int i = j * 64 + lane;
			const int r = i / C::PW, q = i % C::PW;
			if (i < C::GW && q < C::GPRW && n0 + r < p.N)
				o = (unsigned)(n0 + r) * rowbytes + (unsigned)q * 16u;
		} else if (j < C::I) {
			const int i = (j - C::IW) * 64 + lane;
			const int m = i / C::GAR, sl = i % C::GAR;
			if (m < Mz)
				o = (unsigned)(m * p.lda_b) + (unsigned)((sl ^ (m & 15)) * 16);
		}
		off[t] = o;
	}

	auto issue = [&](int ch) {
		char *st = smem + (ch % C::ST) * C::SB;
		const unsigned wi = (unsigned)ch * (KC * 36);
		const unsigned ai = (unsigned)ch * (KC * 32 * C::ES);
#pragma unroll
		for (int t = 0; t < C::NPW; ++t) {
			const int j = t * C::WV + wave;
			if (j < C::IW)
				dma16(st + j * 1024, rw, off[t] + wi);
			else if (j < C::I)
				dma16(st + C::SW + (j - C::IW) * 1024, ra, off[t] + ai);
			else
				dma16(smem + C::ST * C::SB, rw, S3K_OOB);
		}
	};

	s3k_f32x4 acc[NT][C::MT];
	const int nch = p.K / (KC * 32);

	/* f32 / bf16 rows are rounded with factor 1 first while each lane
	 * tracks the largest |value| of its rows; rows that need another
	 * factor (rare) make the workgroup run the pass again with the factors */
	float inv[C::MT], amx[C::MT];
#pragma unroll
	for (int mt = 0; mt < C::MT; ++mt)
		inv[mt] = 1.0f, amx[mt] = 0.0f;

	/* S3K_A_LN: the row statistics of layernorm_v (blockops.hip) for rows
	 * of K = 256 * slots f32 values, one wave per row: lane l sums its
	 * 16-byte pieces (64 s + l) of each slot s in order, then the wave
	 * sums; the same for the centred squares. The same operations in the
	 * same order, so the normalized rows below have LayerNorm's bits. The
	 * first chunks' loads are already in flight (the ring is primed
	 * before), so the statistics' one round trip overlaps them. */
	auto ln_stats = [&]() {
		constexpr int RPW = (MR + WV - 1) / WV; /* rows per wave */
		const int slots = p.K / 256;
		float4 xv[RPW][8];
#pragma unroll
		for (int r = 0; r < RPW; ++r) {
			const int m = wave + r * WV;
			const float *xr = (const float *)(abase + (long long)(m < Mz ? m : 0) * p.lda_b);
#pragma unroll
			for (int i = 0; i < 8; ++i)
				if (i < slots && m < Mz)
					xv[r][i] = *(const float4 *)(xr + (i * 64 + lane) * 4);
		}
#pragma unroll
		for (int r = 0; r < RPW; ++r) {
			const int m = wave + r * WV;
			if (m >= Mz)
				continue;
			float sum = 0.0f;
#pragma unroll
			for (int i = 0; i < 8; ++i)
				if (i < slots) {
					sum += xv[r][i].x;
					sum += xv[r][i].y;
					sum += xv[r][i].z;
					sum += xv[r][i].w;
				}
			sum = wave_xor_sum(sum);
			const float mean = sum / (float)p.K;
			float var = 0.0f;
#pragma unroll
			for (int i = 0; i < 8; ++i)
				if (i < slots) {
					float d = sub_rn(xv[r][i].x, mean);
					var = fmaf(d, d, var);
					d = sub_rn(xv[r][i].y, mean);
					var = fmaf(d, d, var);
					d = sub_rn(xv[r][i].z, mean);
					var = fmaf(d, d, var);
					d = sub_rn(xv[r][i].w, mean);
					var = fmaf(d, d, var);
				}
			var = wave_xor_sum(var);
			if (lane == 0) {
				lnst[2 * m] = mean;
				lnst[2 * m + 1] = 1.0f / sqrtf(var / (float)p.K + 1e-5f);
			}
		}
	};

	auto prime = [&]() {
#pragma unroll
		for (int s = 0; s < C::ST - 1; ++s)
			if (s < nch)
				issue(s);
	};

	/* primed: the first ST - 1 chunks were issued before */
	auto pass = [&](bool track, bool primed) {
#pragma unroll
		for (int t = 0; t < NT; ++t)
#pragma unroll
			for (int mt = 0; mt < C::MT; ++mt)
				acc[t][mt] = (s3k_f32x4){0.f, 0.f, 0.f, 0.f};
		if (!primed)
			prime();

		for (int ch = 0; ch < nch; ++ch) {
			/* this wave's loads of chunk ch done (younger chunks may fly) */
			if (ch + C::ST - 2 < nch)
				wait_vm<(C::ST - 2) * C::NPW>();
			else
				wait_vm<0>();
			wg_barrier();
			if (ch + C::ST - 1 < nch)
				issue(ch + C::ST - 1);

			if (C::CW < WV && wave >= C::CW)
				continue;
			const char *Ws = smem + (ch % C::ST) * C::SB;
			const char *As = Ws + C::SW;
			/* operands of this wave's U k-blocks first, then all MFMAs,
			 * then the scale FMAs: independent chains instead of one per
			 * block */
			uint4 af[C::U][C::MT], wf[C::U][NT];
			float sc[C::U][NT];
#pragma unroll
			for (int u = 0; u < C::U; ++u) {
				const int kb = u * C::CW + wave;
#pragma unroll
				for (int mt = 0; mt < C::MT; ++mt) {
					const int m = mt * 16 + l16;
					af[u][mt] = make_uint4(0, 0, 0, 0);
					if (m < MR) {
						const char *row = As + m * (C::GAR * 16);
						float v[8];
						if constexpr (AK == S3K_F32) {
							const int q0 = kb * 8 + 2 * g16;
							const uint4 x = *(const uint4 *)(row + ((q0 ^ (m & 15)) << 4));
							const uint4 y = *(const uint4 *)(row + (((q0 + 1) ^ (m & 15)) << 4));
							v[0] = __uint_as_float(x.x), v[1] = __uint_as_float(x.y);
							v[2] = __uint_as_float(x.z), v[3] = __uint_as_float(x.w);
							v[4] = __uint_as_float(y.x), v[5] = __uint_as_float(y.y);
							v[6] = __uint_as_float(y.z), v[7] = __uint_as_float(y.w);
							if (LN && p.ln && m < Mz) {
								/* layernorm_v's (x - mean) * rstd * g + b,
								 * each step rounded */
								const int k0 = ch * (KC * 32) + kb * 32 + 8 * g16;
								const float mean = lnst[2 * m], rstd = lnst[2 * m + 1];
								float gv[8], bv[8];
#pragma unroll
								for (int e = 0; e < 8; e += 4) {
									const float4 gq = *(const float4 *)(lng + k0 + e);
									const float4 bq = *(const float4 *)(lnb + k0 + e);
									gv[e] = gq.x, gv[e + 1] = gq.y, gv[e + 2] = gq.z, gv[e + 3] = gq.w;
									bv[e] = bq.x, bv[e + 1] = bq.y, bv[e + 2] = bq.z, bv[e + 3] = bq.w;
								}
#pragma unroll
								for (int e = 0; e < 8; ++e) {
									float t = mul_rn(sub_rn(v[e], mean), rstd);
									if (p.ln & 2)
										t = mul_rn(t, gv[e]);
									if (p.ln & 4)
										t = add_rn(t, bv[e]);
									v[e] = t;
								}
							}
						} else if constexpr (AK == S3K_BF16) {
							const int q0 = kb * 4 + g16;
							const uint4 x = *(const uint4 *)(row + ((q0 ^ (m & 15)) << 4));
							v[0] = bf16_to_f32(x.x & 0xFFFF), v[1] = bf16_to_f32(x.x >> 16);
							v[2] = bf16_to_f32(x.y & 0xFFFF), v[3] = bf16_to_f32(x.y >> 16);
							v[4] = bf16_to_f32(x.z & 0xFFFF), v[5] = bf16_to_f32(x.z >> 16);
							v[6] = bf16_to_f32(x.w & 0xFFFF), v[7] = bf16_to_f32(x.w >> 16);
						} else {
							const int q0 = kb * 4 + g16;
							af[u][mt] = *(const uint4 *)(row + ((q0 ^ (m & 15)) << 4));
						}
						if constexpr (SCALE) {
							if (track) {
#pragma unroll
								for (int e = 0; e < 8; ++e)
									amx[mt] = fmaxf(amx[mt], finite_abs(v[e]));
							}
							const float f = inv[mt];
							af[u][mt] = make_uint4(pack_f16x2(v[0] * f, v[1] * f),
									       pack_f16x2(v[2] * f, v[3] * f),
									       pack_f16x2(v[4] * f, v[5] * f),
									       pack_f16x2(v[6] * f, v[7] * f));
						}
					}
				}
#pragma unroll
				for (int t = 0; t < NT; ++t) {
					const char *blk = Ws + (t * 16 + l16) * (C::PW * 16) + kb * 36;
					sc[u][t] = *(const float *)blk;
					const uint32_t w0 = *(const uint32_t *)(blk + 4 + 8 * g16) ^ 0x80808080u;
					const uint32_t w1 = *(const uint32_t *)(blk + 8 + 8 * g16) ^ 0x80808080u;
					wf[u][t].x = q8pair_to_f16(w0, 0x04010400u);
					wf[u][t].y = q8pair_to_f16(w0, 0x04030402u);
					wf[u][t].z = q8pair_to_f16(w1, 0x04010400u);
					wf[u][t].w = q8pair_to_f16(w1, 0x04030402u);
				}
			}
			s3k_f32x4 part[C::U][NT][C::MT];
#pragma unroll
			for (int u = 0; u < C::U; ++u)
#pragma unroll
				for (int t = 0; t < NT; ++t)
#pragma unroll
					for (int mt = 0; mt < C::MT; ++mt)
						part[u][t][mt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(
							__builtin_bit_cast(s3k_f16x8, af[u][mt]),
							__builtin_bit_cast(s3k_f16x8, wf[u][t]),
							(s3k_f32x4){0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
#pragma unroll
			for (int u = 0; u < C::U; ++u)
#pragma unroll
				for (int t = 0; t < NT; ++t)
#pragma unroll
					for (int mt = 0; mt < C::MT; ++mt)
#pragma unroll
						for (int j = 0; j < 4; ++j)
							acc[t][mt][j] += part[u][t][mt][j] * sc[u][t];
		}
		wait_vm<0>();
		wg_barrier();
	};

	if constexpr (LN) {
		/* gamma and beta into LDS ahead of the ring's loads (older, so
		 * the ring's waits cover them; K * 4 bytes each, 1 KiB per wave
		 * load, piece j by wave j; absent ones are not read) */
		if (p.ln) {
			const int pieces = p.K / 256;
			const s3k_i32x4 rg = buf_rsrc(p.ln_g, (p.ln & 2) ? (unsigned)p.K * 4u : 0u);
			const s3k_i32x4 rb = buf_rsrc(p.ln_b, (p.ln & 4) ? (unsigned)p.K * 4u : 0u);
			if (wave < pieces && (p.ln & 2))
				dma16(lng + wave * 256, rg, (unsigned)(wave * 1024 + lane * 16));
			else if (wave >= pieces && wave < 2 * pieces && (p.ln & 4))
				dma16(lnb + (wave - pieces) * 256, rb,
				      (unsigned)((wave - pieces) * 1024 + lane * 16));
		}
	}
	prime();
	if constexpr (LN) {
		if (p.ln) {
			ln_stats();
			__syncthreads();
		}
	}
	pass(SCALE, true);
	if constexpr (SCALE) {
		/* each row's largest |value|: over the 4 lanes of a wave that hold
		 * it (g16), then over the waves through LDS; rsc = 2^-e, 2^e */
#pragma unroll
		for (int mt = 0; mt < C::MT; ++mt) {
			float a = amx[mt];
			a = fmaxf(a, __shfl_xor(a, 16));
			a = fmaxf(a, __shfl_xor(a, 32));
			const int m = mt * 16 + l16;
			if (g16 == 0 && m < MR)
				rmx[wave * MR + m] = a;
		}
		__builtin_amdgcn_s_waitcnt(0xC07F); /* lgkmcnt(0) */
		wg_barrier();
		if (threadIdx.x < MR) {
			float a = 0.0f;
			for (int w = 0; w < C::CW; ++w)
				a = fmaxf(a, rmx[w * MR + threadIdx.x]);
			const int ex = threadIdx.x < Mz ? scale_exp_of(a) : 0;
			rsc[threadIdx.x] = pow2f(-ex);
			rsc[MR + threadIdx.x] = pow2f(ex);
			rmx[threadIdx.x] = ex != 0 ? 1.0f : 0.0f; /* rows 0..MR-1 of wave 0 are read */
		}
		__builtin_amdgcn_s_waitcnt(0xC07F);
		wg_barrier();
		bool again = false;
		for (int m = 0; m < MR; ++m)
			again |= rmx[m] != 0.0f;
		if (again) {
#pragma unroll
			for (int mt = 0; mt < C::MT; ++mt) {
				const int m = mt * 16 + l16;
				inv[mt] = m < MR ? rsc[m] : 1.0f;
			}
			pass(false, false);
		}
	}

	/* Cross-wave reduction in a fixed order, then bias/GELU and store. */
	constexpr int NV = NT * C::MT * 4;
	wait_vm<0>();
	wg_barrier();
	float *red = (float *)smem;
#pragma unroll
	for (int t = 0; t < NT; ++t)
#pragma unroll
		for (int mt = 0; mt < C::MT; ++mt)
#pragma unroll
			for (int j = 0; j < 4; ++j)
				red[((wave * NV) + (t * C::MT + mt) * 4 + j) * 64 + lane] = acc[t][mt][j];
	__syncthreads();

	float *cb = (float *)p.c + blockIdx.y * p.sc;
#pragma unroll 1
	for (int v = threadIdx.x; v < NV * 64; v += C::WV * 64) {
		float s = 0.0f;
#pragma unroll
		for (int w = 0; w < C::WV; ++w)
			s += red[w * NV * 64 + v];
		const int ln = v & 63, slot = v >> 6;
		const int j = slot & 3, tm = slot >> 2;
		const int mt = tm % C::MT, t = tm / C::MT;
		const int m = mt * 16 + 4 * (ln >> 4) + j;
		const int n = n0 + t * 16 + (ln & 15);
		if (m >= Mz || n >= p.N)
			continue;
		if constexpr (SCALE)
			s *= rsc[MR + m];
		if (p.flags & S3K_EPI_ROWSCALE)
			s *= p.rs[blockIdx.y * p.rs_sb + m0 + m];
		const float bv = (p.flags & S3K_EPI_BIAS) ? ((const float *)p.bias)[n] : 0.0f;
		float o = epilogue<0>(s, bv, p.flags);
		if (p.flags & S3K_EPI_RES)
			o += p.res[(long long)(m0 + m) * p.N + n];
		if (p.flags & S3K_EPI_QKV) {
			/* column n: operand y, head h, element d; row: (b, s) */
			const int D = 1 << p.qkv_dsh, E = p.qkv_H << p.qkv_dsh;
			const int y = (n >= E) + (n >= 2 * E), r = n - y * E;
			const int mm = m0 + m, b = mm / p.qkv_S, sq = mm - b * p.qkv_S;
			float *oy = y == 0 ? p.qkv_out[0] : y == 1 ? p.qkv_out[1] : p.qkv_out[2];
			oy[(((long long)b * p.qkv_H + (r >> p.qkv_dsh)) * p.qkv_S + sq) * D + (r & (D - 1))] = o;
		} else {
			cb[(long long)(m0 + m) * p.ldc + n] = o;
		}
	}
}

/*
 * q8_gemv: one f32 activation row times Q8_0 W[N,K] (the text encoder at
 * one token, decoder steps, config 4's M = 1). The weights and the row
 * stream through q8_stream's LDS ring (same chunks, loads and waits), but
 * the products run on the VALU in f32: lane (row l16 of a 16-row tile,
 * group g16) multiplies its 8 activations of a k-block by the 8 int8
 * weights converted exactly to f32, sums them in order, and adds that
 * sum times the block's f32 scale to its accumulator (cpu_matmul_q8.c:
 * 124-131 forms a * q * scale in f32 as well). Nothing is rounded to f16,
 * so there is no row factor and no second pass, and per chunk a wave
 * issues about a quarter of q8_stream's instructions (no activation
 * conversion, no MFMA operand packing), the cost that bounds a launch
 * over few workgroups. The 4 lanes of a row then add their sums
 * (xor 16, then 32) and the waves theirs through LDS in wave order:
 * deterministic. S3K_A_LN normalizes the row as q8_stream does
 * (layernorm_v's statistics and steps), with gamma and beta in LDS.
 *
 * S3K_A_ATT1: the row is the attention output of one query over one key
 * per head (the text encoder at one token), formed from v as the
 * attention kernel forms it (cpu_sdpa.c:49-159 for a one-key row):
 * waves 0.. load q and k into LDS ahead of the weight ring, 1024
 * elements each, and D/16 lanes per head chain the dot product's fmaf
 * over d in order (16 elements per lane, the running sum handed on by
 * lane shifts); the score s = dot * scale (+ the mask entry) gives
 * attn_generic's softmax weight p = expf(s - max(-FLT_MAX, s)) (NaN
 * scores drop out of its max) and 1 / p (0 unless p > 0), stored per
 * head in LDS before the first chunk's barrier; each element is then
 * fmaf(p, v, 0) * (1 / p), the kernel's accumulate-and-normalize steps.
 */
template <int NT, int KC>
__global__ void __launch_bounds__(1024) q8_gemv(StreamArgs p)
{
	using C = StreamCfg<S3K_F32, 1, NT, KC>;
	constexpr int WV = C::WV;
	__shared__ __attribute__((aligned(1024))) char smem[C::LDS];
	extern __shared__ __attribute__((aligned(16))) float lnsm[];
	float *const lng = lnsm, *const lnb = lnsm + p.K, *const lnst = lnsm + 2 * p.K;
	/* S3K_A_ATT1: q, k and per head (p, 1 / p) in the same space */
	float *const atq = lnsm, *const atk = lnsm + p.K, *const atst = lnsm + 2 * p.K;
	const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
	const int g16 = lane >> 4, l16 = lane & 15;

	/* workgroup -> weight-row group (one activation row: zsplit 1); ids
	 * of a group of 8 row groups lie on the 8 XCDs, as in q8_stream */
	const int gi = blockIdx.x;
	const int n0 = gi * C::NR;
	const int KB = p.K / 32;
	const unsigned rowbytes = (unsigned)KB * 36u;
	const char *abase = p.a + blockIdx.y * p.sa_b;
	const s3k_i32x4 rw = buf_rsrc(p.w + blockIdx.y * p.sw_b, p.w_ext);
	const s3k_i32x4 ra = buf_rsrc(abase, (unsigned)(p.K * 4));

	/* the loads of a chunk, as q8_stream's (A: the one row, 16-B slots
	 * unswizzled since row 0's swizzle is the identity) */
	unsigned off[C::NPW];
#pragma unroll
	for (int t = 0; t < C::NPW; ++t) {
		const int j = t * C::WV + wave;
		unsigned o = S3K_OOB;
		if (j < C::IW) {
			const int i = j * 64 + lane;
			const int r = i / C::PW, q = i % C::PW;
			if (i < C::GW && q < C::GPRW && n0 + r < p.N)
				o = (unsigned)(n0 + r) * rowbytes + (unsigned)q * 16u;
		} else if (j < C::I) {
			const int i = (j - C::IW) * 64 + lane;
			if (i < C::GAR)
				o = (unsigned)(i * 16);
		}
		off[t] = o;
	}
	auto issue = [&](int ch) {
		char *st = smem + (ch % C::ST) * C::SB;
		const unsigned wi = (unsigned)ch * (KC * 36);
		const unsigned ai = (unsigned)ch * (KC * 32 * 4);
#pragma unroll
		for (int t = 0; t < C::NPW; ++t) {
			const int j = t * C::WV + wave;
			if (j < C::IW)
				dma16(st + j * 1024, rw, off[t] + wi);
			else if (j < C::I)
				dma16(st + C::SW + (j - C::IW) * 1024, ra, off[t] + ai);
			else
				dma16(smem + C::ST * C::SB, rw, S3K_OOB);
		}
	};
	const int nch = p.K / (KC * 32);

	/* S3K_A_ATT1: wave w loads q and k elements [1024 w, 1024 w + 1024) */
	const bool att_wave = p.att && wave * 1024 < p.K;
	if (att_wave) {
		const s3k_i32x4 rq = buf_rsrc(p.att_q, (unsigned)p.K * 4u);
		const s3k_i32x4 rk = buf_rsrc(p.att_k, (unsigned)p.K * 4u);
#pragma unroll
		for (int j = 0; j < 4; ++j) {
			const int e0 = wave * 1024 + j * 256;
			if (e0 < p.K) {
				dma16(atq + e0, rq, (unsigned)(e0 * 4 + lane * 16));
				dma16(atk + e0, rk, (unsigned)(e0 * 4 + lane * 16));
			}
		}
	}

	if (p.ln) {
		const int pieces = p.K / 256;
		const s3k_i32x4 rg = buf_rsrc(p.ln_g, (p.ln & 2) ? (unsigned)p.K * 4u : 0u);
		const s3k_i32x4 rb = buf_rsrc(p.ln_b, (p.ln & 4) ? (unsigned)p.K * 4u : 0u);
		if (wave < pieces && (p.ln & 2))
			dma16(lng + wave * 256, rg, (unsigned)(wave * 1024 + lane * 16));
		else if (wave >= pieces && wave < 2 * pieces && (p.ln & 4))
			dma16(lnb + (wave - pieces) * 256, rb, (unsigned)((wave - pieces) * 1024 + lane * 16));
	}
#pragma unroll
	for (int s = 0; s < C::ST - 1; ++s)
		if (s < nch)
			issue(s);
	if (p.ln) {
		/* layernorm_v's statistics of the row (wave 0), as q8_stream's */
		if (wave == 0) {
			const int slots = p.K / 256;
			const float *xr = (const float *)abase;
			float4 xv[8];
#pragma unroll
			for (int i = 0; i < 8; ++i)
				if (i < slots)
					xv[i] = *(const float4 *)(xr + (i * 64 + lane) * 4);
			float sum = 0.0f;
#pragma unroll
			for (int i = 0; i < 8; ++i)
				if (i < slots) {
					sum += xv[i].x;
					sum += xv[i].y;
					sum += xv[i].z;
					sum += xv[i].w;
				}
			sum = wave_xor_sum(sum);
			const float mean = sum / (float)p.K;
			float var = 0.0f;
#pragma unroll
			for (int i = 0; i < 8; ++i)
				if (i < slots) {
					float d = sub_rn(xv[i].x, mean);
					var = fmaf(d, d, var);
					d = sub_rn(xv[i].y, mean);
					var = fmaf(d, d, var);
					d = sub_rn(xv[i].z, mean);
					var = fmaf(d, d, var);
					d = sub_rn(xv[i].w, mean);
					var = fmaf(d, d, var);
				}
			var = wave_xor_sum(var);
			if (lane == 0) {
				lnst[0] = mean;
				lnst[1] = 1.0f / sqrtf(var / (float)p.K + 1e-5f);
			}
		}
		__syncthreads();
	}
	if (att_wave) {
		/* the mask entry by a scalar load (lgkmcnt, not the vmcnt that
		 * counts the DMAs), then this wave's q and k, whose DMAs were
		 * issued before the prime */
		const float att_mv =
			p.att_mask ? *(const __attribute__((address_space(4))) float *)p.att_mask : 0.0f;
		if (nch >= C::ST - 1)
			wait_vm<(C::ST - 1) * C::NPW>();
		else
			wait_vm<0>();
		const int lph = (1 << p.att_dsh) >> 4; /* lanes per head */
		const int seg = lane & (lph - 1);
		const int e0 = wave * 1024 + lane * 16;
		float qv[16], kv[16];
#pragma unroll
		for (int i = 0; i < 16; i += 4) {
			const float4 a4 = *(const float4 *)(atq + e0 + i);
			const float4 b4 = *(const float4 *)(atk + e0 + i);
			qv[i] = a4.x, qv[i + 1] = a4.y, qv[i + 2] = a4.z, qv[i + 3] = a4.w;
			kv[i] = b4.x, kv[i + 1] = b4.y, kv[i + 2] = b4.z, kv[i + 3] = b4.w;
		}
		/* the dot's fmaf chain over d in order: after step t the lanes
		 * of segments <= t hold their prefix */
		float dot = 0.0f;
		for (int t = 0; t < lph; ++t) {
			const float prev = __shfl_up(dot, 1);
			float d = seg == 0 ? 0.0f : prev;
#pragma unroll
			for (int i = 0; i < 16; ++i)
				d = fmaf(qv[i], kv[i], d);
			dot = d;
		}
		if (seg == lph - 1 && e0 < p.K) {
			float sc = dot * p.att_scale;
			if (p.att_mask)
				sc += att_mv;
			const float mt = sc != sc ? -__builtin_inff() : sc;
			const float m_new = fmaxf(-3.402823466e38f, mt);
			const float pj = expf(sc - m_new);
			const int h = e0 >> p.att_dsh;
			atst[2 * h] = pj;
			atst[2 * h + 1] = pj > 0.0f ? 1.0f / pj : 0.0f;
		}
		/* the stores land before the first chunk's barrier */
		__builtin_amdgcn_s_waitcnt(0xC07F);
	}

	float acc[NT];
#pragma unroll
	for (int t = 0; t < NT; ++t)
		acc[t] = 0.0f;
	for (int ch = 0; ch < nch; ++ch) {
		if (ch + C::ST - 2 < nch)
			wait_vm<(C::ST - 2) * C::NPW>();
		else
			wait_vm<0>();
		wg_barrier();
		if (ch + C::ST - 1 < nch)
			issue(ch + C::ST - 1);
		if (C::CW < WV && wave >= C::CW)
			continue;
		const char *Ws = smem + (ch % C::ST) * C::SB;
		const char *As = Ws + C::SW;
#pragma unroll
		for (int u = 0; u < C::U; ++u) {
			const int kb = u * C::CW + wave;
			const int q0 = kb * 8 + 2 * g16;
			const float4 x = *(const float4 *)(As + (q0 << 4));
			const float4 y = *(const float4 *)(As + ((q0 + 1) << 4));
			float a[8] = {x.x, x.y, x.z, x.w, y.x, y.y, y.z, y.w};
			if (p.ln) {
				/* layernorm_v's (x - mean) * rstd * g + b, each step rounded */
				const int k0 = ch * (KC * 32) + kb * 32 + 8 * g16;
				const float mean = lnst[0], rstd = lnst[1];
				float gv[8], bv[8];
#pragma unroll
				for (int e = 0; e < 8; e += 4) {
					const float4 gq = *(const float4 *)(lng + k0 + e);
					const float4 bq = *(const float4 *)(lnb + k0 + e);
					gv[e] = gq.x, gv[e + 1] = gq.y, gv[e + 2] = gq.z, gv[e + 3] = gq.w;
					bv[e] = bq.x, bv[e + 1] = bq.y, bv[e + 2] = bq.z, bv[e + 3] = bq.w;
				}
#pragma unroll
				for (int e = 0; e < 8; ++e) {
					float t = mul_rn(sub_rn(a[e], mean), rstd);
					if (p.ln & 2)
						t = mul_rn(t, gv[e]);
					if (p.ln & 4)
						t = add_rn(t, bv[e]);
					a[e] = t;
				}
			}
			if (p.att) {
				/* the attention kernel's fmaf(p, v, 0) * (1 / p) */
				const int k0 = ch * (KC * 32) + kb * 32 + 8 * g16;
				const float2 pw = *(const float2 *)(atst + 2 * (k0 >> p.att_dsh));
#pragma unroll
				for (int e = 0; e < 8; ++e)
					a[e] = fmaf(pw.x, a[e], 0.0f) * pw.y;
			}
#pragma unroll
			for (int t = 0; t < NT; ++t) {
				const char *blk = Ws + (t * 16 + l16) * (C::PW * 16) + kb * 36;
				const float sc = *(const float *)blk;
				const uint32_t w0 = *(const uint32_t *)(blk + 4 + 8 * g16);
				const uint32_t w1 = *(const uint32_t *)(blk + 8 + 8 * g16);
				float s8 = 0.0f;
#pragma unroll
				for (int e = 0; e < 4; ++e)
					s8 = fmaf(a[e], (float)(int)(signed char)(w0 >> (8 * e)), s8);
#pragma unroll
				for (int e = 0; e < 4; ++e)
					s8 = fmaf(a[4 + e], (float)(int)(signed char)(w1 >> (8 * e)), s8);
				acc[t] = fmaf(sc, s8, acc[t]);
			}
		}
	}

	/* the row's 4 lanes, then the waves in order */
	wait_vm<0>();
	wg_barrier();
	float *red = (float *)smem;
#pragma unroll
	for (int t = 0; t < NT; ++t) {
		float v = acc[t] + __int_as_float(__builtin_amdgcn_ds_swizzle(__float_as_int(acc[t]),
									      0x401F));
		{
			const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v),
									 __float_as_uint(v), false, false);
			v = __uint_as_float(r[0]) + __uint_as_float(r[1]);
		}
		if (g16 == 0)
			red[wave * C::NR + t * 16 + l16] = v;
	}
	__syncthreads();
	if (threadIdx.x < C::NR) {
		const int v = threadIdx.x, n = n0 + v;
		if (n < p.N) {
			float s = 0.0f;
#pragma unroll
			for (int w = 0; w < WV; ++w)
				s += red[w * C::NR + v];
			if (p.flags & S3K_EPI_ROWSCALE)
				s *= p.rs[blockIdx.y * p.rs_sb];
			const float bv = (p.flags & S3K_EPI_BIAS) ? ((const float *)p.bias)[n] : 0.0f;
			float o = epilogue<0>(s, bv, p.flags);
			if (p.flags & S3K_EPI_RES)
				o += p.res[n];
			if (p.flags & S3K_EPI_QKV) {
				const int D = 1 << p.qkv_dsh, E = p.qkv_H << p.qkv_dsh;
				const int y = (n >= E) + (n >= 2 * E), r = n - y * E;
				float *oy = y == 0 ? p.qkv_out[0] : y == 1 ? p.qkv_out[1] : p.qkv_out[2];
				oy[(long long)(r >> p.qkv_dsh) * p.qkv_S * D + (r & (D - 1))] = o;
			} else {
				((float *)p.c + blockIdx.y * p.sc)[n] = o;
			}
		}
	}
}

/*
 * q8_gemv_tasks: q8_gemv over a batch of weight matrices (config 4's
 * streams of one activation row) as a persistent grid of one workgroup
 * per CU. The tasks are (copy z, weight-row group g), task t = z * groups
 * + g; workgroup w runs tasks w, w + G, w + 2G, ... (G workgroups) and
 * streams all their chunks through one ring, so the loads of a task's
 * first chunks are in flight while the previous task's last chunks are
 * multiplied; no workgroup starts or drains per task. With 8-block
 * chunks and TSPLIT the two waves of a block take half the row tiles
 * each (q8_gemv leaves 8 of its 16 waves idle there). At a
 * task's last chunk the sums go through LDS (the row's 4 lanes, then the
 * blocks in order) and the epilogue stores the task's outputs: the
 * arithmetic of q8_gemv<NT, KC>, so its bits (a launch of one copy runs
 * 16-block chunks when K % 512 == 0, which split k over the waves
 * differently from 8-block ones; with KC = 8 for such K the sums agree
 * to a few ulps). Rows are whole groups (N % NR == 0) and K whole
 * chunks; bias and GELU only.
 */
template <int NT, int KC, bool TSPLIT>
__global__ void __launch_bounds__(1024) q8_gemv_tasks(StreamArgs p)
{
	using C = StreamCfg<S3K_F32, 1, NT, KC, 144>;
	constexpr int WV = C::WV;
	/* TSPLIT: every wave multiplies; with fewer k-blocks per chunk than
	 * waves (KC = 8) the waves of block kb split the row tiles, TS ways.
	 * Otherwise waves past CW only load. */
	constexpr int TS = TSPLIT ? WV / C::CW : 1, NTW = NT / TS;
	static_assert(C::U == 1 || TS == 1, "tiles split only with one block per wave");
	static_assert(NT % TS == 0, "tiles split evenly");
	__shared__ __attribute__((aligned(1024))) char smem[C::ST * C::SB + 1024];
	__shared__ float red[C::CW * C::NR];
	const int lane = threadIdx.x & 63;
	const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6); /* wave-uniform LDS addresses */
	const int g16 = lane >> 4, l16 = lane & 15;
	const int kw = wave % C::CW, t0 = (wave / C::CW) * NTW; /* block slot, first tile */
	const bool active = wave < C::CW * TS;

	const unsigned rowbytes = (unsigned)(p.K / 32) * 36u;
	const int nch = p.K / (KC * 32);
	const int ntask = p.groups * p.nbatch;
	const int G = (int)gridDim.x;
	const int mine = (ntask - (int)blockIdx.x + G - 1) / G;
	const int total = mine * nch;

	/* per-lane part of the loads of a chunk (the task's rows and k go in
	 * the scalar offset) */
	unsigned off[C::NPW];
#pragma unroll
	for (int t = 0; t < C::NPW; ++t) {
		const int j = t * C::WV + wave;
		unsigned o = S3K_OOB;
		if (j < C::IW) {
			const int i = j * 64 + lane;
			const int r = i / C::PW, q = i % C::PW;
			if (i < C::GW && q < C::GPRW)
				o = (unsigned)r * rowbytes + (unsigned)q * 16u;
		} else if (j < C::I) {
			const int i = (j - C::IW) * 64 + lane;
			if (i < C::GAR)
				o = (unsigned)(i * 16);
		}
		off[t] = o;
	}
	const unsigned lds0 = lds_addr_of(smem);
	auto issue = [&](int c) {
		const int i = c / nch, ch = c - i * nch;
		const int task = (int)blockIdx.x + i * G;
		const int z = task / p.groups, g = task - z * p.groups;
		const s3k_i32x4 rw = buf_rsrc(p.w + z * p.sw_b, p.w_ext);
		const s3k_i32x4 ra = buf_rsrc(p.a + z * p.sa_b, (unsigned)(p.K * 4));
		const unsigned wso = (unsigned)g * C::NR * rowbytes + (unsigned)ch * (KC * 36);
		const unsigned aso = (unsigned)ch * (KC * 32 * 4);
		const unsigned st = lds0 + (unsigned)((c % C::ST) * C::SB);
#pragma unroll
		for (int t = 0; t < C::NPW; ++t) {
			const int j = t * C::WV + wave;
			if (j < C::IW)
				dma16s(st + j * 1024, rw, off[t], wso);
			else if (j < C::I)
				dma16s(st + C::SW + (j - C::IW) * 1024, ra, off[t], aso);
			else
				dma16s(lds0 + C::ST * C::SB, rw, S3K_OOB, 0);
		}
	};

#pragma unroll
	for (int s = 0; s < C::ST - 1; ++s)
		if (s < total)
			issue(s);

	float acc[NTW];
#pragma unroll
	for (int t = 0; t < NTW; ++t)
		acc[t] = 0.0f;
	for (int c = 0; c < total; ++c) {
		if (c + C::ST - 2 < total)
			wait_vm<(C::ST - 2) * C::NPW>();
		else
			wait_vm<0>();
		wg_barrier();
		if (c + C::ST - 1 < total)
			issue(c + C::ST - 1);
		const int i = c / nch, ch = c - i * nch;
		if (active) {
			const char *Ws = smem + (c % C::ST) * C::SB;
			const char *As = Ws + C::SW;
#pragma unroll
			for (int u = 0; u < C::U; ++u) {
				const int kb = u * C::CW + kw;
				const int q0 = kb * 8 + 2 * g16;
				const float4 x = *(const float4 *)(As + (q0 << 4));
				const float4 y = *(const float4 *)(As + ((q0 + 1) << 4));
				const float a[8] = {x.x, x.y, x.z, x.w, y.x, y.y, y.z, y.w};
#pragma unroll
				for (int tt = 0; tt < NTW; ++tt) {
					const int t = t0 + tt;
					const char *blk = Ws + (t * 16 + l16) * (C::PW * 16) + kb * 36;
					const float sc = *(const float *)blk;
					const uint32_t w0 = *(const uint32_t *)(blk + 4 + 8 * g16);
					const uint32_t w1 = *(const uint32_t *)(blk + 8 + 8 * g16);
					float s8 = 0.0f;
#pragma unroll
					for (int e = 0; e < 4; ++e)
						s8 = fmaf(a[e], (float)(int)(signed char)(w0 >> (8 * e)), s8);
#pragma unroll
					for (int e = 0; e < 4; ++e)
						s8 = fmaf(a[4 + e], (float)(int)(signed char)(w1 >> (8 * e)), s8);
					acc[tt] = fmaf(sc, s8, acc[tt]);
				}
			}
		}
		if (ch == nch - 1) {
			/* the task's sums: the row's 4 lanes, then the block slots
			 * in order */
#pragma unroll
			for (int tt = 0; tt < NTW; ++tt) {
				float v = acc[tt] + __int_as_float(__builtin_amdgcn_ds_swizzle(
							    __float_as_int(acc[tt]), 0x401F));
				const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v),
										 __float_as_uint(v), false, false);
				v = __uint_as_float(r[0]) + __uint_as_float(r[1]);
				if (g16 == 0 && active)
					red[kw * C::NR + (t0 + tt) * 16 + l16] = v;
				acc[tt] = 0.0f;
			}
			__builtin_amdgcn_s_waitcnt(0xC07F); /* lgkmcnt(0) */
			wg_barrier();
			if (threadIdx.x < C::NR) {
				const int task = (int)blockIdx.x + i * G;
				const int z = task / p.groups, g = task - z * p.groups;
				const int n = g * C::NR + (int)threadIdx.x;
				float sum = 0.0f;
#pragma unroll
				for (int w = 0; w < C::CW; ++w)
					sum += red[w * C::NR + threadIdx.x];
				const float bv = (p.flags & S3K_EPI_BIAS) ? ((const float *)p.bias)[n] : 0.0f;
				((float *)p.c + z * p.sc)[n] = epilogue<0>(sum, bv, p.flags);
			}
		}
	}
	wait_vm<0>();
}

/*
 * q8_stream_tasks: a batch of weight matrices times 2-16 f16 activation
 * rows each (config 4's streams of a few tokens), as a persistent grid
 * with q8_gemv_tasks' walk: tasks (copy z, 128-row group g), task
 * t = z * groups + g, workgroup w taking tasks w, w + G, ..., all their
 * 8-block chunks (weight rows and the activation rows) through one
 * ring. Every task covers all M <= MR rows. Wave w multiplies weight
 * tile w & 7 (16 rows) by blocks 4 (w >> 3) .. + 3 of each chunk: per
 * block one v_mfma_f32_16x16x32_f16 of the f16 activations and the exact
 * integers q, times the block scale in f32 (q8_stream's products), added
 * into the wave's accumulators block by block. At a task's last chunk
 * the waves leave their accumulators in a buffer beside the ring (whose
 * next chunks are in flight) and each output is the sum of its two
 * halves of k. Rows are whole groups (N % 128 == 0) and K whole chunks;
 * row factors (S3K_EPI_ROWSCALE), bias and GELU.
 */
template <int MR>
__global__ void __launch_bounds__(1024) q8_stream_tasks(StreamArgs p)
{
	constexpr int NT = 8, KC = 8;
	using C = StreamCfg<S3K_F16, MR, NT, KC, 140>;
	constexpr int WV = C::WV;
	static_assert(C::MT == 1 && WV == 2 * NT, "one 16-row A tile; two waves per weight tile");
	__shared__ __attribute__((aligned(1024))) char smem[C::ST * C::SB + 1024];
	__shared__ float red[WV * 4 * 64];
	const int lane = threadIdx.x & 63;
	const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
	const int g16 = lane >> 4, l16 = lane & 15;
	const int wt = wave & 7, kh = wave >> 3;

	const unsigned rowbytes = (unsigned)(p.K / 32) * 36u;
	const int nch = p.K / (KC * 32);
	const int ntask = p.groups * p.nbatch;
	const int G = (int)gridDim.x;
	const int mine = (ntask - (int)blockIdx.x + G - 1) / G;
	const int total = mine * nch;

	/* per-lane part of a chunk's loads: weight rows (PW slots each, the
	 * last a zero pad), then the M activation rows (XOR-swizzled slots,
	 * rows past M read zeros), then padding loads into the spare KiB */
	unsigned off[C::NPW];
#pragma unroll
	for (int t = 0; t < C::NPW; ++t) {
		const int j = t * C::WV + wave;
		unsigned o = S3K_OOB;
		if (j < C::IW) {
			const int i = j * 64 + lane;
			const int r = i / C::PW, q = i % C::PW;
			if (i < C::GW && q < C::GPRW)
				o = (unsigned)r * rowbytes + (unsigned)q * 16u;
		} else if (j < C::I) {
			const int i = (j - C::IW) * 64 + lane;
			const int m = i / C::GAR, sl = i % C::GAR;
			if (m < p.M)
				o = (unsigned)(m * p.lda_b) + (unsigned)((sl ^ (m & 15)) * 16);
		}
		off[t] = o;
	}
	const unsigned lds0 = lds_addr_of(smem);
	const unsigned aext = (unsigned)((p.M - 1) * p.lda_b + p.K * 2);
	auto issue = [&](int c) {
		const int i = c / nch, ch = c - i * nch;
		const int task = (int)blockIdx.x + i * G;
		const int z = task / p.groups, g = task - z * p.groups;
		const s3k_i32x4 rw = buf_rsrc(p.w + z * p.sw_b, p.w_ext);
		const s3k_i32x4 ra = buf_rsrc(p.a + z * p.sa_b, aext);
		const unsigned wso = (unsigned)g * C::NR * rowbytes + (unsigned)ch * (KC * 36);
		const unsigned aso = (unsigned)ch * (KC * 32 * 2);
		const unsigned st = lds0 + (unsigned)((c % C::ST) * C::SB);
#pragma unroll
		for (int t = 0; t < C::NPW; ++t) {
			const int j = t * C::WV + wave;
			if (j < C::IW)
				dma16s(st + j * 1024, rw, off[t], wso);
			else if (j < C::I)
				dma16s(st + C::SW + (j - C::IW) * 1024, ra, off[t], aso);
			else
				dma16s(lds0 + C::ST * C::SB, rw, S3K_OOB, 0);
		}
	};

#pragma unroll
	for (int s = 0; s < C::ST - 1; ++s)
		if (s < total)
			issue(s);

	s3k_f32x4 acc = {0.f, 0.f, 0.f, 0.f};
	for (int c = 0; c < total; ++c) {
		if (c + C::ST - 2 < total)
			wait_vm<(C::ST - 2) * C::NPW>();
		else
			wait_vm<0>();
		wg_barrier();
		if (c + C::ST - 1 < total)
			issue(c + C::ST - 1);
		const int i = c / nch, ch = c - i * nch;
		{
			const char *Ws = smem + (c % C::ST) * C::SB;
			const char *As = Ws + C::SW;
			/* the four blocks' operands first, then the MFMAs, then
			 * the scale FMAs in block order */
			uint4 af[4], wf[4];
			float sc[4];
#pragma unroll
			for (int u = 0; u < 4; ++u) {
				const int kb = 4 * kh + u;
				af[u] = make_uint4(0, 0, 0, 0);
				if (l16 < MR) {
					const int q0 = kb * 4 + g16;
					af[u] = *(const uint4 *)(As + l16 * (C::GAR * 16) + ((q0 ^ l16) << 4));
				}
				const char *blk = Ws + (wt * 16 + l16) * (C::PW * 16) + kb * 36;
				sc[u] = *(const float *)blk;
				const uint32_t w0 = *(const uint32_t *)(blk + 4 + 8 * g16) ^ 0x80808080u;
				const uint32_t w1 = *(const uint32_t *)(blk + 8 + 8 * g16) ^ 0x80808080u;
				wf[u].x = q8pair_to_f16(w0, 0x04010400u);
				wf[u].y = q8pair_to_f16(w0, 0x04030402u);
				wf[u].z = q8pair_to_f16(w1, 0x04010400u);
				wf[u].w = q8pair_to_f16(w1, 0x04030402u);
			}
			s3k_f32x4 part[4];
#pragma unroll
			for (int u = 0; u < 4; ++u)
				part[u] = __builtin_amdgcn_mfma_f32_16x16x32_f16(
					__builtin_bit_cast(s3k_f16x8, af[u]), __builtin_bit_cast(s3k_f16x8, wf[u]),
					(s3k_f32x4){0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
#pragma unroll
			for (int u = 0; u < 4; ++u)
#pragma unroll
				for (int j = 0; j < 4; ++j)
					acc[j] += part[u][j] * sc[u];
		}
		if (ch == nch - 1) {
			/* the task's outputs: each wave's accumulators into red,
			 * then output o = (tile, j, lane) of the first half of k
			 * plus the same of the second; two per thread */
#pragma unroll
			for (int j = 0; j < 4; ++j)
				red[(wave * 4 + j) * 64 + lane] = acc[j];
			acc = (s3k_f32x4){0.f, 0.f, 0.f, 0.f};
			__builtin_amdgcn_s_waitcnt(0xC07F); /* lgkmcnt(0) */
			wg_barrier();
			const int task = (int)blockIdx.x + i * G;
			const int z = task / p.groups, g = task - z * p.groups;
#pragma unroll
			for (int h = 0; h < 2; ++h) {
				const int o = (int)threadIdx.x + h * 1024;
				float s = red[o] + red[o + NT * 4 * 64];
				const int ln = o & 63, j = (o >> 6) & 3, t = o >> 8;
				const int m = 4 * (ln >> 4) + j;
				const int n = g * C::NR + t * 16 + (ln & 15);
				if (m < p.M) {
					if (p.flags & S3K_EPI_ROWSCALE)
						s *= p.rs[z * p.rs_sb + m];
					const float bv = (p.flags & S3K_EPI_BIAS) ? ((const float *)p.bias)[n] : 0.0f;
					((float *)p.c + z * p.sc)[(long long)m * p.ldc + n] =
						epilogue<0>(s, bv, p.flags);
				}
			}
		}
	}
	wait_vm<0>();
}

} /* namespace s3k */

using namespace s3k;

/* q8_stream's requirements: whole 256-k chunks, 16-byte aligned weight
 * rows (K % 256 == 0 makes the row pitch a multiple of 16), every buffer
 * range under 2 GiB. */
static bool stream_ok(const struct s3k_gemm *g)
{
	const int es = g->a_kind == S3K_F32 ? 4 : 2;
	if (g->K % 256 || ((uintptr_t)g->b & 15u))
		return false;
	const long long wext = (long long)g->N * (g->K / 32) * 36;
	const long long aext = (long long)(g->M - 1) * g->lda * es + (long long)g->K * es;
	if (wext > 0x7FFFFFF0LL || aext > 0x7FFFFFF0LL)
		return false;
	if (g->batch > 1 && (g->stride_b % 16 || (g->stride_a * es) % 16))
		return false;
	return true;
}

/* Whether the skinny launch of g rounds f32 / bf16 activations to f16
 * with per-row power-of-two factors itself (q8_stream), so that no
 * row-scaled f16 copy is needed before it. */
extern "C" int s3k_skinny_scales_rows(const struct s3k_gemm *g)
{
	return (g->a_kind == S3K_F32 || g->a_kind == S3K_BF16) && stream_ok(g) &&
	       !(g->flags & S3K_EPI_ROWSCALE);
}

/* S3K_A_LN's conditions: f32 rows that layernorm_v would normalize
 * (K % 256 == 0, K <= 2048, 16-byte aligned rows, gamma and beta), one
 * slice, on q8_stream, with K % 512 == 0 (see q8_stream's LN). */
static bool stream_ln_ok(const struct s3k_gemm *g)
{
	return g->a_kind == S3K_F32 && stream_ok(g) && g->batch == 1 && g->K <= 2048 &&
	       g->K % 512 == 0 &&
	       g->lda == g->K && !((uintptr_t)g->a & 15u) && !((uintptr_t)g->ln_g & 15u) &&
	       !((uintptr_t)g->ln_b & 15u) && !(g->flags & S3K_EPI_ROWSCALE);
}

/* S3K_A_ATT1's conditions: one f32 row of K = heads * D (D a power of
 * two from 16 to 1024, K <= 4096) on q8_gemv, q, k and v 16-byte
 * aligned, no other input form or row factor. */
static bool gemv_att_ok(const struct s3k_gemm *g)
{
	const int D = g->att_D;
	return g->a_kind == S3K_F32 && g->M == 1 && g->batch == 1 && stream_ok(g) &&
	       g->lda == g->K && g->K <= 4096 && D >= 16 && D <= 1024 && !(D & (D - 1)) &&
	       g->K % D == 0 && g->att_q && g->att_k && !((uintptr_t)g->a & 15u) &&
	       !((uintptr_t)g->att_q & 15u) && !((uintptr_t)g->att_k & 15u) &&
	       !((uintptr_t)g->att_mask & 3u) &&
	       !(g->flags & (S3K_A_LN | S3K_EPI_ROWSCALE | S3K_EPI_QKV)) && s3h_settings()->gemv_f32;
}

extern "C" int s3k_skinny_ok(const struct s3k_gemm *g)
{
	if (g->b_kind != S3K_Q8 || !(g->flags & S3K_B_NT) || g->c_kind != S3K_F32 || g->batch < 1)
		return 0;
	if (g->M < 1 || g->M > 128 || g->N < 1 || g->K < 32 || g->K % 32)
		return 0;
	if (g->a_kind != S3K_F32 && g->a_kind != S3K_BF16 && g->a_kind != S3K_F16)
		return 0;
	const int es = g->a_kind == S3K_F32 ? 4 : 2;
	if (((uintptr_t)g->a & 15u) || ((long long)g->lda * es) % 16 || ((uintptr_t)g->b & 3u))
		return 0;
	if (g->batch > 1 && !stream_ok(g))
		return 0;
	if ((g->flags & S3K_A_LN) && !stream_ln_ok(g))
		return 0;
	if ((g->flags & S3K_A_ATT1) && !gemv_att_ok(g))
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

template <int AK, int MR, int NT, int KC>
static int launch_stream_k(const struct s3k_gemm *g, void *stream)
{
	/* the instances q8_stream builds S3K_A_LN into */
	if ((g->flags & S3K_A_LN) && !(AK == S3K_F32 && !(MR == 1 && KC == 8)))
		return (int)hipErrorInvalidValue;
	const int es = AK == S3K_F32 ? 4 : 2;
	StreamArgs p;
	p.a = (const char *)g->a;
	p.w = (const char *)g->b;
	p.c = (char *)g->c;
	p.bias = (const char *)g->bias;
	p.M = g->M;
	p.N = g->N;
	p.K = g->K;
	p.lda_b = g->lda * es;
	p.ldc = g->ldc;
	p.sa_b = g->stride_a * es;
	p.sw_b = g->stride_b;
	p.sc = g->stride_c;
	p.w_ext = (unsigned)((long long)g->N * (g->K / 32) * 36);
	p.flags = g->flags;
	p.groups = (g->N + 16 * NT - 1) / (16 * NT);
	p.zsplit = (g->M + MR - 1) / MR;
	p.rs = g->rs;
	p.rs_sb = g->rs_sb;
	p.res = (const float *)g->res;
	for (int y = 0; y < 3; ++y)
		p.qkv_out[y] = g->qkv_out[y];
	p.qkv_S = g->qkv_S;
	p.qkv_H = g->qkv_H;
	p.qkv_dsh = g->qkv_D > 0 ? __builtin_ctz((unsigned)g->qkv_D) : 0;
	/* bit 0: normalize A's rows; bits 1, 2: gamma, beta given */
	p.ln = (g->flags & S3K_A_LN) ? 1 | (g->ln_g ? 2 : 0) | (g->ln_b ? 4 : 0) : 0;
	p.ln_g = g->ln_g;
	p.ln_b = g->ln_b;
	dim3 grid(p.groups * p.zsplit, g->batch);
	/* S3K_A_LN's dynamic LDS: gamma, beta [K], row statistics [2 * MR] */
	const size_t dyn = p.ln ? (size_t)(2 * g->K + 2 * MR) * 4 : 0;
	hipLaunchKernelGGL((q8_stream<AK, MR, NT, KC>), grid,
			   dim3(StreamCfg<AK, MR, NT, KC>::WV * 64), dyn, (hipStream_t)stream, p);
	return (int)hipGetLastError();
}

template <int NT, int KC>
static int launch_gemv_k(const struct s3k_gemm *g, void *stream)
{
	using C = StreamCfg<S3K_F32, 1, NT, KC>;
	StreamArgs p;
	memset(&p, 0, sizeof p);
	p.a = (const char *)g->a;
	p.w = (const char *)g->b;
	p.c = (char *)g->c;
	p.bias = (const char *)g->bias;
	p.M = 1;
	p.N = g->N;
	p.K = g->K;
	p.lda_b = g->lda * 4;
	p.ldc = g->ldc;
	p.sa_b = g->stride_a * 4;
	p.sw_b = g->stride_b;
	p.sc = g->stride_c;
	p.w_ext = (unsigned)((long long)g->N * (g->K / 32) * 36);
	p.flags = g->flags;
	p.groups = (g->N + C::NR - 1) / C::NR;
	p.zsplit = 1;
	p.rs = g->rs;
	p.rs_sb = g->rs_sb;
	p.res = (const float *)g->res;
	for (int y = 0; y < 3; ++y)
		p.qkv_out[y] = g->qkv_out[y];
	p.qkv_S = g->qkv_S;
	p.qkv_H = g->qkv_H;
	p.qkv_dsh = g->qkv_D > 0 ? __builtin_ctz((unsigned)g->qkv_D) : 0;
	p.ln = (g->flags & S3K_A_LN) ? 1 | (g->ln_g ? 2 : 0) | (g->ln_b ? 4 : 0) : 0;
	p.ln_g = g->ln_g;
	p.ln_b = g->ln_b;
	p.att = (g->flags & S3K_A_ATT1) ? 1 : 0;
	p.att_dsh = p.att ? __builtin_ctz((unsigned)g->att_D) : 0;
	p.att_q = g->att_q;
	p.att_k = g->att_k;
	p.att_mask = g->att_mask;
	p.att_scale = g->att_scale;
	const size_t dyn = p.ln    ? (size_t)(2 * g->K + 2) * 4
			   : p.att ? (size_t)(2 * g->K + 2 * (g->K >> p.att_dsh)) * 4
				   : 0;
	dim3 grid(p.groups, g->batch);
	hipLaunchKernelGGL((q8_gemv<NT, KC>), grid, dim3(C::WV * 64), dyn, (hipStream_t)stream, p);
	return (int)hipGetLastError();
}

/* q8_gemv_tasks' conditions: a batch of weight matrices times one f32
 * row each (or one shared row), whole row groups of 16 * nt and whole
 * chunks, bias and GELU only, enough tasks to keep one workgroup per CU
 * busy. (Measured on config 4's streams against 64 rows and 16 k-blocks
 * per chunk: 64 rows in 8-block chunks with 6 in flight 4.1-4.6 TB/s,
 * 32-block chunks of 32 or 16 rows 3.5-6.1, against 5.5-6.3.) */
static bool gemv_tasks_ok(const struct s3k_gemm *g, int nt, int kc)
{
	const long long ntask = (long long)(g->N / (16 * nt)) * g->batch;
	return g->a_kind == S3K_F32 && g->M == 1 && g->batch > 1 && g->N % (16 * nt) == 0 &&
	       g->K % (kc * 32) == 0 && stream_ok(g) && s3h_settings()->gemv_tasks &&
	       !(g->flags & ~(S3K_EPI_BIAS | S3K_EPI_GELU | S3K_B_NT)) && ntask >= 256 &&
	       ntask * (g->K / (kc * 32)) < (1LL << 31); /* tasks and chunks in int */
}

/* The persistent GEMV's row groups for g: 128 rows in 8-block chunks up
 * to K = 1024, 64 rows in 16-block chunks above (config 4's streams, one
 * box: K 256 4.35 against 3.6-3.7 TB/s for 64-row tasks, K 1024
 * 5.7-5.9 against 5.5, K 4096 6.1-6.2 against 6.3; giving the 8-block
 * chunks the 16-block chunks' split of k over the waves, so that K 1024
 * kept the bits of one copy's launch, measured 5.0-5.3); 0 when it does
 * not take g. */
static int gemv_tasks_nt(const struct s3k_gemm *g)
{
	const bool k16 = g->K % 512 == 0;
	if ((!k16 || g->K <= 1024) && gemv_tasks_ok(g, 8, 8))
		return 8;
	return gemv_tasks_ok(g, 4, k16 ? 16 : 8) ? 4 : 0;
}

extern "C" int s3k_gemv_tasks_take(const struct s3k_gemm *g)
{
	return g->b_kind == S3K_Q8 && (g->flags & S3K_B_NT) && g->c_kind == S3K_F32 &&
	       g->lda % 4 == 0 && s3h_settings()->gemv_f32 && gemv_tasks_nt(g) != 0;
}

template <int NT, int KC>
static int launch_gemv_tasks_k(const struct s3k_gemm *g, void *stream)
{
	using C = StreamCfg<S3K_F32, 1, NT, KC, 144>;
	StreamArgs p;
	memset(&p, 0, sizeof p);
	p.a = (const char *)g->a;
	p.w = (const char *)g->b;
	p.c = (char *)g->c;
	p.bias = (const char *)g->bias;
	p.M = 1;
	p.N = g->N;
	p.K = g->K;
	p.lda_b = g->lda * 4;
	p.ldc = g->ldc;
	p.sa_b = g->stride_a * 4;
	p.sw_b = g->stride_b;
	p.sc = g->stride_c;
	p.w_ext = (unsigned)((long long)g->N * (g->K / 32) * 36);
	p.flags = g->flags;
	p.groups = g->N / C::NR;
	p.zsplit = 1;
	p.nbatch = g->batch;
	/* one workgroup per CU of the MI355X (256), fewer for fewer tasks */
	const long long ntask = (long long)p.groups * g->batch;
	const int grid = ntask < 256 ? (int)ntask : 256;
	/* tasks of one chunk (K = 256): all waves multiply, split over the
	 * row tiles (config 4, K 256: 4.8 against 4.35 TB/s); from two
	 * chunks on the idle half measured faster (K 1024: 5.85 against 5.7),
	 * same bits either way */
	if (g->K == KC * 32)
		hipLaunchKernelGGL((q8_gemv_tasks<NT, KC, true>), dim3(grid), dim3(C::WV * 64), 0,
				   (hipStream_t)stream, p);
	else
		hipLaunchKernelGGL((q8_gemv_tasks<NT, KC, false>), dim3(grid), dim3(C::WV * 64), 0,
				   (hipStream_t)stream, p);
	return (int)hipGetLastError();
}

/* q8_stream_tasks' conditions: a batch of weight matrices times 2-16 f16
 * activation rows each (or shared), whole 128-row groups and 256-k
 * chunks, row factors, bias and GELU only, enough tasks to keep one
 * workgroup per CU busy. */
static bool stream_tasks_ok(const struct s3k_gemm *g)
{
	const long long ntask = (long long)(g->N / 128) * g->batch;
	return g->a_kind == S3K_F16 && g->M >= 2 && g->M <= 16 && g->batch > 1 && g->N % 128 == 0 &&
	       stream_ok(g) && s3h_settings()->gemv_tasks &&
	       !(g->flags & ~(S3K_EPI_BIAS | S3K_EPI_GELU | S3K_EPI_ROWSCALE | S3K_B_NT)) &&
	       ntask >= 256 && ntask * (g->K / 256) < (1LL << 31); /* tasks and chunks in int */
}

extern "C" int s3k_stream_tasks_take(const struct s3k_gemm *g)
{
	return g->b_kind == S3K_Q8 && (g->flags & S3K_B_NT) && g->c_kind == S3K_F32 &&
	       s3k_skinny_ok(g) && stream_tasks_ok(g);
}

template <int MR>
static int launch_stream_tasks_k(const struct s3k_gemm *g, void *stream)
{
	StreamArgs p;
	memset(&p, 0, sizeof p);
	p.a = (const char *)g->a;
	p.w = (const char *)g->b;
	p.c = (char *)g->c;
	p.bias = (const char *)g->bias;
	p.M = g->M;
	p.N = g->N;
	p.K = g->K;
	p.lda_b = g->lda * 2;
	p.ldc = g->ldc;
	p.sa_b = g->stride_a * 2;
	p.sw_b = g->stride_b;
	p.sc = g->stride_c;
	p.w_ext = (unsigned)((long long)g->N * (g->K / 32) * 36);
	p.flags = g->flags;
	p.groups = g->N / 128;
	p.zsplit = 1;
	p.rs = g->rs;
	p.rs_sb = g->rs_sb;
	p.nbatch = g->batch;
	/* one workgroup per CU of the MI355X (256), fewer for fewer tasks */
	const long long ntask = (long long)p.groups * g->batch;
	const int grid = ntask < 256 ? (int)ntask : 256;
	hipLaunchKernelGGL((q8_stream_tasks<MR>), dim3(grid), dim3(1024), 0, (hipStream_t)stream, p);
	return (int)hipGetLastError();
}

template <int AK, int KC>
static int launch_stream_a(const struct s3k_gemm *g, int mr, int nt, void *stream)
{
#define S3K_SK(MR_)                                                              \
	case MR_:                                                                \
		return nt == 1 ? launch_stream_k<AK, MR_, 1, KC>(g, stream)     \
		     : nt == 2 ? launch_stream_k<AK, MR_, 2, KC>(g, stream)     \
			       : launch_stream_k<AK, MR_, 4, KC>(g, stream);
	switch (mr) {
	S3K_SK(1)
	S3K_SK(4)
	S3K_SK(8)
	S3K_SK(16)
	case 32:
		if constexpr (KC == 8)
			return nt == 1 ? launch_stream_k<AK, 32, 1, KC>(g, stream)
			     : nt == 2 ? launch_stream_k<AK, 32, 2, KC>(g, stream)
				       : launch_stream_k<AK, 32, 4, KC>(g, stream);
		return (int)hipErrorInvalidValue;
	default: return (int)hipErrorInvalidValue;
	}
#undef S3K_SK
}

/*
 * Shape choice for q8_stream: activation rows per workgroup MR (M is
 * split over ceil(M / MR) workgroups) and weight rows 16 * NT.
 *   - Many workgroups (a batch, or >= 512 workgroups of 64 rows): NT = 4
 *     and MR = M rounded up to 1/4/8/16/32; wide row groups amortize each
 *     workgroup's start and end (measured best on every config-4 shape).
 *   - One small launch, M <= 32: its time is one workgroup's latency, so
 *     rows go to as many CUs as possible (NT = 1), with M split when that
 *     evens out the bytes a CU moves. Estimate: the largest of per-CU time
 *     ceil(WGs/256) * bytes per WG / 32 B/clk (activation bytes counted
 *     at half: L2 serves them), HBM time weight bytes times
 *     (1 + (groups - 1) / 2) / 2600 B/clk (about 6.2 TB/s; each group of
 *     activation rows reads the weights) and L2 time WGs * bytes per WG /
 *     10000 B/clk; ties go to more workgroups.
 *   - One small launch, M > 32: MR = 32 with NT = 4 when that still makes
 *     128 workgroups, else MR = 16 with NT = 2.
 * SAM3_HIP_SK_CFG="mr,nt" forces a shape.
 */
static void stream_pick(const struct s3k_gemm *g, int *mr_out, int *nt_out)
{
	{
		const int mr = s3h_settings()->sk_mr, nt = s3h_settings()->sk_nt;
		if ((nt == 1 || nt == 2 || nt == 4) &&
		    (mr == 1 || mr == 4 || mr == 8 || mr == 16 || mr == 32)) {
			*mr_out = mr;
			*nt_out = nt;
			return;
		}
	}
	static const int mrs[5] = {1, 4, 8, 16, 32};
	int mr_all = 32;
	for (int i = 0; i < 5; ++i)
		if (mrs[i] >= g->M) {
			mr_all = mrs[i];
			break;
		}
	const long long z_all = (g->M + mr_all - 1) / mr_all;
	const long long groups4 = (g->N + 63) / 64;
	if (g->batch > 1 || groups4 * z_all >= 512) {
		*mr_out = mr_all;
		*nt_out = 4;
		return;
	}
	if (g->M > 32) {
		const bool wide = groups4 * z_all >= 128;
		*mr_out = wide ? 32 : 16;
		*nt_out = wide ? 4 : 2;
		return;
	}
	const int es = g->a_kind == S3K_F32 ? 4 : 2;
	const double K = g->K, N = g->N, M = g->M;
	double best_t = 1e300;
	long long best_w = 0;
	int best_mr = mr_all;
	for (int i = 0; i < 5; ++i) {
		const int mr = mrs[i];
		if (i > 0 && mrs[i - 1] >= g->M)
			break; /* a smaller MR already covers M */
		const long long z = (g->M + mr - 1) / mr;
		if (z > 8)
			continue;
		/* bytes a workgroup moves: its 16 weight rows from HBM, and its
		 * activation rows, which every workgroup of the launch reads and
		 * L2 serves, at half weight (the text encoder's qkv at 32 tokens,
		 * N 3072: 32-row tiles 13.0 us, 16 15.6, 8 18.2) */
		const double per = 16.0 * K * 1.125 + 0.5 * (mr < M ? mr : M) * K * es;
		const long long wgs = (long long)((g->N + 15) / 16) * z;
		double t = (double)((wgs + 255) / 256) * per / 32.0;
		/* HBM: each of the z activation groups reads the weights, and L2
		 * catches about half of the repeats */
		const double th = N * K * 1.125 * (1.0 + 0.5 * (double)(z - 1)) / 2600.0;
		const double tl = (double)wgs * per / 10000.0;
		t = t > th ? t : th;
		t = t > tl ? t : tl;
		if (t < best_t * 0.97 || (t <= best_t * 1.03 && wgs > best_w && wgs <= 512)) {
			best_t = t;
			best_w = wgs;
			best_mr = mr;
		}
	}
	*mr_out = best_mr;
	*nt_out = 1;
}

extern "C" int s3k_skinny_launch(const struct s3k_gemm *g, void *stream)
{
	if (((g->flags & S3K_A_LN) && !stream_ln_ok(g)) ||
	    ((g->flags & S3K_A_ATT1) && !gemv_att_ok(g)))
		return (int)hipErrorInvalidValue;
	/* the head-split stores (no RoPE) exist in q8_stream only */
	if ((g->flags & S3K_EPI_QKV) && (!stream_ok(g) || g->batch != 1 || g->qkv_rope))
		return (int)hipErrorInvalidValue;
	if (stream_ok(g)) {
		int mr, nt;
		stream_pick(g, &mr, &nt);
		/* 16-block chunks where K allows and the LDS ring stays deep
		 * enough; 8-block chunks otherwise */
		const bool k16 = g->K % 512 == 0 && mr <= 16;
		/* one f32 activation row: the f32 VALU kernel */
		if (g->a_kind == S3K_F32 && g->M == 1 && g->lda % 4 == 0 && s3h_settings()->gemv_f32) {
			/* a batch: the persistent grid over (copy, row group) tasks */
			const int tnt = gemv_tasks_nt(g);
			if (tnt == 8)
				return launch_gemv_tasks_k<8, 8>(g, stream);
			if (tnt == 4)
				return k16 ? launch_gemv_tasks_k<4, 16>(g, stream)
					   : launch_gemv_tasks_k<4, 8>(g, stream);
			if (nt == 1)
				return k16 ? launch_gemv_k<1, 16>(g, stream) : launch_gemv_k<1, 8>(g, stream);
			if (nt == 2)
				return k16 ? launch_gemv_k<2, 16>(g, stream) : launch_gemv_k<2, 8>(g, stream);
			return k16 ? launch_gemv_k<4, 16>(g, stream) : launch_gemv_k<4, 8>(g, stream);
		}
		/* a batch of a few f16 rows: the persistent grid over tasks */
		if (stream_tasks_ok(g))
			return g->M <= 8 ? launch_stream_tasks_k<8>(g, stream)
					 : launch_stream_tasks_k<16>(g, stream);
		switch (g->a_kind) {
		case S3K_F32:
			return k16 ? launch_stream_a<S3K_F32, 16>(g, mr, nt, stream)
				   : launch_stream_a<S3K_F32, 8>(g, mr, nt, stream);
		case S3K_BF16:
			return k16 ? launch_stream_a<S3K_BF16, 16>(g, mr, nt, stream)
				   : launch_stream_a<S3K_BF16, 8>(g, mr, nt, stream);
		default:
			return k16 ? launch_stream_a<S3K_F16, 16>(g, mr, nt, stream)
				   : launch_stream_a<S3K_F16, 8>(g, mr, nt, stream);
		}
	}
	if (g->batch != 1)
		return (int)hipErrorInvalidValue;
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
	p.rs = g->rs;
	p.res = (const float *)g->res;
	hipStream_t st = (hipStream_t)stream;
	switch (g->a_kind) {
	case S3K_F32:  return launch_mt<S3K_F32>(p, st);
	case S3K_BF16: return launch_mt<S3K_BF16>(p, st);
	default:       return launch_mt<S3K_F16>(p, st);
	}
}
