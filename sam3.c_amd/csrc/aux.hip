/*
 * aux.hip - the small HBM-bound kernels around the matmul:
 *
 *   - Q8_0 -> f16 unpacking for Q8 layouts the tiled GEMM does not read
 *     directly: B[K,N] with blocks over the flat index k*N+n (the
 *     reference kernel contract, cpu_matmul_q8.c:29-35) and W[N,K] with
 *     K % 32 != 0 (blocks straddle rows). Output is f16 [N,K], value
 *     q*scale rounded once to f16 (src/core/quant.c:134-165 gives q*scale).
 *   - bias add over the last dim, same-shape add, tanh-GELU and 2-D
 *     transpose, with the reference's per-op rounding
 *     (cpu_elementwise.c:28-63, cpu_add_bf16.c:62-63, cpu_gelu.c:23-38,
 *     cpu_transpose.c:355-366), used when a graph pattern cannot fuse.
 */
#include "s3k.h"
#include "s3k_dev.h"

namespace s3k {

/* One thread per 2 outputs of f16 [N,K]; element (n,k) reads block
 * lin/32 of the flat Q8 array, lin = k*N+n (KN) or n*K+k (NK). */
template <bool KN>
__global__ void __launch_bounds__(256) q8_to_f16_nk(const char *blk, uint16_t *out, int K, int N)
{
	const long long i = (long long)blockIdx.x * 256 + threadIdx.x;
	const long long tot = (long long)N * K;
	if (i >= tot)
		return;
	const int n = (int)(i / K), k = (int)(i % K);
	const long long lin = KN ? (long long)k * N + n : i;
	const char *b = blk + (lin >> 5) * 36;
	const float s = *(const float *)b;
	const float q = (float)(int)(int8_t)b[4 + (lin & 31)];
	out[i] = (uint16_t)f32_to_f16(q * s);
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

extern "C" int s3k_q8_kn_to_f16_nk(const void *blocks, void *out, int K, int N, void *stream)
{
	const long long tot = (long long)K * N;
	if (tot <= 0)
		return 0;
	hipLaunchKernelGGL(q8_to_f16_nk<true>, grid1(tot), dim3(256), 0, (hipStream_t)stream,
			   (const char *)blocks, (uint16_t *)out, K, N);
	return (int)hipGetLastError();
}

extern "C" int s3k_q8_nk_to_f16_nk(const void *blocks, void *out, int K, int N, void *stream)
{
	const long long tot = (long long)K * N;
	if (tot <= 0)
		return 0;
	hipLaunchKernelGGL(q8_to_f16_nk<false>, grid1(tot), dim3(256), 0, (hipStream_t)stream,
			   (const char *)blocks, (uint16_t *)out, K, N);
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
