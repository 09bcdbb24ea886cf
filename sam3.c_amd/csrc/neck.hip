/*
 * neck.hip - the spatial ops of sam3.c's FPN neck besides Conv2D
 * (necks.c:330-365): ConvTranspose2D and MaxPool2D, NHWC, f32 (the
 * reference's dtype table has only F32 for both, cpu_dispatch.c:553-558).
 *
 *   convT_direct_k: one output element per thread, the reference's
 *     gather (cpu_conv_transpose2d.c:55-131): out = 0, then for each tap
 *     (kh, kw) whose input pixel ih = (oh + pad - kh) / stride (exact
 *     division) lies inside the image, out += dot(x[ih, iw, :],
 *     w[oc, kh, kw, :]) with the dot summed over channels in order;
 *     products and sums rounded separately, so the result is bit-exact.
 *   The non-overlapping case (stride = KH = KW, pad 0: the neck's 2x2
 *     upsampling) is a GEMM instead, run by the host code: every input
 *     pixel times the weight viewed as [KH*KW*OC, C] gives its KH x KW
 *     output pixels, which one permute puts in place.
 *   maxpool_k: one output element per thread, the reference's scan
 *     (cpu_maxpool2d.c:68-108): start from the window's first tap, then
 *     keep a tap only if it is greater (so a NaN first tap stays and a
 *     later NaN is skipped), taps past the image skipped.
 */
#include "gemm_common.h"

namespace s3k {

__global__ void __launch_bounds__(256) convT_direct_k(const float *x, const float *w, float *y,
						      int N, int H, int W, int C, int OC, int KH, int KW,
						      int stride, int pad, int OH, int OW)
{
	const long long t = (long long)blockIdx.x * 256 + threadIdx.x;
	const long long total = (long long)N * OH * OW * OC;
	if (t >= total)
		return;
	const int oc = (int)(t % OC);
	const long long pix = t / OC;
	const int ow = (int)(pix % OW), oh = (int)((pix / OW) % OH), n = (int)(pix / ((long long)OW * OH));
	const long long wk = (long long)KH * KW * C;
	float out = 0.0f;
	for (int kh = 0; kh < KH; ++kh) {
		const int ohf = oh + pad - kh;
		if (ohf < 0 || ohf % stride)
			continue;
		const int ih = ohf / stride;
		if (ih >= H)
			continue;
		for (int kw = 0; kw < KW; ++kw) {
			const int owf = ow + pad - kw;
			if (owf < 0 || owf % stride)
				continue;
			const int iw = owf / stride;
			if (iw >= W)
				continue;
			const float *xp = x + ((long long)(n * H + ih) * W + iw) * C;
			const float *wp = w + oc * wk + (long long)(kh * KW + kw) * C;
			float dot = 0.0f;
			for (int ci = 0; ci < C; ++ci)
				dot = add_rn(dot, mul_rn(xp[ci], wp[ci]));
			out = add_rn(out, dot);
		}
	}
	y[t] = out;
}

__global__ void __launch_bounds__(256) maxpool_k(const float *x, float *y, int N, int H, int W,
						 int C, int kernel, int stride, int OH, int OW)
{
	const long long t = (long long)blockIdx.x * 256 + threadIdx.x;
	const long long total = (long long)N * OH * OW * C;
	if (t >= total)
		return;
	const int c = (int)(t % C);
	const long long pix = t / C;
	const int ow = (int)(pix % OW), oh = (int)((pix / OW) % OH), n = (int)(pix / ((long long)OW * OH));
	const int ih0 = oh * stride, iw0 = ow * stride;
	const float *xn = x + (long long)n * H * W * C + c;
	float m = xn[((long long)ih0 * W + iw0) * C];
	for (int kh = 0; kh < kernel; ++kh) {
		const int ih = ih0 + kh;
		for (int kw = 0; kw < kernel; ++kw) {
			const int iw = iw0 + kw;
			if ((kh == 0 && kw == 0) || ih >= H || iw >= W)
				continue;
			const float v = xn[((long long)ih * W + iw) * C];
			if (v > m)
				m = v;
		}
	}
	y[t] = m;
}

/* bias [OC] repeated taps times: the bias of the [pixels, taps*OC] GEMM */
__global__ void __launch_bounds__(256) repeat_k(const float *b, float *out, int n, int times)
{
	const int t = blockIdx.x * 256 + threadIdx.x;
	if (t < n * times)
		out[t] = b[t % n];
}

} /* namespace s3k */

using namespace s3k;

static dim3 neck_grid(long long threads)
{
	return dim3((unsigned)((threads + 255) / 256));
}

extern "C" int s3k_conv_transpose_direct(const float *x, const float *w, float *y, int N, int H,
					 int W, int C, int OC, int KH, int KW, int stride, int pad,
					 int OH, int OW, void *stream)
{
	const long long total = (long long)N * OH * OW * OC;
	if (total <= 0)
		return 0;
	hipLaunchKernelGGL(convT_direct_k, neck_grid(total), dim3(256), 0, (hipStream_t)stream, x, w, y,
			   N, H, W, C, OC, KH, KW, stride, pad, OH, OW);
	return (int)hipGetLastError();
}

extern "C" int s3k_maxpool2d(const float *x, float *y, int N, int H, int W, int C, int kernel,
			     int stride, int OH, int OW, void *stream)
{
	const long long total = (long long)N * OH * OW * C;
	if (total <= 0)
		return 0;
	if (kernel <= 0 || stride <= 0 || (OH - 1) * stride >= H || (OW - 1) * stride >= W)
		return (int)hipErrorInvalidValue;
	hipLaunchKernelGGL(maxpool_k, neck_grid(total), dim3(256), 0, (hipStream_t)stream, x, y, N, H, W,
			   C, kernel, stride, OH, OW);
	return (int)hipGetLastError();
}

extern "C" int s3k_repeat_f32(const float *b, float *out, int n, int times, void *stream)
{
	if (n <= 0 || times <= 0)
		return 0;
	hipLaunchKernelGGL(repeat_k, neck_grid((long long)n * times), dim3(256), 0, (hipStream_t)stream,
			   b, out, n, times);
	return (int)hipGetLastError();
}
