/*
 * noalloc.hip - the fixed device scratch of the allocation-free Q8_0
 * matmul (sam3_hip_matmul_q8_noalloc).
 *
 * Callers that cannot allocate device memory (code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc) still
 * need somewhere to put the f16 copy of their activations. It lives in
 * `scratch`, a file-scope __device__ array: the runtime places one copy
 * on each device when it loads this code object, and the process keeps
 * it until it exits.
 *
 * In host code `scratch` names a host-side stand-in, not device memory.
 * Its device address is looked up once per device, with that device
 * current, by hipGetSymbolAddress, and kept in `dev_ptr[device]`; only
 * that address is ever handed to kernels. Every call on a device shares
 * the device's array and leaves its contents behind, so calls that
 * overlap on one device race.
 */
#include <hip/hip_runtime.h>
#include <pthread.h>

#include "s3k.h"

/* 48 MiB: the f16 activations and row factors of a 5184 x 4096 GEMM (the
 * ViT-L fc2 shape, 42.5 MB) fit. */
#define S3K_NOALLOC_BYTES (48u << 20)
#define S3K_NOALLOC_MAX_DEVICES 64

static __device__ __align__(256) unsigned char scratch[S3K_NOALLOC_BYTES];

static void *dev_ptr[S3K_NOALLOC_MAX_DEVICES];
static pthread_mutex_t dev_lock = PTHREAD_MUTEX_INITIALIZER;

extern "C" int s3k_noalloc_scratch(void **ptr, size_t *bytes)
{
	int dev = -1;
	hipError_t e = hipGetDevice(&dev);
	if (e != hipSuccess)
		return (int)e;
	if (dev < 0 || dev >= S3K_NOALLOC_MAX_DEVICES)
		return (int)hipErrorInvalidDevice;
	pthread_mutex_lock(&dev_lock);
	if (!dev_ptr[dev]) {
		void *p = nullptr;
		e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
		if (e == hipSuccess)
			dev_ptr[dev] = p;
	}
	*ptr = dev_ptr[dev];
	pthread_mutex_unlock(&dev_lock);
	*bytes = S3K_NOALLOC_BYTES;
	return e == hipSuccess && *ptr ? (int)hipSuccess : (int)(e != hipSuccess ? e : hipErrorUnknown);
}
