"""ctypes binding of libsam3hip.so, the MI355X matmul backend (C ABI in
include/sam3_hip.h).

This plays the part of sam3.c's own Python binding (bindings/python/sam3/
_lib.py loads libsam3 through cffi): it loads the shared library built
in-tree by ``make -C sam3.c_amd/csrc`` and declares every exported entry
point. There is no fallback: if the library is missing or cannot be
loaded, ``load()`` raises, so nothing silently runs elsewhere.
"""
import ctypes as C
from pathlib import Path

import numpy as np

from . import abi

LIB_PATH = Path(__file__).resolve().parent / "libsam3hip.so"

_vp, _i, _ll, _sz = C.c_void_p, C.c_int, C.c_longlong, C.c_size_t
_P = C.POINTER

# name -> (restype, argtypes); mirrors include/sam3_hip.h
SIGNATURES = {
    "sam3_hip_backend_ops": (_vp, []),
    "sam3_hip_backend_create": (_vp, [_i]),
    "sam3_hip_backend_destroy": (None, [_vp]),
    "sam3_hip_backend_set_host_dispatch": (None, [_vp, _vp, _vp]),
    "sam3_hip_backend_stream": (_vp, [_vp]),
    "sam3_hip_backend_last_stats": (None, [_vp, _vp]),
    "sam3_hip_backend_map_weights": (_i, [_vp, _vp, C.c_size_t]),
    "sam3_hip_backend_weight_ptr": (_vp, [_vp, _vp]),
    "sam3_hip_backend_fuse_rows": (_i, [_vp, _vp, _i, _vp]),
    "sam3_hip_kernel_matmul": (_i, [_vp, _vp]),
    "sam3_hip_kernel_matmul_f16": (_i, [_vp, _vp]),
    "sam3_hip_kernel_matmul_bf16": (_i, [_vp, _vp]),
    "sam3_hip_kernel_matmul_q8": (_i, [_vp, _vp]),
    "sam3_hip_kernel_sdpa": (_i, [_vp, _vp]),
    "sam3_hip_kernel_conv2d": (_i, [_vp, _vp]),
    "sam3_hip_conv2d_path": (_i, [_vp]),
    "sam3_hip_conv2d_on_path": (_i, [_i, _vp, _vp]),
    "sam3_hip_kernel_bias_add": (_i, [_vp, _vp]),
    "sam3_hip_kernel_conv_transpose2d": (_i, [_vp, _vp]),
    "sam3_hip_conv_transpose2d_path": (_i, [_vp]),
    "sam3_hip_conv_transpose2d_on_path": (_i, [_i, _vp, _vp]),
    "sam3_hip_kernel_maxpool2d": (_i, [_vp, _vp]),
    "sam3_hip_kernel_layernorm": (_i, [_vp, _vp]),
    "sam3_hip_kernel_rope": (_i, [_vp, _vp]),
    "sam3_hip_kernel_slice": (_i, [_vp, _vp]),
    "sam3_hip_kernel_transpose": (_i, [_vp, _vp]),
    "sam3_hip_kernel_reshape": (_i, [_vp]),
    "sam3_hip_kernel_cast": (_i, [_vp, _vp]),
    "sam3_hip_cast_on_path": (_i, [_i, _vp, _vp]),
    "sam3_hip_dispatch_node": (_i, [_vp, _vp]),
    "sam3_hip_matmul": (_i, [_i, _vp, _i, _vp, _i, _vp, _i, _i, _i, _vp, _i, _vp]),
    "sam3_hip_matmul_batched": (_i, [_i, _vp, _vp, _vp, _i, _i, _i, _i, _ll, _ll, _ll, _i, _vp]),
    "sam3_hip_matmul_q8_batched": (_i, [_i, _vp, _vp, _vp, _i, _i, _i, _i, _ll, _ll, _ll,
                                        _vp, _i, _vp]),
    "sam3_hip_matmul_q8_noalloc": (_i, [_i, _vp, _vp, _vp, _i, _i, _i, _vp, _i, _vp]),
    "sam3_hip_sdpa": (_i, [_i, _vp, _vp, _vp, _vp, _vp, _i, _i, _i, _i, _vp]),
    "sam3_hip_sdpa_on_path": (_i, [_i, _i, _vp, _vp, _vp, _vp, _vp, _i, _i, _i, _i, _vp]),
    "sam3_hip_q8_quantize": (_i, [_vp, _vp, _i, _vp]),
    "sam3_hip_q8_dequantize": (_i, [_vp, _vp, _i, _vp]),
    "sam3_hip_matmul_path": (_i, [_i, _i, _i, _i, _i, _i, _i]),
    "sam3_hip_matmul_on_path": (_i, [_i, _i, _vp, _i, _vp, _i, _vp, _i, _i, _i, _vp, _i, _vp]),
    "sam3_hip_device_count": (_i, []),
    "sam3_hip_set_device": (_i, [_i]),
    "sam3_hip_malloc": (_i, [_P(_vp), _sz]),
    "sam3_hip_free": (_i, [_vp]),
    "sam3_hip_memcpy_h2d": (_i, [_vp, _vp, _sz]),
    "sam3_hip_memcpy_d2h": (_i, [_vp, _vp, _sz]),
    "sam3_hip_memcpy_d2d": (_i, [_vp, _vp, _sz]),
    "sam3_hip_synchronize": (_i, []),
    "sam3_hip_stream_create": (_i, [_P(_vp)]),
    "sam3_hip_stream_destroy": (_i, [_vp]),
    "sam3_hip_stream_synchronize": (_i, [_vp]),
    "sam3_hip_event_create": (_i, [_P(_vp)]),
    "sam3_hip_event_destroy": (_i, [_vp]),
    "sam3_hip_event_record": (_i, [_vp, _vp]),
    "sam3_hip_event_elapsed_ms": (_i, [_P(C.c_float), _vp, _vp]),
    "sam3_hip_device_arch": (C.c_char_p, [_i]),
    "sam3_hip_last_error": (C.c_char_p, []),
    "sam3_hip_reload_settings": (C.c_int, []),
}

# kernel paths (sam3_hip_matmul_path)
PATH_NONE, PATH_MFMA, PATH_SKINNY, PATH_GENERIC = 0, 1, 2, 3
BIAS, GELU, B_NT = 1, 2, 4


class EvalStats(C.Structure):
    _fields_ = [(n, C.c_int) for n in ("gpu_nodes", "fused_nodes", "host_nodes",
                                       "uploads", "cache_hits", "downloads",
                                       "mapped_reads", "prep_hits", "operand_writes",
                                       "range_reruns")]


class HipError(RuntimeError):
    def __init__(self, code, what, msg):
        super().__init__(f"{what} failed: {abi.ERROR_NAMES.get(code, code)} ({msg})")
        self.code = code


_lib = None


def load(path=LIB_PATH):
    """Load libsam3hip.so once and declare its entry points. Raises if the
    library is absent (build it with `make -C sam3.c_amd/csrc`)."""
    global _lib
    if _lib is not None:
        return _lib
    if not Path(path).exists():
        raise FileNotFoundError(f"{path} not built: run `make -C sam3.c_amd/csrc`")
    lib = C.CDLL(str(path))
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _lib = lib
    return lib


def check(rc, what):
    if rc != abi.OK:
        msg = load().sam3_hip_last_error().decode(errors="replace")
        raise HipError(rc, what, msg)


# ---------------------------------------------------------------- memory
class DeviceBuffer:
    """A device allocation (hipMalloc) with numpy upload/download."""

    def __init__(self, nbytes):
        self.lib = load()
        self.nbytes = int(nbytes)
        p = C.c_void_p()
        check(self.lib.sam3_hip_malloc(C.byref(p), self.nbytes), "malloc")
        self.ptr = p.value

    @classmethod
    def of(cls, arr):
        arr = np.ascontiguousarray(arr)
        buf = cls(max(arr.nbytes, 1))
        buf.upload(arr)
        return buf

    def upload(self, arr):
        arr = np.ascontiguousarray(arr)
        assert arr.nbytes <= self.nbytes
        check(self.lib.sam3_hip_memcpy_h2d(self.ptr, arr.ctypes.data, arr.nbytes), "memcpy_h2d")

    def download(self, dtype, shape):
        out = np.empty(shape, dtype=dtype)
        check(self.lib.sam3_hip_memcpy_d2h(out.ctypes.data, self.ptr, out.nbytes), "memcpy_d2h")
        return out

    def free(self):
        if self.ptr:
            check(self.lib.sam3_hip_free(self.ptr), "free")
            self.ptr = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


def download_ptr(ptr, nbytes, dtype=np.uint8):
    """Copy nbytes at device address ptr into a new host array."""
    out = np.empty(int(nbytes) // np.dtype(dtype).itemsize, dtype=dtype)
    check(load().sam3_hip_memcpy_d2h(out.ctypes.data, ptr, out.nbytes), "memcpy_d2h")
    return out


def synchronize():
    check(load().sam3_hip_synchronize(), "synchronize")


def device_count():
    return load().sam3_hip_device_count()


class Event:
    def __init__(self):
        self.lib = load()
        p = C.c_void_p()
        check(self.lib.sam3_hip_event_create(C.byref(p)), "event_create")
        self.ptr = p.value

    def record(self, stream=None):
        check(self.lib.sam3_hip_event_record(self.ptr, stream), "event_record")

    def elapsed_ms(self, end):
        ms = C.c_float()
        check(self.lib.sam3_hip_event_elapsed_ms(C.byref(ms), self.ptr, end.ptr), "event_elapsed")
        return ms.value

    def __del__(self):
        try:
            self.lib.sam3_hip_event_destroy(self.ptr)
        except Exception:
            pass


# --------------------------------------------------------------- matmul
def matmul_dev(a_dtype, a_ptr, b_dtype, b_ptr, c_dtype, c_ptr, M, N, K, bias_ptr=None,
               flags=0, stream=None, path=0):
    lib = load()
    if path:
        rc = lib.sam3_hip_matmul_on_path(path, a_dtype, a_ptr, b_dtype, b_ptr, c_dtype, c_ptr,
                                         M, N, K, bias_ptr, flags, stream)
    else:
        rc = lib.sam3_hip_matmul(a_dtype, a_ptr, b_dtype, b_ptr, c_dtype, c_ptr, M, N, K,
                                 bias_ptr, flags, stream)
    check(rc, "sam3_hip_matmul")


_NP = {abi.F32: np.float32, abi.F16: np.uint16, abi.BF16: np.uint16}


def matmul(a, a_dtype, b, b_dtype, c_dtype, M, N, K, bias=None, flags=0, path=0):
    """Host arrays in, host array out (uploads, runs, downloads)."""
    da, db = DeviceBuffer.of(a), DeviceBuffer.of(b)
    dc = DeviceBuffer(M * N * (4 if c_dtype == abi.F32 else 2))
    dbias = DeviceBuffer.of(bias) if bias is not None else None
    matmul_dev(a_dtype, da.ptr, b_dtype, db.ptr, c_dtype, dc.ptr, M, N, K,
               dbias.ptr if dbias else None, flags, None, path)
    synchronize()
    return dc.download(_NP[c_dtype], (M, N))


def matmul_path(a_dtype, b_dtype, c_dtype, M, N, K, flags=0):
    return load().sam3_hip_matmul_path(a_dtype, b_dtype, c_dtype, M, N, K, flags)


def batched(dtype, a, b, batch, M, N, K, b_nt):
    lib = load()
    es = 4 if dtype == abi.F32 else 2
    da, db = DeviceBuffer.of(a), DeviceBuffer.of(b)
    dc = DeviceBuffer(batch * M * N * es)
    check(lib.sam3_hip_matmul_batched(dtype, da.ptr, db.ptr, dc.ptr, batch, M, N, K,
                                      M * K, K * N, M * N, B_NT if b_nt else 0, None),
          "matmul_batched")
    synchronize()
    return dc.download(_NP[dtype], (batch, M, N))


def q8_batched_dev(a_dtype, a_ptr, w_ptr, c_ptr, batch, M, N, K, stride_a, stride_w, stride_c,
                   bias_ptr=None, flags=0, stream=None):
    check(load().sam3_hip_matmul_q8_batched(a_dtype, a_ptr, w_ptr, c_ptr, batch, M, N, K,
                                            stride_a, stride_w, stride_c, bias_ptr, flags,
                                            stream), "matmul_q8_batched")


def q8_quantize(x):
    """f32 host array -> Q8_0 blocks (uint8 host array), quantized on the
    device (sam3_hip_q8_quantize)."""
    x = np.ascontiguousarray(x, np.float32).ravel()
    n = x.size
    out = np.zeros(((n + 31) // 32) * 36, np.uint8)
    if n == 0:
        return out
    dx = DeviceBuffer.of(x)
    dq = DeviceBuffer(out.nbytes)
    check(load().sam3_hip_q8_quantize(dx.ptr, dq.ptr, n, None), "q8_quantize")
    synchronize()
    out = dq.download(np.uint8, (out.nbytes,))
    dx.free(); dq.free()  # noqa: E702
    return out


def sdpa(q, k, v, mask=None, dtype=None, path=0):
    """Fused attention on the device: q [BH, Sq, D], k and v [BH, Sk, D]
    host arrays of one dtype (float32, float16, or bfloat16 bits as uint16
    with dtype=abi.BF16); mask float32 [Sq, Sk] or None. Returns out
    [BH, Sq, D] with q's element type (uint16 bits for bf16)."""
    if dtype is None:
        dtype = {np.dtype(np.float32): abi.F32, np.dtype(np.float16): abi.F16}[q.dtype]
    BH, Sq, D = q.shape
    Sk = k.shape[1]
    host_t = {abi.F32: np.float32, abi.F16: np.float16, abi.BF16: np.uint16}[dtype]
    bufs = [DeviceBuffer.of(np.ascontiguousarray(x, host_t)) for x in (q, k, v)]
    dm = DeviceBuffer.of(np.ascontiguousarray(mask, np.float32)) if mask is not None else None
    do = DeviceBuffer(max(1, BH * Sq * D) * np.dtype(host_t).itemsize)
    try:
        check(load().sam3_hip_sdpa_on_path(path, dtype, bufs[0].ptr, bufs[1].ptr, bufs[2].ptr,
                                           dm.ptr if dm else None, do.ptr, BH, Sq, Sk, D, None),
              "sdpa")
        synchronize()
        return do.download(host_t, (BH, Sq, D))
    finally:
        for b in bufs + [do] + ([dm] if dm else []):
            b.free()


def q8_dequantize(blocks, n):
    blocks = np.ascontiguousarray(blocks, np.uint8)
    if n == 0:
        return np.zeros(0, np.float32)
    db = DeviceBuffer.of(blocks)
    dx = DeviceBuffer(n * 4)
    check(load().sam3_hip_q8_dequantize(db.ptr, dx.ptr, n, None), "q8_dequantize")
    synchronize()
    out = dx.download(np.float32, (n,))
    db.free(); dx.free()  # noqa: E702
    return out


# --------------------------------------------------------------- backend
HOST_DISPATCH_FN = C.CFUNCTYPE(C.c_int, C.c_void_p, C.c_void_p)


class Backend:
    """sam3_hip_backend_create / graph_eval through the ops vtable."""

    def __init__(self, device=0):
        self.lib = load()
        self.be = self.lib.sam3_hip_backend_create(device)
        if not self.be:
            raise HipError(abi.EBACKEND, "sam3_hip_backend_create",
                           self.lib.sam3_hip_last_error().decode(errors="replace"))
        ops = C.cast(self.lib.sam3_hip_backend_ops(), C.POINTER(abi.BackendOps)).contents
        self.ops = ops
        self._host_fn = None

    def alloc_tensor(self, t):
        return self.ops.alloc_tensor(self.be, C.byref(t))

    def graph_eval(self, g):
        return self.ops.graph_eval(self.be, C.byref(g))

    def arena_reset(self):
        self.ops.arena_reset(self.be)

    def cache_invalidate(self, start, length):
        self.ops.cache_invalidate(self.be, start, length)

    def set_host_dispatch(self, fn):
        self._host_fn = HOST_DISPATCH_FN(fn) if fn else None
        self.lib.sam3_hip_backend_set_host_dispatch(self.be, self._host_fn, None)

    def map_weights(self, host_ptr, nbytes):
        """sam3_hip_backend_map_weights: copy [host_ptr, +nbytes) to HBM once."""
        return self.lib.sam3_hip_backend_map_weights(self.be, host_ptr, nbytes)

    def weight_ptr(self, host_ptr):
        return self.lib.sam3_hip_backend_weight_ptr(self.be, host_ptr)

    def fuse_rows(self, parts, out):
        """sam3_hip_backend_fuse_rows over a list of abi.Tensor headers."""
        arr = (C.POINTER(abi.Tensor) * len(parts))(*[C.pointer(t) for t in parts])
        return self.lib.sam3_hip_backend_fuse_rows(self.be, arr, len(parts), C.byref(out))

    def stats(self):
        s = EvalStats()
        self.lib.sam3_hip_backend_last_stats(self.be, C.byref(s))
        return s

    def close(self):
        if self.be:
            self.lib.sam3_hip_backend_destroy(self.be)
            self.be = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
