"""ctypes bindings for the CPU checkers (test infrastructure only).

* ``Oracle`` wraps oracle/liboracle.so, the C11 restatement of the
  reference's CPU matmul path (oracle/sam3_oracle.c).
* ``Ref`` wraps oracle/_ref/libsam3ref.so, the reference's own CPU sources
  compiled in place by oracle/Makefile when /root/reference exists. Its
  kernels are driven exactly the way the reference tests drive them: a
  hand-built ``sam3_node`` passed to ``cpu_kernel_*(node, pool)``
  (tests/test_matmul_q8.c:66-116).
"""
import ctypes as C
import os
import sys
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[1]
sys.path.insert(0, str(ROOT / "sam3.c_amd"))

from sam3_amd import abi  # noqa: E402

ORACLE_SO = ROOT / "oracle" / "liboracle.so"
REF_SO = ROOT / "oracle" / "_ref" / "libsam3ref.so"

_vp = C.c_void_p
_i = C.c_int


def _ptr(a):
    return a.ctypes.data_as(_vp)


def _c(a, dtype):
    return np.ascontiguousarray(a, dtype=dtype)


class Oracle:
    def __init__(self, path=ORACLE_SO):
        if not Path(path).exists():
            raise FileNotFoundError(f"{path} missing: run `make -C oracle`")
        L = self.lib = C.CDLL(str(path))
        for name in ["oracle_matmul_f32", "oracle_matmul_bf16", "oracle_matmul_f16",
                     "oracle_matmul_f16_acc32", "oracle_matmul_q8", "oracle_matmul_q8_nt"]:
            getattr(L, name).argtypes = [_vp, _vp, _vp, _i, _i, _i, _i]
            getattr(L, name).restype = None
        L.oracle_q8_quantize.argtypes = [_vp, _vp, _i]
        L.oracle_q8_dequantize.argtypes = [_vp, _vp, _i]
        L.oracle_q8_block_count.argtypes = [_i]
        L.oracle_q8_nbytes.argtypes = [_i]
        L.oracle_q8_nbytes.restype = C.c_size_t
        L.oracle_f32_to_bf16.argtypes = [C.c_float]
        L.oracle_f32_to_bf16.restype = C.c_uint16
        L.oracle_f32_to_fp16.argtypes = [C.c_float]
        L.oracle_f32_to_fp16.restype = C.c_uint16
        for name in ["oracle_cast_f32_to_bf16", "oracle_cast_f32_to_fp16",
                     "oracle_cast_bf16_to_f32", "oracle_cast_fp16_to_f32",
                     "oracle_gelu_f32", "oracle_gelu_bf16", "oracle_gelu_f16"]:
            getattr(L, name).argtypes = [_vp, _vp, _i]
        for name in ["oracle_bias_add_f32", "oracle_bias_add_bf16", "oracle_bias_add_f16"]:
            getattr(L, name).argtypes = [_vp, _vp, _vp, _i, _i]
        L.oracle_transpose_u16.argtypes = [_vp, _vp, _i, _i]
        L.oracle_transpose_f32.argtypes = [_vp, _vp, _i, _i]
        L.oracle_matmul_bf16_batched.argtypes = [_vp, _vp, _vp, _i, _i, _i, _i, _i, _i]
        L.oracle_sdpa_f32.argtypes = [_vp, _vp, _vp, _vp, _vp, _i, _i, _i, _i, _i]
        for name in ["oracle_layernorm_f32", "oracle_layernorm_bf16", "oracle_layernorm_f16"]:
            getattr(L, name).argtypes = [_vp, _vp, _vp, _vp, _i, _i, _i]
        for name in ["oracle_rope_f32", "oracle_rope_bf16", "oracle_rope_f16"]:
            getattr(L, name).argtypes = [_vp, _vp, _vp, _vp, _i, _i, _i, _i]

    # ---- Q8 ----
    def q8_quantize(self, x):
        x = _c(x, np.float32).ravel()
        out = np.zeros(abi.q8_nbytes(x.size), dtype=np.uint8)
        self.lib.oracle_q8_quantize(_ptr(x), _ptr(out), x.size)
        return out

    def q8_dequantize(self, blocks, n):
        blocks = _c(blocks, np.uint8)
        out = np.empty(n, dtype=np.float32)
        self.lib.oracle_q8_dequantize(_ptr(blocks), _ptr(out), n)
        return out

    # ---- conversions ----
    def _cast(self, name, x, in_t, out_t):
        x = _c(x, in_t).ravel()
        out = np.empty(x.size, dtype=out_t)
        getattr(self.lib, name)(_ptr(x), _ptr(out), x.size)
        return out

    def f32_to_bf16(self, x):
        return self._cast("oracle_cast_f32_to_bf16", x, np.float32, np.uint16)

    def f32_to_fp16(self, x):
        return self._cast("oracle_cast_f32_to_fp16", x, np.float32, np.uint16)

    def bf16_to_f32(self, x):
        return self._cast("oracle_cast_bf16_to_f32", x, np.uint16, np.float32)

    def fp16_to_f32(self, x):
        return self._cast("oracle_cast_fp16_to_f32", x, np.uint16, np.float32)

    # ---- GEMMs ----
    def _mm(self, name, a, b, M, K, N, out_t, in_a, in_b, threads):
        a = _c(a, in_a)
        b = _c(b, in_b)
        c = np.empty((M, N), dtype=out_t)
        getattr(self.lib, name)(_ptr(a), _ptr(b), _ptr(c), M, K, N, threads)
        return c

    def matmul_f32(self, a, b, threads=1):
        (M, K), N = a.shape, b.shape[1]
        return self._mm("oracle_matmul_f32", a, b, M, K, N, np.float32, np.float32, np.float32, threads)

    def matmul_bf16(self, a, b, threads=1):
        (M, K), N = a.shape, b.shape[1]
        return self._mm("oracle_matmul_bf16", a, b, M, K, N, np.uint16, np.uint16, np.uint16, threads)

    def matmul_f16(self, a, b, threads=1):
        (M, K), N = a.shape, b.shape[1]
        return self._mm("oracle_matmul_f16", a, b, M, K, N, np.uint16, np.uint16, np.uint16, threads)

    def matmul_f16_acc32(self, a, b, threads=1):
        (M, K), N = a.shape, b.shape[1]
        return self._mm("oracle_matmul_f16_acc32", a, b, M, K, N, np.uint16, np.uint16, np.uint16, threads)

    def matmul_q8(self, a, b_blocks, K, N, threads=1):
        M = a.shape[0]
        return self._mm("oracle_matmul_q8", a, b_blocks, M, K, N, np.float32, np.float32, np.uint8, threads)

    def matmul_q8_nt(self, a, w_blocks, K, N, threads=1):
        M = a.shape[0]
        return self._mm("oracle_matmul_q8_nt", a, w_blocks, M, K, N, np.float32, np.float32, np.uint8, threads)

    def matmul_bf16_batched(self, a, b, b_nt=False, threads=1):
        batch, M, K = a.shape
        N = b.shape[1] if b_nt else b.shape[2]
        a = _c(a, np.uint16)
        b = _c(b, np.uint16)
        c = np.empty((batch, M, N), dtype=np.uint16)
        self.lib.oracle_matmul_bf16_batched(_ptr(a), _ptr(b), _ptr(c), batch, M, K, N,
                                            int(b_nt), threads)
        return c

    def transpose_u16(self, x):
        R, Cc = x.shape
        x = _c(x, np.uint16)
        out = np.empty((Cc, R), dtype=np.uint16)
        self.lib.oracle_transpose_u16(_ptr(x), _ptr(out), R, Cc)
        return out

    def transpose_f32(self, x):
        R, Cc = x.shape
        x = _c(x, np.float32)
        out = np.empty((Cc, R), dtype=np.float32)
        self.lib.oracle_transpose_f32(_ptr(x), _ptr(out), R, Cc)
        return out

    # ---- epilogues ----
    def bias_add(self, x, bias, kind):
        x = np.ascontiguousarray(x)
        rows, N = x.shape
        t = np.float32 if kind == "f32" else np.uint16
        x = _c(x, t)
        bias = _c(bias, t)
        out = np.empty_like(x)
        getattr(self.lib, f"oracle_bias_add_{kind}")(_ptr(x), _ptr(bias), _ptr(out), rows, N)
        return out

    def gelu(self, x, kind):
        t = np.float32 if kind == "f32" else np.uint16
        x = _c(x, t)
        out = np.empty_like(x)
        getattr(self.lib, f"oracle_gelu_{kind}")(_ptr(x), _ptr(out), x.size)
        return out


def _oracle_sdpa(self, q, k, v, mask=None, threads=1):
    """q [BH,Sq,D], k/v [BH,Sk,D] f32, mask [Sq,Sk] f32 or None."""
    q, k, v = _c(q, np.float32), _c(k, np.float32), _c(v, np.float32)
    BH, Sq, D = q.shape
    Sk = k.shape[1]
    m = _c(mask, np.float32) if mask is not None else None
    out = np.empty_like(q)
    self.lib.oracle_sdpa_f32(_ptr(q), _ptr(k), _ptr(v), _ptr(m) if m is not None else None,
                             _ptr(out), BH, Sq, Sk, D, threads)
    return out


Oracle.sdpa = _oracle_sdpa

_KIND_NP = {"f32": np.float32, "bf16": np.uint16, "f16": np.uint16}
_KIND_DT = {"f32": abi.F32, "bf16": abi.BF16, "f16": abi.F16}


def _oracle_layernorm(self, x, gamma=None, beta=None, kind="f32", threads=1):
    """x [..., cols] of `kind` (bf16/f16 as uint16 bits); gamma/beta [cols]."""
    t = _KIND_NP[kind]
    x = _c(x, t)
    cols = x.shape[-1]
    g = _c(gamma, t) if gamma is not None else None
    b = _c(beta, t) if beta is not None else None
    out = np.empty_like(x)
    getattr(self.lib, f"oracle_layernorm_{kind}")(_ptr(x), _ptr(g) if g is not None else None,
                                                   _ptr(b) if b is not None else None, _ptr(out),
                                                   x.size // cols, cols, threads)
    return out


def _oracle_rope(self, x, cos_t, sin_t, kind="f32"):
    """x [batch, seq, heads, hd] of `kind`; cos/sin f32 [seq, hd/2]."""
    x = _c(x, _KIND_NP[kind])
    cos_t, sin_t = _c(cos_t, np.float32), _c(sin_t, np.float32)
    out = np.empty_like(x)
    getattr(self.lib, f"oracle_rope_{kind}")(_ptr(x), _ptr(cos_t), _ptr(sin_t), _ptr(out),
                                              *x.shape)
    return out


Oracle.layernorm = _oracle_layernorm
Oracle.rope = _oracle_rope


def _oracle_conv2d(self, x, w, stride=1, ph=0, pw=None, groups=1, kind="f32", out_hw=None,
                   threads=8):
    """x [N,H,W,C], w [OC,KH,KW,C/groups] (f32 arrays, or uint16 bits for
    bf16/f16) -> y [N,OH,OW,OC]."""
    pw = ph if pw is None else pw
    N, H, W, C = x.shape
    OC, KH, KW, _ = w.shape
    OH, OW = out_hw or ((H + 2 * ph - KH) // stride + 1, (W + 2 * pw - KW) // stride + 1)
    dt = np.float32 if kind == "f32" else np.uint16
    x, w = _c(x, dt), _c(w, dt)
    y = np.zeros((N, OH, OW, OC), dt)
    fn = getattr(self.lib, f"oracle_conv2d_{kind}")
    fn.argtypes = [_vp, _vp, _vp] + [_i] * 14
    fn(_ptr(x), _ptr(w), _ptr(y), N, H, W, C, OC, KH, KW, stride, ph, pw, groups, OH, OW,
       threads)
    return y


Oracle.conv2d = _oracle_conv2d


def _oracle_conv_transpose2d(self, x, w, stride=1, pad=0, threads=8):
    """x [N,H,W,C], w [OC,KH,KW,C] f32 -> [N,OH,OW,OC]."""
    N, H, W, C = x.shape
    OC, KH, KW, _ = w.shape
    OH, OW = (H - 1) * stride - 2 * pad + KH, (W - 1) * stride - 2 * pad + KW
    x, w = _c(x, np.float32), _c(w, np.float32)
    y = np.zeros((N, OH, OW, OC), np.float32)
    fn = self.lib.oracle_conv_transpose2d_f32
    fn.argtypes = [_vp, _vp, _vp] + [_i] * 10
    fn(_ptr(x), _ptr(w), _ptr(y), N, H, W, C, OC, KH, KW, stride, pad, threads)
    return y


def _oracle_maxpool2d(self, x, kernel=2, stride=None):
    stride = stride or kernel
    N, H, W, C = x.shape
    x = _c(x, np.float32)
    y = np.zeros((N, (H - kernel) // stride + 1, (W - kernel) // stride + 1, C), np.float32)
    fn = self.lib.oracle_maxpool2d_f32
    fn.argtypes = [_vp, _vp] + [_i] * 6
    fn(_ptr(x), _ptr(y), N, H, W, C, kernel, stride)
    return y


Oracle.conv_transpose2d = _oracle_conv_transpose2d
Oracle.maxpool2d = _oracle_maxpool2d


class Ref:
    """The reference's own kernels, called through hand-built nodes."""

    def __init__(self, path=REF_SO):
        if not Path(path).exists():
            raise FileNotFoundError(str(path))
        L = self.lib = C.CDLL(str(path))
        for name in ["cpu_kernel_matmul", "cpu_kernel_matmul_bf16", "cpu_kernel_matmul_f16",
                     "cpu_kernel_matmul_q8", "cpu_kernel_add", "cpu_kernel_add_bf16",
                     "cpu_kernel_add_f16", "cpu_kernel_gelu", "cpu_kernel_gelu_bf16",
                     "cpu_kernel_gelu_f16", "cpu_kernel_cast", "cpu_kernel_transpose"]:
            getattr(L, name).argtypes = [_vp, _vp]
            getattr(L, name).restype = C.c_int
        L.cpu_kernel_sdpa.argtypes = [_vp, _vp]
        L.cpu_kernel_sdpa.restype = C.c_int
        L.cpu_dispatch_node.argtypes = [_vp, _vp, _vp]
        L.cpu_dispatch_node.restype = C.c_int
        L.sam3_q8_quantize.argtypes = [_vp, _vp, _i]
        L.sam3_q8_dequantize.argtypes = [_vp, _vp, _i]
        L.sam3_q8_block_count.argtypes = [_i]
        L.sam3_q8_nbytes.argtypes = [_i]
        L.sam3_q8_nbytes.restype = C.c_size_t
        L.sam3_threadpool_create.argtypes = [_i]
        L.sam3_threadpool_create.restype = _vp
        L.sam3_threadpool_free.argtypes = [_vp]
        self._pools = {}

    def pool(self, n):
        """None -> serial (pool NULL), 0 -> all online CPUs, n -> n threads."""
        if n is None:
            return None
        if n not in self._pools:
            self._pools[n] = self.lib.sam3_threadpool_create(n)
        return self._pools[n]

    def close(self):
        for p in self._pools.values():
            self.lib.sam3_threadpool_free(p)
        self._pools.clear()

    def q8_quantize(self, x):
        x = _c(x, np.float32).ravel()
        out = np.zeros(abi.q8_nbytes(x.size), dtype=np.uint8)
        self.lib.sam3_q8_quantize(_ptr(x), _ptr(out), x.size)
        return out

    def q8_dequantize(self, blocks, n):
        blocks = _c(blocks, np.uint8)
        out = np.empty(n, dtype=np.float32)
        self.lib.sam3_q8_dequantize(_ptr(blocks), _ptr(out), n)
        return out

    def run(self, fn, op, ins, out_dtype, out_dims, out_np_dtype, threads=None, params=(0, 0, 0, 0)):
        """ins: list of (sam3 dtype, dims, numpy array)."""
        keep = []
        tens = []
        for dt, dims, arr in ins:
            arr = np.ascontiguousarray(arr)
            keep.append(arr)
            tens.append(abi.make_tensor(dt, dims, arr.ctypes.data, arr.nbytes))
        out = np.zeros(out_dims, dtype=out_np_dtype)
        tout = abi.make_tensor(out_dtype, list(out_dims), out.ctypes.data, out.nbytes)
        node = abi.make_node(op, tens, tout, params)
        if fn == "dispatch":
            scratch = (C.c_char * 64)()
            rc = self.lib.cpu_dispatch_node(C.byref(node), C.byref(scratch), self.pool(threads))
        else:
            rc = getattr(self.lib, fn)(C.byref(node), self.pool(threads))
        return rc, out

    def conv2d(self, x, w, stride=1, ph=0, pw=None, groups=1, kind="f32", out_hw=None,
               threads=8):
        """cpu_dispatch_node on a CONV2D node (cpu_conv2d.c:296-435 and its
        twins) with a real scratch arena for the column matrix."""
        N, H, W, Cin = x.shape
        OC, KH, KW, KIC = w.shape
        p_w = ph if pw is None else pw
        OH, OW = out_hw or ((H + 2 * ph - KH) // stride + 1, (W + 2 * p_w - KW) // stride + 1)
        dt = {"f32": abi.F32, "bf16": abi.BF16, "f16": abi.F16}[kind]
        npt = np.float32 if kind == "f32" else np.uint16
        arena = _ArenaC()
        self.lib.sam3_arena_init.argtypes = [C.POINTER(_ArenaC), C.c_size_t]
        self.lib.sam3_arena_free.argtypes = [C.POINTER(_ArenaC)]
        need = OH * OW * KH * KW * KIC * 4 + KH * KW * KIC * OC * 4 + 64 * 8 * OC * 4 + (1 << 20)
        assert self.lib.sam3_arena_init(C.byref(arena), need) == 0
        try:
            keep = []
            xa, wa = _c(x, npt), _c(w, npt)
            tx = abi.make_tensor(dt, [N, H, W, Cin], xa.ctypes.data, xa.nbytes)
            tw = abi.make_tensor(dt, [OC, KH, KW, KIC], wa.ctypes.data, wa.nbytes)
            y = np.zeros((N, OH, OW, OC), npt)
            ty = abi.make_tensor(dt, [N, OH, OW, OC], y.ctypes.data, y.nbytes)
            keep += [xa, wa, tx, tw, ty]
            node = abi.make_node(abi.OP_CONV2D, [tx, tw], ty,
                                 (stride, ph, groups, 0 if pw is None else pw))
            rc = self.lib.cpu_dispatch_node(C.byref(node), C.byref(arena), self.pool(threads))
        finally:
            self.lib.sam3_arena_free(C.byref(arena))
        return rc, y

    def conv_transpose2d(self, x, w, stride=1, pad=0, threads=8):
        """cpu_dispatch_node on a CONV_TRANSPOSE2D node (f32)."""
        N, H, W, Cin = x.shape
        OC, KH, KW, _ = w.shape
        OH, OW = (H - 1) * stride - 2 * pad + KH, (W - 1) * stride - 2 * pad + KW
        xa, wa = _c(x, np.float32), _c(w, np.float32)
        y = np.zeros((N, OH, OW, OC), np.float32)
        tx = abi.make_tensor(abi.F32, [N, H, W, Cin], xa.ctypes.data, xa.nbytes)
        tw = abi.make_tensor(abi.F32, [OC, KH, KW, Cin], wa.ctypes.data, wa.nbytes)
        ty = abi.make_tensor(abi.F32, [N, OH, OW, OC], y.ctypes.data, y.nbytes)
        node = abi.make_node(abi.OP_CONV_TRANSPOSE2D, [tx, tw], ty, (stride, pad, 0, 0))
        scratch = (C.c_char * 64)()
        rc = self.lib.cpu_dispatch_node(C.byref(node), C.byref(scratch), self.pool(threads))
        return rc, y

    def maxpool2d(self, x, kernel=2, stride=0):
        N, H, W, Cin = x.shape
        k, st = kernel, stride or kernel
        xa = _c(x, np.float32)
        y = np.zeros((N, (H - k) // st + 1, (W - k) // st + 1, Cin), np.float32)
        tx = abi.make_tensor(abi.F32, [N, H, W, Cin], xa.ctypes.data, xa.nbytes)
        ty = abi.make_tensor(abi.F32, list(y.shape), y.ctypes.data, y.nbytes)
        node = abi.make_node(abi.OP_MAXPOOL2D, [tx], ty, (kernel, stride, 0, 0))
        scratch = (C.c_char * 64)()
        rc = self.lib.cpu_dispatch_node(C.byref(node), C.byref(scratch), self.pool(4))
        return rc, y

    def matmul_f32(self, a, b, threads=None):
        (M, K), N = a.shape, b.shape[1]
        rc, c = self.run("cpu_kernel_matmul", abi.OP_MATMUL,
                         [(abi.F32, [M, K], _c(a, np.float32)), (abi.F32, [K, N], _c(b, np.float32))],
                         abi.F32, (M, N), np.float32, threads)
        assert rc == 0
        return c

    def matmul_bf16(self, a, b, threads=None):
        (M, K), N = a.shape, b.shape[1]
        rc, c = self.run("cpu_kernel_matmul_bf16", abi.OP_MATMUL,
                         [(abi.BF16, [M, K], _c(a, np.uint16)), (abi.BF16, [K, N], _c(b, np.uint16))],
                         abi.BF16, (M, N), np.uint16, threads)
        assert rc == 0
        return c

    def matmul_f16(self, a, b, threads=None):
        (M, K), N = a.shape, b.shape[1]
        rc, c = self.run("cpu_kernel_matmul_f16", abi.OP_MATMUL,
                         [(abi.F16, [M, K], _c(a, np.uint16)), (abi.F16, [K, N], _c(b, np.uint16))],
                         abi.F16, (M, N), np.uint16, threads)
        assert rc == 0
        return c

    def matmul_q8(self, a, b_blocks, K, N, threads=None):
        M = a.shape[0]
        rc, c = self.run("cpu_kernel_matmul_q8", abi.OP_MATMUL,
                         [(abi.F32, [M, K], _c(a, np.float32)),
                          (abi.Q8_0, [K, N], _c(b_blocks, np.uint8))],
                         abi.F32, (M, N), np.float32, threads)
        assert rc == 0
        return c

    def cast(self, x, in_dtype, out_dtype, out_np):
        x = np.ascontiguousarray(x).ravel()
        # params[0] names the target dtype (cpu_cast.c:170-180)
        rc, out = self.run("cpu_kernel_cast", abi.OP_CAST, [(in_dtype, [x.size], x)],
                           out_dtype, (x.size,), out_np, params=(out_dtype, 0, 0, 0))
        assert rc == 0
        return out

    def add(self, x, bias, kind):
        rows, N = x.shape
        dt = {"f32": abi.F32, "bf16": abi.BF16, "f16": abi.F16}[kind]
        npt = np.float32 if kind == "f32" else np.uint16
        fn = {"f32": "cpu_kernel_add", "bf16": "cpu_kernel_add_bf16", "f16": "cpu_kernel_add_f16"}[kind]
        rc, out = self.run(fn, abi.OP_ADD, [(dt, [rows, N], _c(x, npt)), (dt, [N], _c(bias, npt))],
                           dt, (rows, N), npt)
        assert rc == 0
        return out

    def gelu(self, x, kind):
        dt = {"f32": abi.F32, "bf16": abi.BF16, "f16": abi.F16}[kind]
        npt = np.float32 if kind == "f32" else np.uint16
        fn = {"f32": "cpu_kernel_gelu", "bf16": "cpu_kernel_gelu_bf16", "f16": "cpu_kernel_gelu_f16"}[kind]
        x = _c(x, npt).ravel()
        rc, out = self.run(fn, abi.OP_GELU, [(dt, [x.size], x)], dt, (x.size,), npt)
        assert rc == 0
        return out


def _ref_sdpa(self, q, k, v, mask=None, threads=None):
    """cpu_kernel_sdpa on Q [1,BH,Sq,D] (4-D path), or [Sq,D] when BH == 1
    and `two_d` layouts are wanted by the caller (cpu_sdpa.c:216-288)."""
    q, k, v = _c(q, np.float32), _c(k, np.float32), _c(v, np.float32)
    BH, Sq, D = q.shape
    Sk = k.shape[1]
    ins = [(abi.F32, [1, BH, Sq, D], q), (abi.F32, [1, BH, Sk, D], k), (abi.F32, [1, BH, Sk, D], v)]
    if mask is not None:
        ins.append((abi.F32, [Sq, Sk], _c(mask, np.float32)))
    rc, out = self.run("cpu_kernel_sdpa", abi.OP_SDPA, ins, abi.F32, (1, BH, Sq, D), np.float32,
                       threads, params=(D, 0, 0, 0))
    assert rc == 0
    return out.reshape(BH, Sq, D)


Ref.sdpa = _ref_sdpa


def _ref_layernorm(self, x, gamma=None, beta=None, kind="f32", threads=None):
    """SAM3_OP_LAYERNORM through cpu_dispatch_node (cpu_layernorm*.c)."""
    t, dt = _KIND_NP[kind], _KIND_DT[kind]
    x = _c(x, t)
    ins = [(dt, list(x.shape), x)]
    for p in (gamma, beta):
        if p is None:
            break
        ins.append((dt, [x.shape[-1]], _c(p, t)))
    rc, out = self.run("dispatch", abi.OP_LAYERNORM, ins, dt, x.shape, t, threads)
    assert rc == 0
    return out


def _ref_rope(self, x, cos_t, sin_t, kind="f32"):
    """SAM3_OP_ROPE through cpu_dispatch_node (cpu_rope*.c)."""
    t, dt = _KIND_NP[kind], _KIND_DT[kind]
    x = _c(x, t)
    ins = [(dt, list(x.shape), x), (abi.F32, list(cos_t.shape), _c(cos_t, np.float32)),
           (abi.F32, list(sin_t.shape), _c(sin_t, np.float32))]
    rc, out = self.run("dispatch", abi.OP_ROPE, ins, dt, x.shape, t, None,
                       params=(x.shape[3], 0, 0, 0))
    assert rc == 0
    return out


def _ref_slice(self, x, dt, axis, start, end):
    """SAM3_OP_SLICE (cpu_slice.c:19-88) on a numpy array of sam3 dtype dt."""
    x = np.ascontiguousarray(x)
    dims = list(x.shape)
    dims[axis] = end - start
    rc, out = self.run("dispatch", abi.OP_SLICE, [(dt, list(x.shape), x)], dt, dims, x.dtype,
                       None, params=(axis, start, end, 0))
    assert rc == 0
    return out


def _ref_permute(self, x, dt, axes):
    """SAM3_OP_TRANSPOSE with explicit axes (cpu_transpose.c:313-387)."""
    x = np.ascontiguousarray(x)
    dims = [x.shape[a] for a in axes]
    params = tuple(axes) + (0,) * (4 - len(axes))
    rc, out = self.run("dispatch", abi.OP_TRANSPOSE, [(dt, list(x.shape), x)], dt, dims, x.dtype,
                       None, params=params)
    assert rc == 0
    return out


Ref.layernorm = _ref_layernorm
Ref.rope = _ref_rope
Ref.slice = _ref_slice
Ref.permute = _ref_permute


def have_ref():
    return REF_SO.exists()


class _ArenaC(C.Structure):
    """struct sam3_arena (src/core/alloc.h)."""
    _fields_ = [("base", _vp), ("size", C.c_size_t), ("offset", C.c_size_t), ("skip_data", _i)]


# ---- the reference's .sam3 container (src/core/weight.{h,c}) ----

class _WeightFileC(C.Structure):
    """struct sam3_weight_file (src/core/weight.h:83-94), x86-64 layout."""
    _fields_ = [("mapped", _vp), ("mapped_size", C.c_size_t), ("header", _vp), ("tensors", _vp),
                ("data_base", _vp), ("hash_table", _vp), ("hash_capacity", C.c_uint32),
                ("prefetch_thread", C.c_ulong), ("prefetch_active", _i),
                ("text_backbone", C.c_uint32)]


class _TensorInfoC(C.Structure):
    """struct weight_tensor_info (weight.h:180-186)."""
    _fields_ = [("name", C.c_char_p), ("dtype", _i), ("n_dims", _i), ("dims", _i * 4),
                ("nbytes", C.c_size_t)]


_R_OPEN = C.CFUNCTYPE(_i, _vp, C.c_char_p)
_R_N = C.CFUNCTYPE(_i, _vp)
_R_INFO = C.CFUNCTYPE(_i, _vp, _i, C.POINTER(_TensorInfoC))
_R_READ = C.CFUNCTYPE(_i, _vp, _i, _vp, C.c_size_t)
_R_CLOSE = C.CFUNCTYPE(None, _vp)


class _ReaderOpsC(C.Structure):
    """struct weight_reader_ops (weight.h:188-196)."""
    _fields_ = [("open", _R_OPEN), ("n_tensors", _R_N), ("get_tensor_info", _R_INFO),
                ("read_tensor_data", _R_READ), ("close", _R_CLOSE)]


class _ReaderC(C.Structure):
    _fields_ = [("ops", C.POINTER(_ReaderOpsC)), ("impl", _vp)]


class _ModelConfigC(C.Structure):
    """struct sam3_model_config (include/sam3/sam3_types.h:145-155)."""
    _fields_ = [(k, _i) for k in ("image_size", "encoder_dim", "decoder_dim", "n_encoder_layers",
                                  "n_decoder_layers", "backbone_type", "n_fpn_scales", "variant",
                                  "text_backbone")]


def _ref_weight_api(L):
    L.sam3_weight_write.argtypes = [C.c_char_p, C.POINTER(_ModelConfigC), C.POINTER(_ReaderC)]
    L.sam3_weight_write.restype = _i
    L.sam3_weight_open.argtypes = [C.POINTER(_WeightFileC), C.c_char_p]
    L.sam3_weight_open.restype = _i
    L.sam3_weight_close.argtypes = [C.POINTER(_WeightFileC)]
    L.sam3_weight_find.argtypes = [C.POINTER(_WeightFileC), C.c_char_p]
    L.sam3_weight_find.restype = _vp
    L.sam3_weight_to_tensor.argtypes = [C.POINTER(_WeightFileC), _vp, C.POINTER(abi.Tensor)]
    L.sam3_weight_to_tensor.restype = _i


def ref_weight_write(ref, path, tensors, config=None):
    """sam3_weight_write driven by an in-memory weight_reader the way
    tests/test_weight_q8.c:23-99 builds one: tensors are
    (name, dtype, dims, numpy array of the bytes)."""
    _ref_weight_api(ref.lib)
    arrs = [np.ascontiguousarray(a).reshape(-1).view(np.uint8) for _, _, _, a in tensors]
    names = [n.encode() for n, _, _, _ in tensors]

    def info(r, idx, out):
        _, dt, dims, _ = tensors[idx]
        out.contents.name = names[idx]
        out.contents.dtype = dt
        out.contents.n_dims = len(dims)
        for d in range(4):
            out.contents.dims[d] = dims[d] if d < len(dims) else 0
        out.contents.nbytes = arrs[idx].nbytes
        return 0

    def read(r, idx, dst, size):
        if size < arrs[idx].nbytes:
            return abi.EINVAL
        C.memmove(dst, arrs[idx].ctypes.data, arrs[idx].nbytes)
        return 0

    cbs = [_R_OPEN(lambda r, p: 0), _R_N(lambda r: len(tensors)), _R_INFO(info),
           _R_READ(read), _R_CLOSE(lambda r: None)]
    ops = _ReaderOpsC(*cbs)
    reader = _ReaderC(C.pointer(ops), None)
    cfg = _ModelConfigC(**(config or {}))
    return ref.lib.sam3_weight_write(str(path).encode(), C.byref(cfg), C.byref(reader))


class RefWeightFile:
    """sam3_weight_open / find / to_tensor / close of the reference."""

    def __init__(self, ref, path):
        _ref_weight_api(ref.lib)
        self.lib = ref.lib
        self.wf = _WeightFileC()
        self.rc = self.lib.sam3_weight_open(C.byref(self.wf), str(path).encode())

    def find(self, name):
        return self.lib.sam3_weight_find(C.byref(self.wf), name.encode())

    def to_tensor(self, desc):
        t = abi.Tensor()
        rc = self.lib.sam3_weight_to_tensor(C.byref(self.wf), desc, C.byref(t))
        return rc, t

    def close(self):
        self.lib.sam3_weight_close(C.byref(self.wf))
