"""Shared helpers of the GPU parity tests: tolerance checks and the
oracle-side compositions the HIP results are compared with."""
import numpy as np

from oracle_bind import Oracle
from sam3_amd import abi, hip

_O = None


def oracle():
    global _O
    if _O is None:
        _O = Oracle()
    return _O


def bf16_to_f32(bits):
    return (np.asarray(bits, np.uint16).astype(np.uint32) << 16).view(np.float32)


def f16_to_f32(bits):
    return np.asarray(bits, np.uint16).view(np.float16).astype(np.float32)


def ulp_bf16(x):
    """Spacing of bf16 numbers at |x| (2^(e-7)), floor at the smallest normal."""
    e = np.floor(np.log2(np.maximum(np.abs(x), 2.0 ** -126)))
    return 2.0 ** (e - 7)


def ulp_f16(x):
    e = np.floor(np.log2(np.maximum(np.abs(x), 2.0 ** -14)))
    return 2.0 ** (e - 10)


def assert_f32_close(got, ref, rtol=1e-3, floor=2e-3, what=""):
    """f32 outputs against the reference, three conditions:
      1. max relative error (normwise) max|g - r| / max|r| <= rtol: the
         north-star bound "max relative error 1e-3";
      2. elementwise |g - r| <= rtol*|r| + floor*rms(r): the reference's
         atol + rtol*|expected| form (tests/test_helpers.h:89-108) with
         the atol tied to the output's scale, since a reordered sum has
         unbounded relative error where the output crosses zero;
      3. cosine >= 0.9999 (tests/test_metal.c:252).
    The f16-operand Q8 GEMM rounds A and q*scale to f16 (2^-11 each), an
    expected normwise error near 3e-4."""
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    assert got.shape == ref.shape
    assert np.all(np.isfinite(got)), f"{what}: non-finite output"
    if ref.size == 0:
        return
    err = np.abs(got - ref)
    amax = max(np.abs(ref).max(), 1e-30)
    assert err.max() <= rtol * amax, f"{what}: max normwise error {err.max() / amax:.3e} > {rtol}"
    rms = np.sqrt(np.mean(ref ** 2))
    lim = rtol * np.abs(ref) + floor * rms
    bad = err > lim
    assert not bad.any(), (f"{what}: {bad.sum()} / {bad.size} outside elementwise bound; "
                           f"max err {err.max():.3e}, max normwise {err.max() / amax:.3e}")
    if ref.size > 1 and rms > 0:
        cos = (got * ref).sum() / (np.linalg.norm(got) * np.linalg.norm(ref))
        assert cos >= 0.9999, f"{what}: cosine {cos}"


def assert_bf16_close(got_bits, ref_bits, atol=2e-2, what=""):
    """bf16 outputs: |g - r| <= max(atol, 1 bf16 ulp of r). atol 2e-2 is
    the bf16 bound of tests/test_matmul_bf16.c:113; the ulp term covers a
    different f32 summation order flipping the final rounding."""
    g, r = bf16_to_f32(got_bits).astype(np.float64), bf16_to_f32(ref_bits).astype(np.float64)
    err = np.abs(g - r)
    lim = np.maximum(atol, ulp_bf16(r))
    bad = err > lim
    assert not bad.any(), f"{what}: {bad.sum()} / {bad.size} bf16 outputs off; max err {err.max():.3e}"


def assert_f16_close(got_bits, ref_bits, atol=5e-3, what=""):
    """f16 outputs: |g - r| <= max(atol, 2 f16 ulps of r); atol 5e-3 is the
    f16 bound of tests/test_matmul_f16.c."""
    g, r = f16_to_f32(got_bits).astype(np.float64), f16_to_f32(ref_bits).astype(np.float64)
    err = np.abs(g - r)
    lim = np.maximum(atol, 2 * ulp_f16(r))
    bad = err > lim
    assert not bad.any(), f"{what}: {bad.sum()} / {bad.size} f16 outputs off; max err {err.max():.3e}"


def ref_linear(kind, a, b, bias=None, gelu=False, b_nt=False, threads=8):
    """Oracle composition of MATMUL -> ADD(bias) -> GELU with the
    reference's rounding after each node. kind: 'f32', 'bf16', 'f16'
    (f16 uses the f32-accumulate restatement)."""
    O = oracle()
    if b_nt:
        b = np.ascontiguousarray(b.T)
    if kind == "f32":
        c = O.matmul_f32(a, b, threads)
    elif kind == "bf16":
        c = O.matmul_bf16(a, b, threads)
    else:
        c = O.matmul_f16_acc32(a, b, threads)
    if bias is not None:
        c = O.bias_add(c, bias, kind)
    if gelu:
        c = O.gelu(c, kind).reshape(c.shape)
    return c


def ref_q8(a_f32, w_blocks, K, N, nt, bias=None, gelu=False, threads=8):
    O = oracle()
    c = O.matmul_q8_nt(a_f32, w_blocks, K, N, threads) if nt else \
        O.matmul_q8(a_f32, w_blocks, K, N, threads)
    if bias is not None:
        c = O.bias_add(c, bias, "f32")
    if gelu:
        c = O.gelu(c, "f32").reshape(c.shape)
    return c


def require_gpu():
    n = hip.device_count()
    assert n > 0, "no HIP device visible"
    arch = hip.load().sam3_hip_device_arch(0).decode()
    assert arch.startswith("gfx950"), f"expected gfx950, got {arch}"
