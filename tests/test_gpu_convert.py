"""fp16/bf16 conversions on the GPU against sam3.c's half.h.

The CAST node kernel (sam3_hip_kernel_cast, replacing cpu_kernel_cast,
cpu_cast.c:162-215) converts by integer arithmetic and must be bit-exact
with the reference's scalar converters (half.h:58-210) on every input.
That includes NaN payloads, f16 subnormals and ties.

The GEMM epilogues round with the hardware conversion instructions
(sam3_hip_cast_on_path path 2). What this file pins about them, measured
over every 16-bit pattern and 2.6M f32 patterns:
  - v_cvt_pk_bf16_f32 is bit-exact with half.h's f32_to_bf16 everywhere,
    the quiet-NaN rule ((u >> 16) | 0x40) included;
  - v_cvt_f16_f32 / v_cvt_f32_f16 give IEEE round-to-nearest-even (numpy's
    float16 conversion) on every non-NaN input. half.h differs from that
    only for f16 subnormal results: it shifts the mantissa down (dropping
    bits) before rounding, so some values round 1 ulp lower. NaNs stay NaNs,
    but the hardware quiets signalling payloads.
The checker is the oracle's restatement of half.h (pinned in
tests/test_oracle.py), and the reference build itself when oracle/_ref
is present.
"""
import ctypes as C

import numpy as np
import pytest

from gpu_util import oracle, require_gpu
from sam3_amd import abi, hip

pytestmark = pytest.mark.gpu

SW, HW = 1, 2


@pytest.fixture(scope="module", autouse=True)
def gpu():
    require_gpu()


def gpu_cast(x, src_dt, dst_dt, dst_np, path=None):
    lib = hip.load()
    n = x.size
    isz = np.dtype(dst_np).itemsize
    ds, dd = hip.DeviceBuffer.of(x), hip.DeviceBuffer(n * isz)
    ti = abi.make_tensor(src_dt, [n], ds.ptr, x.nbytes)
    to = abi.make_tensor(dst_dt, [n], dd.ptr, n * isz)
    nd = abi.Node()
    nd.op, nd.n_inputs = abi.OP_CAST, 1
    nd.inputs[0] = C.pointer(ti)
    nd.output = C.pointer(to)
    nd.params[0] = dst_dt
    rc = (lib.sam3_hip_kernel_cast(C.byref(nd), None) if path is None
          else lib.sam3_hip_cast_on_path(path, C.byref(nd), None))
    hip.check(rc, "cast")
    hip.synchronize()
    return dd.download(dst_np, n)


def ref_cast(x, src_dt, dst_dt):
    """half.h through the oracle: f16/bf16 bits <-> f32."""
    O = oracle()
    to_f32 = {abi.F32: lambda v: v, abi.F16: O.fp16_to_f32, abi.BF16: O.bf16_to_f32}[src_dt]
    from_f32 = {abi.F32: lambda v: v, abi.F16: O.f32_to_fp16, abi.BF16: O.f32_to_bf16}[dst_dt]
    return from_f32(np.asarray(to_f32(x), np.float32))


def bits(a):
    a = np.ascontiguousarray(a)
    return a.view(np.uint32 if a.dtype.itemsize == 4 else np.uint16)


ALL16 = np.arange(65536, dtype=np.uint32).astype(np.uint16)


def f32_patterns():
    rng = np.random.default_rng(0)
    rand = rng.integers(0, 2**32, 1_000_000, dtype=np.uint64).astype(np.uint32)
    # every exponent around the f16 subnormal range, random mantissas
    e = np.arange(98, 116, dtype=np.uint32)
    sub = ((e[:, None] << 23) | rng.integers(0, 2**23, 8000, dtype=np.uint64)
           .astype(np.uint32)[None, :]).ravel()
    # exact ties for bf16 (low half 0x8000) and f16 (low 13 bits 0x1000)
    hi = rng.integers(0, 2**16, 4000, dtype=np.uint64).astype(np.uint32)
    ties = np.concatenate([(hi << 16) | 0x8000, (rand[:4000] & ~np.uint32(0x1FFF)) | 0x1000])
    special = np.array([0, 0x80000000, 0x7F800000, 0xFF800000, 0x7FC00000, 0xFFC00000,
                        0x7F800001, 0x7FBFFFFF, 0xFFC12345, 1, 0x80000001, 0x007FFFFF,
                        0x477FEFFF, 0x477FF000, 0x477FE000, 0x38800000, 0x33800000,
                        0x33000000, 0x33000001, 0x7F7FFFFF], np.uint32)
    u = np.concatenate([special, rand, sub, sub | 0x80000000, ties])
    return u.view(np.float32)


F32 = None


def f32_inputs():
    global F32
    if F32 is None:
        F32 = f32_patterns()
    return F32


CASES = [(abi.F16, abi.F32, np.float32), (abi.BF16, abi.F32, np.float32),
         (abi.F16, abi.BF16, np.uint16), (abi.BF16, abi.F16, np.uint16),
         (abi.F32, abi.F16, np.uint16), (abi.F32, abi.BF16, np.uint16)]


@pytest.mark.parametrize("src,dst,dnp", CASES)
def test_cast_bit_exact_with_half_h(src, dst, dnp):
    x = f32_inputs() if src == abi.F32 else ALL16
    got = gpu_cast(x, src, dst, dnp)
    ref = ref_cast(x, src, dst)
    bad = np.nonzero(bits(got) != bits(ref))[0]
    assert bad.size == 0, (f"{bad.size} differ, first input {bits(x)[bad[0]]:#x}: "
                           f"{bits(ref)[bad[0]]:#x} expected, {bits(got)[bad[0]]:#x} got")


def test_cast_matches_reference_build():
    """The same against cpu_kernel_cast itself (oracle/_ref), where built."""
    from oracle_bind import Ref, have_ref
    if not have_ref():
        pytest.skip("oracle/_ref not built")
    R = Ref()
    for src, dst, dnp in CASES:
        x = f32_inputs() if src == abi.F32 else ALL16
        assert np.array_equal(bits(gpu_cast(x, src, dst, dnp)), bits(R.cast(x, src, dst, dnp)))


def _is_nan16(b):
    return ((b & 0x7C00) == 0x7C00) & ((b & 0x3FF) != 0)


def test_hardware_bf16_conversion_bit_exact():
    """v_cvt_pk_bf16_f32, which rounds every bf16 GEMM output, is half.h's
    f32_to_bf16 bit for bit (RNE, NaN -> (u >> 16) | 0x40)."""
    x = f32_inputs()
    assert np.array_equal(bits(gpu_cast(x, abi.F32, abi.BF16, np.uint16, HW)),
                          bits(ref_cast(x, abi.F32, abi.BF16)))
    assert np.array_equal(bits(gpu_cast(ALL16, abi.F16, abi.BF16, np.uint16, HW)),
                          bits(ref_cast(ALL16, abi.F16, abi.BF16)))
    assert np.array_equal(bits(gpu_cast(ALL16, abi.BF16, abi.F32, np.float32, HW)),
                          bits(ref_cast(ALL16, abi.BF16, abi.F32)))


def test_hardware_f16_conversion_is_ieee_rne():
    x = f32_inputs()
    xb = bits(x)
    nan_in = ((xb & 0x7F800000) == 0x7F800000) & ((xb & 0x7FFFFF) != 0)
    hw = bits(gpu_cast(x, abi.F32, abi.F16, np.uint16, HW))
    ref = bits(ref_cast(x, abi.F32, abi.F16))
    with np.errstate(over="ignore"):
        ieee = x.astype(np.float16).view(np.uint16)
    # every non-NaN input: the correctly rounded f16
    assert np.array_equal(hw[~nan_in], ieee[~nan_in])
    assert _is_nan16(hw[nan_in]).all() and ((hw[nan_in] ^ ref[nan_in]) & 0x8000 == 0).all()
    # half.h agrees except on f16 subnormal results, one ulp below
    diff = np.nonzero((hw != ref) & ~nan_in)[0]
    assert ((ref[diff] & 0x7C00) == 0).all(), "half.h differs outside the subnormal range"
    assert ((hw[diff].astype(np.int32) - ref[diff].astype(np.int32)) == 1).all()
    # f16 -> f32 and bf16 -> f16: exact except NaN payload quieting
    for src, dst, dnp in [(abi.F16, abi.F32, np.float32), (abi.BF16, abi.F16, np.uint16)]:
        g, r = bits(gpu_cast(ALL16, src, dst, dnp, HW)), bits(ref_cast(ALL16, src, dst))
        src_nan = _is_nan16(ALL16) if src == abi.F16 else \
            ((ALL16 & 0x7F80) == 0x7F80) & ((ALL16 & 0x7F) != 0)
        assert np.array_equal(g[~src_nan], r[~src_nan])


def test_cast_node_contract():
    """cpu_kernel_cast's checks: params[0] must be the output dtype
    (EINVAL), same dtype copies, non-float pairs are EDTYPE."""
    lib = hip.load()
    x = np.arange(8, dtype=np.float32)
    ds, dd = hip.DeviceBuffer.of(x), hip.DeviceBuffer(32)

    def node(src_dt, dst_dt, param):
        ti = abi.make_tensor(src_dt, [8], ds.ptr, 32)
        to = abi.make_tensor(dst_dt, [8], dd.ptr, 32)
        nd = abi.Node()
        nd.op, nd.n_inputs = abi.OP_CAST, 1
        nd.inputs[0] = C.pointer(ti)
        nd.output = C.pointer(to)
        nd.params[0] = param
        return nd, ti, to

    nd, *_ = node(abi.F32, abi.F16, abi.BF16)
    assert lib.sam3_hip_kernel_cast(C.byref(nd), None) == abi.EINVAL
    nd, *_ = node(abi.F32, abi.F32, abi.F32)
    assert lib.sam3_hip_kernel_cast(C.byref(nd), None) == abi.OK
    hip.synchronize()
    assert np.array_equal(dd.download(np.float32, 8), x)
    nd, *_ = node(abi.I32, abi.F32, abi.F32)
    assert lib.sam3_hip_kernel_cast(C.byref(nd), None) == abi.EDTYPE
    # through the dispatcher, as cpu_dispatch_node routes SAM3_OP_CAST
    nd, *_ = node(abi.F32, abi.BF16, abi.BF16)
    assert lib.sam3_hip_dispatch_node(C.byref(nd), None) == abi.OK
    hip.synchronize()
    assert np.array_equal(dd.download(np.uint16, 8), oracle().f32_to_bf16(x))
