"""sam3_hip_matmul_q8_noalloc: the Q8_0 matmul that allocates nothing.

It runs the kernels of sam3_hip_matmul with the f16 activation copy in
the library's fixed per-device scratch array and never expands the
weight. With per-call expansion off (SAM3_HIP_Q8_EXPAND=0) sam3_hip_matmul
runs the same kernels, so the outputs must have the same bits, call after
call (the array keeps the previous call's contents). At the default
settings sam3_hip_matmul expands the weight from M = 3072 on (q*scale
rounded to f16 once, not per k-step), and the two agree within the f32
tolerance. Both must match the oracle within it.
"""
import numpy as np
import pytest

from gpu_util import assert_f32_close, bf16_to_f32, oracle, ref_q8, require_gpu
from sam3_amd import abi, hip, synth

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def gpu():
    require_gpu()


def _run_both(a, a_dt, w, M, N, K, bias=None, flags=0):
    """(no-alloc result, sam3_hip_matmul result) on the same device inputs."""
    lib = hip.load()
    da, dw = hip.DeviceBuffer.of(a), hip.DeviceBuffer.of(w)
    db = hip.DeviceBuffer.of(bias) if bias is not None else None
    c1, c2 = hip.DeviceBuffer(M * N * 4), hip.DeviceBuffer(M * N * 4)
    bp = db.ptr if db is not None else None
    hip.check(lib.sam3_hip_matmul_q8_noalloc(a_dt, da.ptr, dw.ptr, c1.ptr, M, N, K, bp, flags,
                                             None), "matmul_q8_noalloc")
    hip.check(lib.sam3_hip_matmul(a_dt, da.ptr, abi.Q8_0, dw.ptr, abi.F32, c2.ptr, M, N, K, bp,
                                  flags | hip.B_NT, None), "matmul")
    hip.synchronize()
    return c1.download(np.float32, (M, N)), c2.download(np.float32, (M, N))


def _rows(M, n=40, seed=3):
    rng = np.random.default_rng(seed)
    return np.unique(np.concatenate([[0, M - 1], rng.integers(0, M, n)]))


def test_noalloc_matches_matmul_twice_second_smaller(env):
    O = oracle()
    # call 1: config 1 (f32 activations [5184, 1024] x Q8_0 [1024, 1024])
    M, N, K = 5184, 1024, 1024
    a = synth.randn(600, (M, K))
    w = O.q8_quantize(synth.randn(601, (N, K), 0.02))
    got, expanded = _run_both(a, abi.F32, w, M, N, K)
    r = _rows(M)
    ref = ref_q8(a[r], w, K, N, nt=True)
    assert_f32_close(got[r], ref, what="noalloc config 1")
    assert_f32_close(expanded[r], ref, what="matmul config 1 (expanded weight)")
    env.set("SAM3_HIP_Q8_EXPAND", 0)
    got, want = _run_both(a, abi.F32, w, M, N, K)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    # call 2: a smaller problem on the GEMV path, activations past f16
    M, N, K = 77, 512, 1024
    a = synth.randn(602, (M, K)) * np.float32(1e6)
    w = O.q8_quantize(synth.randn(603, (N, K), 0.02))
    got, want = _run_both(a, abi.F32, w, M, N, K)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    assert_f32_close(got, ref_q8(a, w, K, N, nt=True), what="noalloc skinny")


def test_noalloc_bf16_bias_gelu():
    O = oracle()
    M, N, K = 512, 768, 1024
    a = O.f32_to_bf16(synth.randn(610, (M, K))).reshape(M, K)
    w = O.q8_quantize(synth.randn(611, (N, K), 0.02))
    bias = synth.randn(612, N, 0.01)
    got, want = _run_both(a, abi.BF16, w, M, N, K, bias, hip.BIAS | hip.GELU)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    ref = ref_q8(bf16_to_f32(a).reshape(M, K), w, K, N, nt=True, bias=bias, gelu=True)
    assert_f32_close(got, ref, what="noalloc bf16 bias gelu")


def test_noalloc_rejects_oversize_before_launch():
    """M * K * 2 bytes past the 48 MiB array: SAM3_EINVAL, output untouched."""
    lib = hip.load()
    M, N, K = 8192, 64, 4096
    out = np.full(M * N, 7.0, np.float32)
    dc = hip.DeviceBuffer.of(out)
    da = hip.DeviceBuffer(M * K * 4)
    dw = hip.DeviceBuffer(N * (K // 32) * 36)
    rc = lib.sam3_hip_matmul_q8_noalloc(abi.F32, da.ptr, dw.ptr, dc.ptr, M, N, K, None, 0, None)
    assert rc == abi.EINVAL
    assert b"scratch" in lib.sam3_hip_last_error()
    hip.synchronize()
    assert np.array_equal(dc.download(np.float32, M * N), out)
    # K not whole Q8_0 blocks
    assert lib.sam3_hip_matmul_q8_noalloc(abi.F32, da.ptr, dw.ptr, dc.ptr, 4, 4, 48, None, 0,
                                          None) == abi.EINVAL
