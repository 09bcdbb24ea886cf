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


class _Graph:
    """Stream capture into a HIP graph through the HIP runtime the library
    loaded (hipStreamBeginCapture / EndCapture / GraphInstantiate)."""

    def __init__(self, stream, record):
        import ctypes as C
        self.rt = rt = C.CDLL("libamdhip64.so.7")
        vp = C.c_void_p
        rt.hipStreamBeginCapture.argtypes = [vp, C.c_int]
        rt.hipStreamEndCapture.argtypes = [vp, C.POINTER(vp)]
        rt.hipGraphInstantiate.argtypes = [C.POINTER(vp), vp, vp, vp, C.c_size_t]
        rt.hipGraphLaunch.argtypes = [vp, vp]
        rt.hipGraphExecDestroy.argtypes = [vp]
        rt.hipGraphDestroy.argtypes = [vp]
        self.stream, self.graph, self.exec = stream, C.c_void_p(), C.c_void_p()
        assert rt.hipStreamBeginCapture(stream, 2) == 0
        try:
            record()
        finally:
            assert rt.hipStreamEndCapture(stream, C.byref(self.graph)) == 0
        assert rt.hipGraphInstantiate(C.byref(self.exec), self.graph, None, None, 0) == 0

    def launch(self):
        assert self.rt.hipGraphLaunch(self.exec, self.stream) == 0

    def close(self):
        self.rt.hipGraphExecDestroy(self.exec)
        self.rt.hipGraphDestroy(self.graph)


@pytest.mark.parametrize("M", [300, 77], ids=["mfma", "skinny"])
def test_noalloc_captured_in_a_hip_graph(M):
    """The entry point's callers run it under HIP graph capture: after one
    eager call (which looks the scratch array up), the call is captured on
    a stream and the graph replayed three times, with eager calls of
    another problem in between that overwrite the shared array. Every
    replay must give the eager call's bits."""
    import ctypes as C
    O = oracle()
    lib = hip.load()
    N, K = 512, 1024
    a = synth.randn(620 + M, (M, K))
    w = O.q8_quantize(synth.randn(621, (N, K), 0.02))
    bias = synth.randn(622, N, 0.01)
    da, dw, db = hip.DeviceBuffer.of(a), hip.DeviceBuffer.of(w), hip.DeviceBuffer.of(bias)
    c_eager, c_graph = hip.DeviceBuffer(M * N * 4), hip.DeviceBuffer(M * N * 4)
    flags = hip.BIAS | hip.GELU
    hip.check(lib.sam3_hip_matmul_q8_noalloc(abi.F32, da.ptr, dw.ptr, c_eager.ptr, M, N, K, db.ptr,
                                             flags, None), "eager")
    hip.synchronize()
    want = c_eager.download(np.float32, (M, N))
    # other work sharing the array between replays
    a2 = synth.randn(623, (64, K)) * np.float32(1e5)
    da2, dc2 = hip.DeviceBuffer.of(a2), hip.DeviceBuffer(64 * N * 4)
    sp = C.c_void_p()
    hip.check(lib.sam3_hip_stream_create(C.byref(sp)), "stream")
    g = _Graph(sp.value, lambda: hip.check(
        lib.sam3_hip_matmul_q8_noalloc(abi.F32, da.ptr, dw.ptr, c_graph.ptr, M, N, K, db.ptr,
                                       flags, sp.value), "captured"))
    try:
        for rep in range(3):
            hip.check(lib.sam3_hip_matmul_q8_noalloc(abi.F32, da2.ptr, dw.ptr, dc2.ptr, 64, N, K,
                                                     None, 0, None), "between")
            hip.synchronize()
            hip.check(lib.sam3_hip_memcpy_h2d(c_graph.ptr, np.zeros(M * N, np.float32).ctypes.data,
                                              M * N * 4), "clear")
            g.launch()
            hip.check(lib.sam3_hip_stream_synchronize(sp.value), "replay")
            got = c_graph.download(np.float32, (M, N))
            assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), f"replay {rep}"
    finally:
        g.close()
        hip.check(lib.sam3_hip_stream_destroy(sp.value), "stream")
    assert_f32_close(want, ref_q8(a, w, K, N, nt=True, bias=bias, gelu=True),
                     what="noalloc bias gelu")
