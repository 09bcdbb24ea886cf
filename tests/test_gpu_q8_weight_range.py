"""Q8_0 weights with small block scales, on every Q8 path of the GPU.

The reference forms (a * q) * scale in f32 for any scale
(cpu_matmul_q8.c:124-131), and its scale amax / 127 can be arbitrarily
small (quant.c:91). The MFMA paths here feed the matrix cores f16 weights:
q * scale formed in f32 and rounded to f16 (the expansion, the unpacking
and the in-pipeline dequantization), or q times the scale rounded to f16.
A weight row whose values lie far below the f16 normal range would lose
its bits there, so each weight row gets a power-of-two factor that brings
its largest |q * scale| into [2^14, 2^15) when it lies outside
[2^-6, 2^15); the f32 epilogue multiplies the row's output column by the
factor again, which is exact.

Weights here: N(0, 1e-3), N(0, 1e-5), and N(0, 0.02) with every seventh
block shrunk to amax 1e-7 and whole rows of amax 1e-7 among ordinary
ones. Every output row and every output column is checked on its own
scale against the oracle's f32 product: max |g - r| <= 1e-3 * max |r|
over that row or column, so a tiny weight row (a tiny output column)
cannot hide under the others.
"""
import numpy as np
import pytest

from gpu_util import assert_f32_close, bf16_to_f32, oracle, ref_q8, require_gpu
from sam3_amd import abi, graph, hip, synth

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def gpu():
    require_gpu()


def small_weights(kind, seed, shape):
    """f32 source of the Q8_0 weight, flat blocks of 32 along the last
    axis's row-major order (the layout q8_quantize blocks)."""
    if kind == "s1e-3":
        return synth.randn(seed, shape, 1e-3)
    if kind == "s1e-5":
        return synth.randn(seed, shape, 1e-5)
    assert kind == "mixed"
    w = synth.randn(seed, shape, 0.02)
    flat = w.reshape(-1)
    nb = flat.size // 32
    blocks = flat[:nb * 32].reshape(nb, 32)
    amax = np.abs(blocks).max(axis=1, keepdims=True)
    pick = np.arange(nb) % 7 == 3
    blocks[pick] *= np.float32(1e-7) / amax[pick]
    rows = w.reshape(shape[0], -1)
    for r in range(1, shape[0], 11):
        rows[r] *= np.float32(1e-7) / np.abs(rows[r]).max()
    return w


def wrows(w_blocks, K, N, nt=True):
    """The dequantized weight as float64 rows [N, K]."""
    d = oracle().q8_dequantize(w_blocks, K * N).astype(np.float64)
    return d.reshape(N, K) if nt else d.reshape(K, N).T


def check(got, ref, a, wd, rtol=1e-3, what=""):
    """Each output row and each output column on its own scale. A row's
    scale is its largest |ref|; a column's is the larger of its largest
    |ref| and 3 * ||w_n|| * max_m ||a_m|| / sqrt(K), about the largest
    |output| of that weight row over a few hundred unit-variance rows. So
    a column of one or a few outputs that cancel to near zero is held to
    the bound a few hundred rows would give it (its f16 rounding of a
    cannot meet a bound relative to one small value), while a tiny weight
    row still gets a tiny scale."""
    g = np.asarray(got, np.float64)
    r = np.asarray(ref, np.float64)
    assert g.shape == r.shape
    assert np.isfinite(g).all(), f"{what}: non-finite outputs"
    err = np.abs(g - r)
    a = np.asarray(a, np.float64)
    K = a.shape[1]
    typ = 3 * np.linalg.norm(wd, axis=1) * np.linalg.norm(a, axis=1).max() / np.sqrt(K)
    scales = (np.abs(r).max(axis=1), np.maximum(np.abs(r).max(axis=0), typ))
    for axis, name, s in ((1, "row", scales[0]), (0, "column", scales[1])):
        e = err.max(axis=axis)
        bad = np.nonzero(e > rtol * s)[0]
        assert bad.size == 0, (f"{what}: {bad.size} {name}s off; {name} {bad[0]} "
                               f"(scale {s[bad[0]]:.3g}) error {e[bad[0]]:.3g}")


KINDS = ["s1e-3", "s1e-5", "mixed"]


@pytest.mark.parametrize("kind", KINDS)
@pytest.mark.parametrize("M,K,N,want", [
    (300, 1024, 512, hip.PATH_MFMA),     # direct-to-LDS Q8 GEMM
    (3072, 1024, 256, hip.PATH_MFMA),    # per-call expansion (cast + expand launch)
    (300, 96, 256, hip.PATH_MFMA),       # K % 64 != 0: register-staged Q8 loader
    (1, 1024, 512, hip.PATH_SKINNY),     # q8_stream
    (77, 96, 256, hip.PATH_SKINNY),      # q8_skinny
])
def test_f32_activations_small_weights_nt(kind, M, K, N, want):
    O = oracle()
    a = synth.randn(700 + M, (M, K))
    w = O.q8_quantize(small_weights(kind, 701 + K, (N, K)))
    assert hip.matmul_path(abi.F32, abi.Q8_0, abi.F32, M, N, K, hip.B_NT) == want
    c = hip.matmul(a, abi.F32, w, abi.Q8_0, abi.F32, M, N, K, flags=hip.B_NT)
    check(c, ref_q8(a, w, K, N, nt=True), a, wrows(w, K, N), what=f"{kind} M={M} K={K} N={N}")


@pytest.mark.parametrize("kind", KINDS)
def test_bf16_activations_small_weights_forced_expansion(kind, env):
    """bf16 x Q8_0 (config 3's pairing), with the expansion forced at a
    small M (the f16 copy of the weight made by the expansion kernel)
    and with it off (the direct kernel)."""
    O = oracle()
    M, K, N = 256, 1024, 384
    a = O.f32_to_bf16(synth.randn(710, (M, K))).reshape(M, K)
    w = O.q8_quantize(small_weights(kind, 711, (N, K)))
    a32 = bf16_to_f32(a).reshape(M, K)
    ref = ref_q8(a32, w, K, N, nt=True)
    for mode in (1, 0):
        env.set("SAM3_HIP_Q8_EXPAND", mode)
        c = hip.matmul(a, abi.BF16, w, abi.Q8_0, abi.F32, M, N, K, flags=hip.B_NT)
        check(c, ref, a32, wrows(w, K, N), what=f"{kind} bf16 expand={mode}")


@pytest.mark.parametrize("kind", KINDS)
def test_unpacked_layouts_small_weights(kind):
    """The reference's kernel contract (blocks along N of [K, N]) and [N, K]
    rows that split blocks (K % 32 != 0): both unpacked to f16 [N, K]."""
    O = oracle()
    M, K, N = 256, 512, 384
    a = synth.randn(720, (M, K))
    w = O.q8_quantize(small_weights(kind, 721, (K, N)))
    check(hip.matmul(a, abi.F32, w, abi.Q8_0, abi.F32, M, N, K), ref_q8(a, w, K, N, nt=False),
          a, wrows(w, K, N, nt=False), what=f"{kind} KN")
    M, K, N = 300, 80, 96
    a = synth.randn(722, (M, K))
    w = O.q8_quantize(small_weights(kind, 723, (N, K)))
    check(hip.matmul(a, abi.F32, w, abi.Q8_0, abi.F32, M, N, K, flags=hip.B_NT),
          ref_q8(a, w, K, N, nt=True), a, wrows(w, K, N),
          what=f"{kind} NK straddling")


@pytest.mark.parametrize("kind", KINDS)
@pytest.mark.parametrize("M", [1, 32])
def test_batched_small_weights(kind, M):
    """sam3_hip_matmul_q8_batched over distinct weights with shared f32
    activations: M = 1 on q8_stream, M = 32 on the tiled Q8 GEMM."""
    O = oracle()
    batch, K, N = 4, 1024, 256
    a = synth.randn(730 + M, (M, K))
    ws = [O.q8_quantize(small_weights(kind, 731 + s, (N, K))) for s in range(batch)]
    da, dw = hip.DeviceBuffer.of(a), hip.DeviceBuffer.of(np.concatenate(ws))
    dc = hip.DeviceBuffer(batch * M * N * 4)
    hip.check(hip.load().sam3_hip_matmul_q8_batched(abi.F32, da.ptr, dw.ptr, dc.ptr, batch, M, N,
                                                     K, 0, ws[0].nbytes, M * N, None, 0, None),
              "q8_batched")
    hip.synchronize()
    c = dc.download(np.float32, (batch, M, N))
    for s in range(batch):
        check(c[s], ref_q8(a, ws[s], K, N, nt=True), a, wrows(ws[s], K, N),
              what=f"{kind} slice {s} M={M}")


@pytest.mark.parametrize("kind", KINDS)
def test_noalloc_small_weights(kind):
    O = oracle()
    M, K, N = 300, 1024, 512
    a = synth.randn(740, (M, K))
    w = O.q8_quantize(small_weights(kind, 741, (N, K)))
    da, dw = hip.DeviceBuffer.of(a), hip.DeviceBuffer.of(w)
    dc = hip.DeviceBuffer(M * N * 4)
    hip.check(hip.load().sam3_hip_matmul_q8_noalloc(abi.F32, da.ptr, dw.ptr, dc.ptr, M, N, K, None,
                                                     0, None), "matmul_q8_noalloc")
    hip.synchronize()
    check(dc.download(np.float32, (M, N)), ref_q8(a, w, K, N, nt=True), a, wrows(w, K, N),
          what=f"{kind} noalloc")


def _out(t, shape):
    import ctypes as C
    return np.ctypeslib.as_array(C.cast(t.data, C.POINTER(C.c_float)), shape=shape).copy()


@pytest.mark.parametrize("kind", KINDS)
def test_graph_small_weights_twice(kind):
    """LN -> Q8_0 linear inside graph_eval (the weight is a constant
    input: its prepared form is made once and kept), evaluated twice on
    one backend so the second eval reads the kept form."""
    O = oracle()
    M, K, N = 512, 1024, 512
    x = synth.randn(750, (M, K))
    gamma, beta = synth.randn(751, (K,)), synth.randn(752, (K,), 0.1)
    wq = O.q8_quantize(small_weights(kind, 753, (N, K)))
    G = graph.Graph()
    t = G.layernorm(G.tensor(abi.F32, (M, K), x), G.tensor(abi.F32, (K,), gamma),
                    G.tensor(abi.F32, (K,), beta))
    y = G.linear(t, G.tensor(abi.Q8_0, (N, K), wq))
    ln = O.layernorm(x, gamma, beta)
    ref = ref_q8(ln, wq, K, N, nt=True)
    be = hip.Backend(0)
    try:
        for ev in range(2):
            assert be.graph_eval(G.g) == abi.OK
            check(_out(y, (M, N)), ref, ln, wrows(wq, K, N), what=f"{kind} graph eval {ev}")
    finally:
        be.close()


@pytest.mark.parametrize("cfg,M", [(2, 300), (15, 300), (7, 20), (9, 77)])
def test_q8_kernel_found_weight_factors_same_bits(env, cfg, M):
    """Per-call weight-row factors found by the Q8 GEMM itself
    (S3K_Q8_WAUTO: a k-loop with factor 1, run again with the factors when
    a row of the tile needs one) give the bits of the factors computed by
    a pass of their own (SAM3_HIP_Q8_WAUTO=0), rows of tiny and of huge
    scales among ordinary ones, for the 128x128, the pipelined and the
    small-M tiles; both within the f32 bound of the oracle."""
    O = oracle()
    N, K = 300, 512
    wf = synth.randn(800 + cfg, (N, K), 0.02)
    wf[3] *= np.float32(1e-7)
    wf[150] *= np.float32(1e5)
    wf[299] *= np.float32(3e-6)
    w = O.q8_quantize(wf)
    a = O.f32_to_fp16(synth.randn(801, (M, K))).reshape(M, K)
    env.set("SAM3_HIP_Q8_EXPAND", 0)
    env.set("SAM3_HIP_DLQ8_CFG", cfg)
    outs = []
    for mode in (1, 0):
        env.set("SAM3_HIP_Q8_WAUTO", mode)
        outs.append(hip.matmul(a, abi.F16, w, abi.Q8_0, abi.F32, M, N, K, flags=hip.B_NT,
                               path=hip.PATH_MFMA))
    assert np.array_equal(outs[0].view(np.uint32), outs[1].view(np.uint32))
    ref = ref_q8(O.fp16_to_f32(a).reshape(M, K), w, K, N, nt=True)
    for r in (3, 150, 299):
        assert_f32_close(outs[0][:, r:r + 1], ref[:, r:r + 1], what=f"row {r}")
    rest = np.setdiff1d(np.arange(N), [3, 150, 299])
    assert_f32_close(outs[0][:, rest], ref[:, rest], what=f"cfg {cfg}")
