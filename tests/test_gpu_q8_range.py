"""Q8_0 matmuls with activations outside the f16 range, on the GPU.

The reference computes the Q8_0 matmul in f32 (cpu_matmul_q8.c:124-131):
c += (a * q) * scale. The MFMA and GEMV kernels here multiply f16
activations. So before any kernel that rounds f32/bf16 activations to
f16, the backend copies them row by row with a power-of-two factor
(s3k_cast_f16_rows). The factor is undone in the f32 epilogue. Inside
graph_eval, producers that write the f16 operand directly (LayerNorm,
permute, GEMM epilogue) flag values the f16 copy cannot hold, and the graph
runs again on f32 operands.

Each row is checked on its own scale against the oracle's f32 product:
max |g - r| <= 1e-3 * max |r| per row. Rows span 1e-30 .. 1e30, so a
tensor-wide norm would hide a wrong small row.
"""
import numpy as np
import pytest

from gpu_util import bf16_to_f32, oracle, ref_q8, require_gpu
from sam3_amd import abi, graph, hip, synth

pytestmark = pytest.mark.gpu

# row magnitudes: in range, past f16 (1e5, 1e6), far past (1e30), tiny
# (1e-6, 1e-12, 1e-30) and an all-zero row
SCALES = np.float32([1.0, 1e6, 3.0, 1e-6, 1e30, 0.0, 1e5, 1e-12, 7e4, 1e-30, 2.0, 65504.0])


@pytest.fixture(scope="module", autouse=True)
def gpu():
    require_gpu()


def wide_rows(seed, M, K):
    x = synth.randn(seed, (M, K))
    return (x * SCALES[np.arange(M) % SCALES.size][:, None]).astype(np.float32)


def assert_rows_close(got, ref, rtol=1e-3, what=""):
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    assert np.isfinite(got).all(), f"{what}: non-finite outputs"
    for r in range(ref.shape[0]):
        s = np.abs(ref[r]).max()
        err = np.abs(got[r] - ref[r]).max()
        assert err <= rtol * s, f"{what}: row {r} (|ref| {s:.3g}) error {err:.3g}"


@pytest.mark.parametrize("M,K,N,want", [
    (1, 1024, 256, hip.PATH_SKINNY),
    (8, 4096, 512, hip.PATH_SKINNY),
    (77, 1024, 1024, hip.PATH_SKINNY),
    (77, 96, 256, hip.PATH_SKINNY),       # not a multiple of 256: q8_skinny
    (300, 1024, 512, hip.PATH_MFMA),      # direct-to-LDS Q8 GEMM
    (300, 96, 256, hip.PATH_MFMA),        # K % 64 != 0: register-staged GEMM
    (3072, 1024, 256, hip.PATH_MFMA),     # per-call expansion: cast + expand in one launch
])
def test_f32_activations_wide_range_nt(M, K, N, want):
    O = oracle()
    a = wide_rows(300 + M, M, K)
    w = O.q8_quantize(synth.randn(301, (N, K), 0.02))
    assert hip.matmul_path(abi.F32, abi.Q8_0, abi.F32, M, N, K, hip.B_NT) == want
    c = hip.matmul(a, abi.F32, w, abi.Q8_0, abi.F32, M, N, K, flags=hip.B_NT)
    assert_rows_close(c, ref_q8(a, w, K, N, nt=True), what=f"Q8 NT M={M} K={K}")


def test_f32_activations_wide_range_kn_unpacked():
    """The reference kernel contract (blocks along N of [K, N]): unpacked to
    f16 [N, K], then the f16 GEMM with f32 activations."""
    O = oracle()
    M, K, N = 256, 512, 384
    a = wide_rows(310, M, K)
    w = O.q8_quantize(synth.randn(311, (K, N), 0.02))
    c = hip.matmul(a, abi.F32, w, abi.Q8_0, abi.F32, M, N, K)
    assert_rows_close(c, ref_q8(a, w, K, N, nt=False), what="Q8 KN")


def test_f32_activations_wide_range_bias_gelu():
    O = oracle()
    M, K, N = 300, 1024, 512
    a = wide_rows(320, M, K) * np.float32(1e-3)
    w = O.q8_quantize(synth.randn(321, (N, K), 0.02))
    bias = synth.randn(322, N, 0.01)
    c = hip.matmul(a, abi.F32, w, abi.Q8_0, abi.F32, M, N, K, bias=bias,
                   flags=hip.B_NT | hip.BIAS | hip.GELU)
    ref = ref_q8(a, w, K, N, nt=True, bias=bias, gelu=True)
    # GELU(x) ~ x for large x, ~0 for large negative x: per-row scale
    # with a floor from the bias
    g, r = np.asarray(c, np.float64), np.asarray(ref, np.float64)
    for row in range(M):
        s = max(np.abs(r[row]).max(), 0.05)
        assert np.abs(g[row] - r[row]).max() <= 1e-3 * s, row


@pytest.mark.parametrize("M", [512, 77, 8], ids=["mfma", "skinny77", "skinny8"])
def test_bf16_activations_near_1e30(M):
    """Config 3's dtype pairing (bf16 activations x Q8_0) with activations
    far outside f16, as bf16 carries the f32 exponent range; on the MFMA
    GEMM (M = 512) and the streaming skinny kernel (M = 77, 8), which
    rounds bf16 to f16 itself."""
    O = oracle()
    K, N = 1024, 512
    a32 = wide_rows(330, M, K)
    a = O.f32_to_bf16(a32).reshape(M, K)
    w = O.q8_quantize(synth.randn(331, (N, K), 0.02))
    c = hip.matmul(a, abi.BF16, w, abi.Q8_0, abi.F32, M, N, K, flags=hip.B_NT)
    ref = ref_q8(bf16_to_f32(a).reshape(M, K), w, K, N, nt=True)
    assert_rows_close(c, ref, what="bf16 x Q8")


@pytest.mark.parametrize("shared", [True, False])
@pytest.mark.parametrize("M", [1, 32])
def test_batched_stream_wide_range(shared, M):
    O = oracle()
    batch, K, N = 6, 1024, 256
    a = wide_rows(340 + M, M if shared else batch * M, K)
    ws = [O.q8_quantize(synth.randn(341 + s, (N, K), 0.02)) for s in range(batch)]
    w_all = np.concatenate(ws)
    sw = ws[0].nbytes
    da, dw = hip.DeviceBuffer.of(a), hip.DeviceBuffer.of(w_all)
    dc = hip.DeviceBuffer(batch * M * N * 4)
    lib = hip.load()
    hip.check(lib.sam3_hip_matmul_q8_batched(abi.F32, da.ptr, dw.ptr, dc.ptr, batch, M, N, K,
                                              0 if shared else M * K, sw, M * N, None, 0,
                                              None), "q8_batched")
    hip.synchronize()
    c = dc.download(np.float32, (batch, M, N))
    for s in range(batch):
        a_s = a if shared else a[s * M:(s + 1) * M]
        assert_rows_close(c[s], ref_q8(a_s, ws[s], K, N, nt=True), what=f"slice {s}")


def _out(t, shape):
    import ctypes as C
    return np.ctypeslib.as_array(C.cast(t.data, C.POINTER(C.c_float)), shape=shape).copy()


@pytest.mark.parametrize("M", [512, 77], ids=["mfma", "skinny"])
def test_graph_layernorm_operand_out_of_range_reruns(M):
    """LN -> Q8 linear. At M = 512 the LayerNorm writes the direct-to-LDS
    GEMM's f16 operand; with gamma of 1e6 on some columns that f16 copy
    overflows, so the eval is redone on f32 (range_reruns == 1) and matches
    the oracle. At M = 77 (the skinny kernel) the LayerNorm writes f32 and
    the GEMM makes its own row-scaled f16 copy: no flag, no rerun, the
    same result."""
    O = oracle()
    K, N = 1024, 512
    skinny = M < 128
    x = synth.randn(350, (M, K))
    beta = synth.randn(352, (K,), 0.1)
    wq = O.q8_quantize(synth.randn(353, (N, K), 0.02))
    bias = synth.randn(354, (N,), 0.02)

    def run(gamma):
        G = graph.Graph()
        t = G.layernorm(G.tensor(abi.F32, (M, K), x), G.tensor(abi.F32, (K,), gamma),
                        G.tensor(abi.F32, (K,), beta))
        y = G.linear(t, G.tensor(abi.Q8_0, (N, K), wq), G.tensor(abi.F32, (N,), bias))
        be = hip.Backend(0)
        try:
            assert be.graph_eval(G.g) == abi.OK
            st = be.stats()
        finally:
            be.close()
        ln = O.layernorm(x, gamma, beta)
        return _out(y, (M, N)), ref_q8(ln, wq, K, N, nt=True, bias=bias), st

    gamma = synth.randn(351, (K,), 1.0)
    y, ref, st = run(gamma)
    assert (st.operand_writes == 0 if skinny else st.operand_writes >= 1)
    assert st.range_reruns == 0
    assert_rows_close(y, ref, what="in range")
    gamma_big = gamma.copy()
    gamma_big[::7] *= np.float32(1e6)
    y, ref, st = run(gamma_big)
    assert st.range_reruns == (0 if skinny else 1), "the f16 operand overflow was not caught"
    assert_rows_close(y, ref, what="LN x 1e6")


def test_graph_gemm_operand_out_of_range_reruns():
    """LN -> fc1 -> fc2 with Q8_0 weights (gh_mlp after the block's LN2):
    the LN writes fc1's f16 operand and fc1's epilogue writes fc2's. A
    bias of 1e5 puts fc1's outputs past f16; the eval is redone."""
    O = oracle()
    M, K, H, N = 512, 256, 1024, 256
    x = synth.randn(360, (M, K))
    gamma, beta = synth.randn(365, (K,)), synth.randn(366, (K,), 0.1)
    w1 = O.q8_quantize(synth.randn(361, (H, K), 0.05))
    w2 = O.q8_quantize(synth.randn(362, (N, H), 0.02))
    b2 = synth.randn(364, (N,), 0.02)

    def run(b1):
        G = graph.Graph()
        t = G.layernorm(G.tensor(abi.F32, (M, K), x), G.tensor(abi.F32, (K,), gamma),
                        G.tensor(abi.F32, (K,), beta))
        h = G.linear(t, G.tensor(abi.Q8_0, (H, K), w1), G.tensor(abi.F32, (H,), b1))
        y = G.linear(h, G.tensor(abi.Q8_0, (N, H), w2), G.tensor(abi.F32, (N,), b2))
        be = hip.Backend(0)
        try:
            assert be.graph_eval(G.g) == abi.OK
            st = be.stats()
        finally:
            be.close()
        h_ref = ref_q8(O.layernorm(x, gamma, beta), w1, K, H, nt=True, bias=b1)
        return _out(y, (M, N)), ref_q8(h_ref, w2, H, N, nt=True, bias=b2), st

    b1 = synth.randn(363, (H,), 0.1)
    y, ref, st = run(b1)
    assert st.operand_writes >= 2 and st.range_reruns == 0
    assert_rows_close(y, ref, what="in range")
    b1_big = b1.copy()
    b1_big[::5] = np.float32(1e5)
    y, ref, st = run(b1_big)
    assert st.range_reruns == 1, "the f16 operand overflow was not caught"
    assert_rows_close(y, ref, what="fc1 bias 1e5")


def test_graph_gemm_operand_tiny_parts_of_rows_do_not_rerun():
    """fc1 + GELU writing fc2's f16 operand (gh_mlp with Q8_0 weights):
    strongly negative pre-activations give GELU outputs of ~1e-9. When
    such runs are only parts of a row (every other group of 8 columns
    here), the row's f16 copy keeps its bits where they matter, so the
    eval is not redone (the GEMM epilogue tags rows, and only a row whose
    nonzero values are all below 2^-10 sets the flag). When whole rows
    are that small (every column), the eval is redone on f32. Both match
    the oracle."""
    O = oracle()
    M, K, H, N = 512, 256, 1024, 256
    x = synth.randn(370, (M, K))
    gamma, beta = synth.randn(375, (K,)), synth.randn(376, (K,), 0.1)
    w1 = O.q8_quantize(synth.randn(371, (H, K), 0.05))
    w2 = O.q8_quantize(synth.randn(372, (N, H), 0.02))
    b2 = synth.randn(374, (N,), 0.02)
    ln = O.layernorm(x, gamma, beta)

    def run(b1):
        G = graph.Graph()
        t = G.layernorm(G.tensor(abi.F32, (M, K), x), G.tensor(abi.F32, (K,), gamma),
                        G.tensor(abi.F32, (K,), beta))
        y = G.mlp(t, G.tensor(abi.Q8_0, (H, K), w1), G.tensor(abi.F32, (H,), b1),
                  G.tensor(abi.Q8_0, (N, H), w2), G.tensor(abi.F32, (N,), b2))
        be = hip.Backend(0)
        try:
            assert be.graph_eval(G.g) == abi.OK
            st = be.stats()
        finally:
            be.close()
        h_ref = ref_q8(ln, w1, K, H, nt=True, bias=b1, gelu=True)
        return _out(y, (M, N)), ref_q8(h_ref, w2, H, N, nt=True, bias=b2), st

    b1 = synth.randn(373, (H,), 0.1)
    half = b1.copy()
    half[(np.arange(H) // 8) % 2 == 0] = np.float32(-6.0)
    y, ref, st = run(half)
    assert st.operand_writes >= 2
    assert st.range_reruns == 0, "tiny parts of rows made the eval run again"
    assert_rows_close(y, ref, what="half the columns tiny")
    y, ref, st = run(np.full(H, -6.0, np.float32))
    assert st.range_reruns == 1, "rows of only tiny values were not caught"
    assert_rows_close(y, ref, what="whole rows tiny")
