"""BASELINE.json's configs at their full sizes, on the GPU.

Each case runs the whole problem on the GPU and checks it twice:
  - every output element against a float64 numpy product of the exact
    operand values (bf16 / f16 bits, Q8_0 blocks dequantized exactly as
    q * scale), at the north star's tolerances: f32 outputs normwise
    max |g - r| / max |r| <= 1e-3 with the elementwise and cosine bounds
    of assert_f32_close; bf16 outputs |g - r| <= max(2e-2, 1 bf16 ulp)
    (after bias + GELU the bound of the three roundings the reference
    makes too, check_bf16_whole); f16 outputs normwise 1e-3 and |g - r| <= max(5e-3, 2 f16
    ulps);
  - a seeded sample of rows (and attention slices) against the oracle,
    the bit-faithful restatement of the reference's kernels.
Cases:
  - config 1: f32 activations x Q8_0 [1024, 1024] at M = 5184;
  - config 2: bf16 and f16 fc1 / fc2, plain and with the fused bias +
    GELU, f16 also with f32 output (the f32-accumulate contract,
    oracle_matmul_f16_acc32);
  - config 3: bf16 activations x Q8_0 weights at M = 5184 for each of
    the four ViT-L layer GEMMs (cpu_matmul_q8.c:124-131 on the bf16
    values), and the 32-layer stream of distinct weights, whose last
    GEMM's output is checked whole;
  - config 5: the batched attention matmuls of the global blocks (16
    heads x 5184 tokens: Q K^T of 860 MB, then P V) and a spread of
    slices of the windowed ones (1296 x 576).
"""
import numpy as np
import pytest

from gpu_util import (assert_bf16_close, assert_f16_close, assert_f32_close, bf16_to_f32,
                      f16_to_f32, oracle, ref_linear, ref_q8, require_gpu, ulp_bf16, ulp_f16)
from sam3_amd import abi, hip, synth

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def gpu():
    require_gpu()


def rows_of(M, n=40, seed=11):
    rng = np.random.default_rng(seed)
    return np.unique(np.concatenate([[0, 1, M - 1], rng.integers(0, M, n)]))


def gelu64(x):
    """tanh-GELU (cpu_gelu.c:30-38) in float64."""
    return 0.5 * x * (1.0 + np.tanh(0.7978845608 * (x + 0.044715 * x ** 3)))


def dq64(w_blocks, N, K):
    """Q8_0 [N, K] blocks as float64 q * scale (exact)."""
    return oracle().q8_dequantize(w_blocks, N * K).reshape(N, K).astype(np.float64)


def check_bf16_whole(c_bits, ref64, pre64=None, what=""):
    """bf16 outputs against float64: |g - r| <= max(2e-2, 1 bf16 ulp of
    r). With pre64 (the exact pre-activation of a fused bias + GELU) the
    reference's chain rounds twice before the GELU (matmul, then bias
    add: up to one ulp of the pre-activation's binade), the GELU's slope
    is at most 1.13, and the output rounds once more: the bound is then
    max(2e-2, 1.25 ulp(pre) + 0.5 ulp(out)), ulps at the larger of
    |g| and |r| for the output."""
    g = bf16_to_f32(c_bits).astype(np.float64)
    err = np.abs(g - ref64)
    if pre64 is None:
        lim = np.maximum(2e-2, ulp_bf16(ref64))
    else:
        lim = np.maximum(2e-2, 1.25 * ulp_bf16(pre64) +
                         0.5 * ulp_bf16(np.maximum(np.abs(g), np.abs(ref64))))
    bad = err > lim
    idx = np.argwhere(bad)[:4]
    assert not bad.any(), (f"{what}: {bad.sum()} / {bad.size} bf16 outputs off the float64 "
                           f"product; max err {err.max():.3e}; (row, col, got, f64): " +
                           ", ".join(f"({i}, {j}, {g[i, j]:.6g}, {ref64[i, j]:.6g})"
                                     for i, j in idx))


def check_f16_whole(c_bits, ref64, what=""):
    g = np.asarray(c_bits, np.uint16).view(np.float16).astype(np.float64)
    assert np.isfinite(g).all(), f"{what}: non-finite outputs"
    err = np.abs(g - ref64)
    assert err.max() <= 1e-3 * np.abs(ref64).max(), f"{what}: normwise {err.max():.3e}"
    bad = err > np.maximum(5e-3, 2 * ulp_f16(ref64))
    assert not bad.any(), f"{what}: {bad.sum()} / {bad.size} f16 outputs off; max {err.max():.3e}"


@pytest.mark.parametrize("which", ["fc1", "fc2"])
def test_config2_f16_full_size(which):
    O = oracle()
    M, (K, N) = 5184, ((1024, 4096) if which == "fc1" else (4096, 1024))
    a = O.f32_to_fp16(synth.randn(700, (M, K))).reshape(M, K)
    w = O.f32_to_fp16(synth.randn(701, (N, K), 0.02)).reshape(N, K)
    bias = O.f32_to_fp16(synth.randn(702, N, 0.01))
    assert hip.matmul_path(abi.F16, abi.F16, abi.F16, M, N, K, hip.B_NT) == hip.PATH_MFMA
    c = hip.matmul(a, abi.F16, w, abi.F16, abi.F16, M, N, K, bias=bias,
                   flags=hip.B_NT | hip.BIAS | hip.GELU)
    assert np.isfinite(c.astype(np.uint16).view(np.float16)).all()
    r = rows_of(M)
    assert_f16_close(c[r], ref_linear("f16", a[r], w, bias, True, b_nt=True), what=which)
    a64 = f16_to_f32(a).astype(np.float64)
    w64 = f16_to_f32(w).astype(np.float64)
    p64 = a64 @ w64.T
    check_f16_whole(c, gelu64(p64 + f16_to_f32(bias).astype(np.float64)),
                    what=f"{which} bias+GELU, whole output")
    # and the plain GEMM with f32 output (the reference's f16 kernel
    # rounds every k; this is the f32-accumulate contract), against the
    # exact products summed in float64, every output
    c32 = hip.matmul(a, abi.F16, w, abi.F16, abi.F32, M, N, K, flags=hip.B_NT)
    assert_f32_close(c32, p64.astype(np.float32), what=f"{which} f32 out, whole output")


@pytest.mark.parametrize("which", ["fc1", "fc2"])
def test_config2_bf16_full_size_whole(which):
    """Config 2 bf16 (the headline GEMM's kind): every output of the plain
    GEMM and of the fused bias + GELU against float64."""
    O = oracle()
    M, (K, N) = 5184, ((1024, 4096) if which == "fc1" else (4096, 1024))
    a = O.f32_to_bf16(synth.randn(705, (M, K))).reshape(M, K)
    w = O.f32_to_bf16(synth.randn(706, (N, K), 0.02)).reshape(N, K)
    bias = O.f32_to_bf16(synth.randn(707, N, 0.01))
    p64 = bf16_to_f32(a).astype(np.float64) @ bf16_to_f32(w).astype(np.float64).T
    c = hip.matmul(a, abi.BF16, w, abi.BF16, abi.BF16, M, N, K, flags=hip.B_NT)
    check_bf16_whole(c, p64, what=f"bf16 {which}, whole output")
    c = hip.matmul(a, abi.BF16, w, abi.BF16, abi.BF16, M, N, K, bias=bias,
                   flags=hip.B_NT | hip.BIAS | hip.GELU)
    x64 = p64 + bf16_to_f32(bias).astype(np.float64)
    check_bf16_whole(c, gelu64(x64), pre64=x64, what=f"bf16 {which} bias+GELU, whole output")


def test_config1_q8_full_size_whole():
    """Config 1: f32 activations N(0,1) x Q8_0 of N(0,0.02) weights, seed 0
    and 1, every output against float64 on the dequantized weight."""
    O = oracle()
    M, N, K = 5184, 1024, 1024
    a = synth.randn(0, (M, K))
    w = O.q8_quantize(synth.randn(1, (N, K), 0.02))
    c = hip.matmul(a, abi.F32, w, abi.Q8_0, abi.F32, M, N, K, flags=hip.B_NT)
    ref = a.astype(np.float64) @ dq64(w, N, K).T
    assert_f32_close(c, ref.astype(np.float32), what="config 1, whole output")


CFG3 = {"qkv": (1024, 3072), "proj": (1024, 1024), "fc1": (1024, 4096), "fc2": (4096, 1024)}


@pytest.mark.parametrize("name", list(CFG3))
def test_config3_bf16_x_q8_full_size(name):
    O = oracle()
    M = 5184
    K, N = CFG3[name]
    a = O.f32_to_bf16(synth.randn(710 + K, (M, K))).reshape(M, K)
    w = O.q8_quantize(synth.randn(711 + N, (N, K), 0.02))
    assert hip.matmul_path(abi.BF16, abi.Q8_0, abi.F32, M, N, K, hip.B_NT) == hip.PATH_MFMA
    c = hip.matmul(a, abi.BF16, w, abi.Q8_0, abi.F32, M, N, K, flags=hip.B_NT)
    assert np.isfinite(c).all()
    r = rows_of(M)
    ref = ref_q8(bf16_to_f32(a[r]).reshape(len(r), K), w, K, N, nt=True)
    assert_f32_close(c[r], ref, what=f"config 3 {name}")
    ref64 = bf16_to_f32(a).astype(np.float64) @ dq64(w, N, K).T
    assert_f32_close(c, ref64.astype(np.float32), what=f"config 3 {name}, whole output")


def test_config3_32_layer_stream_last_output():
    """The 32-layer stream of config 3 as bench.py runs it: 128 GEMMs over
    distinct seeded Q8_0 weights (453 MB), bf16 activations, one output
    buffer. The last GEMM (layer 31's fc2) must leave its whole output,
    checked against float64."""
    M = 5184
    shapes = [(3072, 1024), (1024, 1024), (4096, 1024), (1024, 4096)]
    act = {1024: synth.randn(730, (M, 1024)), 4096: synth.randn(731, (M, 4096))}
    a_bits = {k: oracle().f32_to_bf16(v).reshape(v.shape) for k, v in act.items()}
    dact = {k: hip.DeviceBuffer.of(v) for k, v in a_bits.items()}
    layers, last = [], None
    for L in range(32):
        bufs = []
        for i, (n_, k_) in enumerate(shapes):
            wq = hip.q8_quantize(synth.randn(synth.tensor_seed(3, 100 + 4 * L + i), (n_, k_), 0.02))
            bufs.append(hip.DeviceBuffer.of(wq))
            last = wq
        layers.append(bufs)
    out = hip.DeviceBuffer(M * 4096 * 4)
    for bufs in layers:
        for (n_, k_), wb in zip(shapes, bufs):
            hip.matmul_dev(abi.BF16, dact[k_].ptr, abi.Q8_0, wb.ptr, abi.F32, out.ptr, M, n_, k_,
                           None, hip.B_NT, None)
    hip.synchronize()
    n_, k_ = shapes[-1]
    got = out.download(np.float32, (M, n_))
    ref = bf16_to_f32(a_bits[k_]).astype(np.float64) @ dq64(last, n_, k_).T
    assert_f32_close(got, ref.astype(np.float32), what="layer 31 fc2 of the stream, whole output")


def _slice_rows(dev, s, rows, S, N, es=2):
    """Rows `rows` of slice s of a [BH, S, N] 16-bit device tensor."""
    out = np.empty((len(rows), N), np.uint16)
    for i, row in enumerate(rows):
        out[i] = hip.download_ptr(dev.ptr + ((s * S + int(row)) * N) * es, N * es, np.uint16)
    return out


@pytest.mark.parametrize("BH,S,slices", [(16, 5184, (0, 7, 15)),
                                         (1296, 576, tuple(range(0, 1296, 59)) + (1295,))])
def test_config5_attention_matmuls_full_size(BH, S, slices):
    """gh_multihead_attention's Q K^T and P V (graph_helpers.c:808-843)
    for every head at once, Q, K, V ~ N(0,1)/8 in bf16. P V takes the
    Q K^T output as P (the GEMM is linear in P; those rows were just
    checked against the oracle)."""
    O = oracle()
    D = 64
    q = O.f32_to_bf16(synth.randn(720, (BH, S, D)) / 8).reshape(BH, S, D)
    k = O.f32_to_bf16(synth.randn(721, (BH, S, D)) / 8).reshape(BH, S, D)
    v = O.f32_to_bf16(synth.randn(722, (BH, S, D)) / 8).reshape(BH, S, D)
    lib = hip.load()
    dq, dk, dv = hip.DeviceBuffer.of(q), hip.DeviceBuffer.of(k), hip.DeviceBuffer.of(v)
    ds = hip.DeviceBuffer(BH * S * S * 2)
    do = hip.DeviceBuffer(BH * S * D * 2)
    hip.check(lib.sam3_hip_matmul_batched(abi.BF16, dq.ptr, dk.ptr, ds.ptr, BH, S, S, D,
                                          S * D, S * D, S * S, hip.B_NT, None), "QK^T")
    hip.check(lib.sam3_hip_matmul_batched(abi.BF16, ds.ptr, dv.ptr, do.ptr, BH, S, D, S,
                                          S * S, S * D, S * D, 0, None), "PV")
    hip.synchronize()
    rows = rows_of(S, 24, seed=BH)
    for s in slices:
        srows = _slice_rows(ds, s, rows, S, S)
        ref_s = O.matmul_bf16(q[s][rows], np.ascontiguousarray(O.transpose_u16(k[s])), 8)
        assert_bf16_close(srows, ref_s, what=f"QK^T slice {s}")
        orows = _slice_rows(do, s, rows, S, D)
        ref_o = O.matmul_bf16(srows, v[s], 8)
        assert_bf16_close(orows, ref_o, what=f"PV slice {s}")
    out = do.download(np.uint16, (BH, S, D))
    assert np.isfinite(bf16_to_f32(out)).all()
