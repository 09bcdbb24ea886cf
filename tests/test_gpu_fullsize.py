"""BASELINE.json's configs at their full sizes, on the GPU.

Rows (and attention slices) of a GEMM are independent. So each case runs
the whole problem on the GPU, then checks a seeded sample of rows (and
slices) against the oracle, and the whole output through size-independent
properties: finite, and the checked rows' error within the stated
tolerance.
  - config 2, f16: fc1 / fc2 with the fused bias + GELU, against the
    f32-accumulate restatement (oracle_matmul_f16_acc32);
  - config 3: bf16 activations x Q8_0 weights at M = 5184 for each of
    the four ViT-L layer GEMMs, against the reference's f32 Q8 kernel on
    the bf16 values (cpu_matmul_q8.c:124-131);
  - config 5: the batched attention matmuls of the global blocks (16
    heads x 5184 tokens: Q K^T of 860 MB, then P V) and a spread of
    slices of the windowed ones (1296 x 576).
"""
import numpy as np
import pytest

from gpu_util import (assert_bf16_close, assert_f16_close, assert_f32_close, bf16_to_f32,
                      oracle, ref_linear, ref_q8, require_gpu)
from sam3_amd import abi, hip, synth

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def gpu():
    require_gpu()


def rows_of(M, n=40, seed=11):
    rng = np.random.default_rng(seed)
    return np.unique(np.concatenate([[0, 1, M - 1], rng.integers(0, M, n)]))


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
    # and the plain GEMM with f32 output (the reference's f16 kernel
    # rounds every k; this is the f32-accumulate contract), against the
    # exact products summed in float64
    c32 = hip.matmul(a, abi.F16, w, abi.F16, abi.F32, M, N, K, flags=hip.B_NT)
    a64 = O.fp16_to_f32(a[r]).reshape(len(r), K).astype(np.float64)
    w64 = O.fp16_to_f32(w).reshape(N, K).astype(np.float64)
    assert_f32_close(c32[r], (a64 @ w64.T).astype(np.float32), what=f"{which} f32 out")


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
