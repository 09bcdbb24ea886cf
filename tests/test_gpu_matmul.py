"""GPU parity of the HIP matmul path against the CPU oracle, through the C ABI.

Every case runs the HIP kernels on seeded inputs and compares with the
oracle (oracle/sam3_oracle.c, itself pinned to the reference in
tests/test_oracle.py) or with the reference's golden vectors:
  - generic path: bit-exact with the reference (same per-element order);
  - tiled MFMA / skinny paths: f32 outputs within 1e-3 (relative, with an
    rms floor), bf16 within max(2e-2, 1 ulp), f16 within max(5e-3, 2 ulp).
"""
from pathlib import Path

import numpy as np
import pytest

from gpu_util import (assert_bf16_close, assert_f16_close, assert_f32_close, oracle,
                      ref_linear, ref_q8, require_gpu, bf16_to_f32)
from sam3_amd import abi, hip, synth

pytestmark = pytest.mark.gpu

GOLD = np.load(Path(__file__).parent / "golden" / "matmul_golden.npz")
MFMA, SKINNY, GENERIC = hip.PATH_MFMA, hip.PATH_SKINNY, hip.PATH_GENERIC


@pytest.fixture(scope="module", autouse=True)
def gpu():
    require_gpu()


def bits32(x):
    return np.ascontiguousarray(x, np.float32).view(np.uint32)


def rnd(seed, shape, std=1.0):
    return synth.randn(seed, shape, std)


def q8(w):
    return oracle().q8_quantize(w)


# ------------------------------------------------------------ Q8_0 format
def _cpu_quantizer():
    """The reference's own quantizer when oracle/_ref is built, else the
    restatement (pinned to it in test_oracle.py)."""
    from oracle_bind import Ref, have_ref
    return Ref() if have_ref() else oracle()


def test_q8_quantize_golden_bit_exact():
    qx = GOLD["quant_x"]
    assert np.array_equal(hip.q8_quantize(qx), GOLD["quant_blocks"])
    assert np.array_equal(bits32(hip.q8_dequantize(GOLD["quant_blocks"], qx.size)),
                          bits32(GOLD["quant_deq"]))


def q8_edge_values():
    """Blocks that exercise every branch of sam3_q8_quantize: exact .5 ties
    after scaling (roundf rounds away from zero), a zero block, a block of
    subnormals (its scale's reciprocal overflows), +-inf and NaN (the x86
    conversion of NaN/inf gives INT_MIN, clamped to -127), huge values."""
    blk = []
    t = np.zeros(32, np.float32)
    t[0] = 127.0
    t[1:8] = [0.5, -0.5, 1.5, -2.5, 126.5, -126.5, 63.5]
    blk.append(t)
    blk.append(np.zeros(32, np.float32))
    blk.append(np.full(32, 1e-40, np.float32) * np.arange(-16, 16, dtype=np.float32))
    t = synth.randn(201, 32)
    t[3], t[9] = np.inf, -np.inf
    blk.append(t)
    t = synth.randn(202, 32)
    t[5] = np.nan
    blk.append(t)
    blk.append(synth.randn(203, 32) * np.float32(3e37))
    return np.concatenate(blk).astype(np.float32)


@pytest.mark.parametrize("n", [1, 31, 32, 33, 1000, 65537])
def test_q8_quantize_matches_reference(n):
    Q = _cpu_quantizer()
    x = synth.randn(200 + n, n) * np.float32(0.02 if n % 2 else 3.0)
    assert np.array_equal(hip.q8_quantize(x), Q.q8_quantize(x))
    blocks = Q.q8_quantize(x)
    assert np.array_equal(bits32(hip.q8_dequantize(blocks, n)), bits32(Q.q8_dequantize(blocks, n)))


def test_q8_quantize_edge_blocks():
    Q = _cpu_quantizer()
    x = q8_edge_values()
    got, ref = hip.q8_quantize(x), Q.q8_quantize(x)
    assert np.array_equal(got, ref), np.nonzero(got != ref)[0][:16]
    tie = got[:36]
    assert list(tie[4:12].view(np.int8)) == [127, 1, -1, 2, -3, 127, -127, 64]


# ------------------------------------------------------------ known answers
def test_known_answer_f32_all_paths():
    """tests/test_cpu_kernels.c:474-500: exact [58,64;139,154]."""
    a = np.array([[1, 2, 3], [4, 5, 6]], np.float32)
    b = np.array([[7, 8], [9, 10], [11, 12]], np.float32)
    for path in (0, GENERIC):
        c = hip.matmul(a, abi.F32, b, abi.F32, abi.F32, 2, 2, 3, path=path)
        assert c.tolist() == [[58, 64], [139, 154]]


def test_identity_bf16_f16_mfma():
    """tests/test_matmul_bf16.c:126-181: X @ I == X, on the tiled path."""
    O = oracle()
    n = 64
    x = rnd(1, (n, n))
    eye = np.eye(n, dtype=np.float32)
    xb, ib = O.f32_to_bf16(x).reshape(n, n), O.f32_to_bf16(eye).reshape(n, n)
    assert np.array_equal(hip.matmul(xb, abi.BF16, ib, abi.BF16, abi.BF16, n, n, n, path=MFMA), xb)
    xh, ih = O.f32_to_fp16(x).reshape(n, n), O.f32_to_fp16(eye).reshape(n, n)
    assert np.array_equal(hip.matmul(xh, abi.F16, ih, abi.F16, abi.F16, n, n, n, path=MFMA), xh)


# ---------------------------------------------------- golden vectors (reference)
@pytest.mark.parametrize("name", ["q8_a", "q8_b", "q8_c", "q8_t"])
def test_golden_q8_generic_bit_exact(name):
    M, K, N = (int(v) for v in GOLD[f"{name}_shape"])
    c = hip.matmul(GOLD[f"{name}_a"], abi.F32, GOLD[f"{name}_b"], abi.Q8_0, abi.F32, M, N, K,
                   path=GENERIC)
    assert np.array_equal(bits32(c), bits32(GOLD[f"{name}_c"]))


@pytest.mark.parametrize("name", ["q8_a", "q8_b", "q8_c", "q8_t"])
def test_golden_q8_auto_path(name):
    M, K, N = (int(v) for v in GOLD[f"{name}_shape"])
    c = hip.matmul(GOLD[f"{name}_a"], abi.F32, GOLD[f"{name}_b"], abi.Q8_0, abi.F32, M, N, K)
    assert_f32_close(c, GOLD[f"{name}_c"], what=name)


def test_golden_q8_nt_generic_bit_exact_and_fast_paths():
    M, K, N = (int(v) for v in GOLD["q8nt_shape"])
    a, w = GOLD["q8nt_a"], GOLD["q8nt_w"]
    c = hip.matmul(a, abi.F32, w, abi.Q8_0, abi.F32, M, N, K, flags=hip.B_NT, path=GENERIC)
    assert np.array_equal(bits32(c), bits32(GOLD["q8nt_c"]))
    for path in (MFMA, SKINNY):
        c = hip.matmul(a, abi.F32, w, abi.Q8_0, abi.F32, M, N, K, flags=hip.B_NT, path=path)
        assert_f32_close(c, GOLD["q8nt_c"], what=f"q8nt path {path}")


def test_golden_dense_generic_bit_exact():
    M, K = GOLD["bf16_a"].shape
    N = GOLD["bf16_b"].shape[1]
    c = hip.matmul(GOLD["bf16_a"], abi.BF16, GOLD["bf16_b"], abi.BF16, abi.BF16, M, N, K,
                   path=GENERIC)
    assert np.array_equal(c, GOLD["bf16_c"])
    for name in ("f32", "f32b"):
        a, b = GOLD[f"{name}_a"], GOLD[f"{name}_b"]
        (M, K), N = a.shape, b.shape[1]
        c = hip.matmul(a, abi.F32, b, abi.F32, abi.F32, M, N, K, path=GENERIC)
        assert np.array_equal(bits32(c), bits32(GOLD[f"{name}_c"]))


def test_golden_dense_tiled():
    M, K = GOLD["bf16_a"].shape
    N = GOLD["bf16_b"].shape[1]
    c = hip.matmul(GOLD["bf16_a"], abi.BF16, GOLD["bf16_b"], abi.BF16, abi.BF16, M, N, K,
                   path=MFMA)
    assert_bf16_close(c, GOLD["bf16_c"], what="golden bf16")
    a, b = GOLD["f32b_a"], GOLD["f32b_b"]
    (M, K), N = a.shape, b.shape[1]
    assert hip.matmul_path(abi.F32, abi.F32, abi.F32, M, N, K) == GENERIC  # N=65, K=200
    a, b = GOLD["f32b_a"][:, :128], GOLD["f32b_b"][:128, :64]
    c = hip.matmul(a, abi.F32, b, abi.F32, abi.F32, 33, 64, 128, path=MFMA)
    assert_f32_close(c, oracle().matmul_f32(a, b), rtol=1e-5, floor=1e-5, what="f32 tiled")


def test_golden_f16_generic_equals_acc32_oracle():
    """The reference f16 kernel accumulates in fp16; the HIP path
    accumulates in f32 and equals the oracle's f32-accumulate
    restatement bit for bit on the generic path, and stays closer to
    float64 than the reference's fp16 accumulator does."""
    a, b = GOLD["f16_a"], GOLD["f16_b"]
    (M, K), N = a.shape, b.shape[1]
    c = hip.matmul(a, abi.F16, b, abi.F16, abi.F16, M, N, K, path=GENERIC)
    assert np.array_equal(c, oracle().matmul_f16_acc32(a, b))
    exact = (a.view(np.float16).astype(np.float64) @ b.view(np.float16).astype(np.float64))
    err_hip = np.abs(c.view(np.float16).astype(np.float64) - exact).max()
    err_ref = np.abs(GOLD["f16_c"].view(np.float16).astype(np.float64) - exact).max()
    assert err_hip <= err_ref


# ------------------------------------------------------------- tiled GEMMs
DENSE_SHAPES = [(256, 128, 64), (300, 200, 136), (5, 64, 40), (129, 257, 1032), (64, 512, 8)]


@pytest.mark.parametrize("M,N,K", DENSE_SHAPES)
@pytest.mark.parametrize("nt", [False, True])
def test_bf16_tiled_vs_oracle(M, N, K, nt):
    O = oracle()
    a = O.f32_to_bf16(rnd(10 + M, (M, K))).reshape(M, K)
    b32 = rnd(20 + N, (N, K) if nt else (K, N), 0.2)
    b = O.f32_to_bf16(b32).reshape(b32.shape)
    if hip.matmul_path(abi.BF16, abi.BF16, abi.BF16, M, N, K, hip.B_NT if nt else 0) != MFMA:
        pytest.skip("NN tiles need N % 8 == 0")
    c = hip.matmul(a, abi.BF16, b, abi.BF16, abi.BF16, M, N, K, flags=hip.B_NT if nt else 0,
                   path=MFMA)
    assert_bf16_close(c, ref_linear("bf16", a, b, b_nt=nt), what=f"bf16 {M}x{N}x{K} nt={nt}")


@pytest.mark.parametrize("M,N,K", DENSE_SHAPES)
@pytest.mark.parametrize("nt", [False, True])
def test_f16_tiled_vs_oracle(M, N, K, nt):
    O = oracle()
    a = O.f32_to_fp16(rnd(30 + M, (M, K))).reshape(M, K)
    b32 = rnd(40 + N, (N, K) if nt else (K, N), 0.2)
    b = O.f32_to_fp16(b32).reshape(b32.shape)
    if hip.matmul_path(abi.F16, abi.F16, abi.F16, M, N, K, hip.B_NT if nt else 0) != MFMA:
        pytest.skip("NN tiles need N % 8 == 0")
    c = hip.matmul(a, abi.F16, b, abi.F16, abi.F16, M, N, K, flags=hip.B_NT if nt else 0,
                   path=MFMA)
    assert_f16_close(c, ref_linear("f16", a, b, b_nt=nt), what=f"f16 {M}x{N}x{K} nt={nt}")


@pytest.mark.parametrize("M,N,K", [(128, 128, 64), (100, 72, 36), (257, 130, 512)])
@pytest.mark.parametrize("nt", [False, True])
def test_f32_tiled_vs_oracle(M, N, K, nt, env):
    """The f32 MFMA kernel (v_mfma_f32_32x32x2_f32, exact f32 products)."""
    env.set("SAM3_HIP_F32_SPLIT", "0")
    a = rnd(50 + M, (M, K))
    b = rnd(60 + N, (N, K) if nt else (K, N))
    if hip.matmul_path(abi.F32, abi.F32, abi.F32, M, N, K, hip.B_NT if nt else 0) != MFMA:
        pytest.skip("shape not on the tiled path")
    c = hip.matmul(a, abi.F32, b, abi.F32, abi.F32, M, N, K, flags=hip.B_NT if nt else 0,
                   path=MFMA)
    assert_f32_close(c, ref_linear("f32", a, b, b_nt=nt), rtol=1e-5, floor=1e-5,
                     what=f"f32 {M}x{N}x{K}")


@pytest.mark.parametrize("M,N,K", [(257, 130, 512), (5184, 1024, 1024), (1000, 3072, 1024),
                                   (300, 4096, 4096)])
@pytest.mark.parametrize("epi", [0, 1])
def test_f32_split_gemm(M, N, K, epi):
    """f32 x f32 with W [N,K] on the bf16 MFMA GEMM over a tripled k
    (A' = [Ah|Al|Ah], W' = [Wh|Wh|Wl]): within the f32 bound, and within
    2e-5 normwise of the reference (each product keeps ~16 bits)."""
    a, w = rnd(80 + M, (M, K)), rnd(81 + N, (N, K), 0.05)
    bias = rnd(82, N, 0.3) if epi else None
    flags = hip.B_NT | ((hip.BIAS | hip.GELU) if epi else 0)
    c = hip.matmul(a, abi.F32, w, abi.F32, abi.F32, M, N, K, bias=bias, flags=flags, path=MFMA)
    ref = ref_linear("f32", a, w, bias=bias, gelu=bool(epi), b_nt=True)
    assert_f32_close(c, ref, what=f"f32 split {M}x{N}x{K}")
    err = np.abs(c.astype(np.float64) - ref).max() / np.abs(ref).max()
    assert err <= 2e-5, err


@pytest.mark.parametrize("kind", ["bf16", "f16", "f32"])
def test_fused_bias_gelu(kind):
    """MATMUL -> ADD(bias) -> GELU in one launch, rounded like the three
    reference nodes (cpu_add_bf16.c:62-63, cpu_gelu_bf16.c:62-64)."""
    O = oracle()
    M, N, K = 200, 192, 256
    a32, w32, b32 = rnd(70, (M, K)), rnd(71, (N, K), 0.05), rnd(72, N, 0.3)
    if kind == "f32":
        a, w, bias, dt = a32, w32, b32, abi.F32
    elif kind == "bf16":
        a, w, bias, dt = (O.f32_to_bf16(a32).reshape(M, K), O.f32_to_bf16(w32).reshape(N, K),
                          O.f32_to_bf16(b32), abi.BF16)
    else:
        a, w, bias, dt = (O.f32_to_fp16(a32).reshape(M, K), O.f32_to_fp16(w32).reshape(N, K),
                          O.f32_to_fp16(b32), abi.F16)
    for flags in (hip.BIAS, hip.GELU, hip.BIAS | hip.GELU):
        c = hip.matmul(a, dt, w, dt, dt, M, N, K, bias=bias if flags & hip.BIAS else None,
                       flags=flags | hip.B_NT, path=MFMA)
        ref = ref_linear(kind, a, w, bias if flags & hip.BIAS else None, bool(flags & hip.GELU),
                         b_nt=True)
        {"f32": lambda g, r: assert_f32_close(g, r, what=f"fused {kind} {flags}"),
         "bf16": lambda g, r: assert_bf16_close(g, r, what=f"fused {kind} {flags}"),
         "f16": lambda g, r: assert_f16_close(g, r, what=f"fused {kind} {flags}")}[kind](c, ref)


@pytest.mark.parametrize("cfg", [0, 1, 2, 3, 4, 6, 7, 8, 9, 10, 11, 12, 13])
def test_dl_every_tile_config(env, cfg):
    """Each direct-to-LDS tile configuration (forced) on a ragged bf16 NT
    problem with a k tail, bias and GELU, against the oracle."""
    env.set("SAM3_HIP_DL_CFG", str(cfg))
    O = oracle()
    M, N, K = 300, 520, 200
    a = O.f32_to_bf16(rnd(210, (M, K))).reshape(M, K)
    w = O.f32_to_bf16(rnd(211, (N, K), 0.05)).reshape(N, K)
    bias = O.f32_to_bf16(rnd(212, N, 0.1))
    assert hip.matmul_path(abi.BF16, abi.BF16, abi.BF16, M, N, K, hip.B_NT) == MFMA
    c = hip.matmul(a, abi.BF16, w, abi.BF16, abi.BF16, M, N, K, bias=bias,
                   flags=hip.B_NT | hip.BIAS | hip.GELU)
    ref = ref_linear("bf16", a, w, bias=bias, gelu=True, b_nt=True)
    assert_bf16_close(c, ref, what=f"dl cfg {cfg}")


@pytest.mark.parametrize("cfg", [20, 21, 22, 23, 24, 25, 26])
@pytest.mark.parametrize("K", [64, 128, 320])
def test_dl_pipelined_every_tile_config(env, cfg, K):
    """The pipelined direct-to-LDS kernel (K % 64 == 0: one, two and five
    k-steps, so the peeled last steps and the steady-state loop both run)
    on ragged M and N with bias and GELU, against the oracle, and with the
    same bits as gemm_dl (same accumulation order)."""
    O = oracle()
    M, N = 300, 520
    a = O.f32_to_bf16(rnd(213, (M, K))).reshape(M, K)
    w = O.f32_to_bf16(rnd(214, (N, K), 0.05)).reshape(N, K)
    bias = O.f32_to_bf16(rnd(215, N, 0.1))
    flags = hip.B_NT | hip.BIAS | hip.GELU
    env.set("SAM3_HIP_DL_CFG", str(cfg))
    c = hip.matmul(a, abi.BF16, w, abi.BF16, abi.BF16, M, N, K, bias=bias, flags=flags)
    assert_bf16_close(c, ref_linear("bf16", a, w, bias=bias, gelu=True, b_nt=True),
                      what=f"dlp cfg {cfg} K={K}")
    env.set("SAM3_HIP_DL_CFG", "4")
    c4 = hip.matmul(a, abi.BF16, w, abi.BF16, abi.BF16, M, N, K, bias=bias, flags=flags)
    assert np.array_equal(c, c4)
    # f16 operands with an f32 output through the same kernels
    env.set("SAM3_HIP_DL_CFG", str(cfg))
    a16 = O.f32_to_fp16(rnd(216, (M, K))).reshape(M, K)
    w16 = O.f32_to_fp16(rnd(217, (N, K), 0.05)).reshape(N, K)
    c32 = hip.matmul(a16, abi.F16, w16, abi.F16, abi.F32, M, N, K, flags=hip.B_NT)
    ref = (O.fp16_to_f32(a16).reshape(M, K).astype(np.float64) @
           O.fp16_to_f32(w16).reshape(N, K).astype(np.float64).T)
    assert_f32_close(c32, ref.astype(np.float32), what=f"dlp cfg {cfg} f16 K={K}")


def test_bf16_output_f32():
    """bf16 operands with an f32 output (no rounding of C)."""
    O = oracle()
    M, N, K = 128, 128, 128
    a = O.f32_to_bf16(rnd(80, (M, K))).reshape(M, K)
    b = O.f32_to_bf16(rnd(81, (N, K))).reshape(N, K)
    c = hip.matmul(a, abi.BF16, b, abi.BF16, abi.F32, M, N, K, flags=hip.B_NT, path=MFMA)
    exact = bf16_to_f32(a).astype(np.float64) @ bf16_to_f32(b).astype(np.float64).T
    assert_f32_close(c, exact, rtol=1e-4, what="bf16->f32")


# ----------------------------------------------------------------- Q8 paths
Q8_SHAPES = [(256, 256, 256), (300, 136, 512), (64, 1024, 1024), (130, 96, 4096)]


@pytest.mark.parametrize("M,N,K", Q8_SHAPES)
def test_q8_nt_tiled_f32_activations(M, N, K):
    a = rnd(90 + M, (M, K))
    w = q8(rnd(91 + N, (N, K), 0.02))
    c = hip.matmul(a, abi.F32, w, abi.Q8_0, abi.F32, M, N, K, flags=hip.B_NT, path=MFMA)
    assert_f32_close(c, ref_q8(a, w, K, N, nt=True), what=f"q8 nt {M}x{N}x{K}")


@pytest.mark.parametrize("M,N,K", [(256, 256, 256), (77, 200, 1024)])
def test_q8_nt_tiled_bf16_and_f16_activations(M, N, K):
    """bf16 activations (config 3): the reference has no bf16 x Q8 kernel,
    so the oracle upcasts the activations to f32 exactly first."""
    O = oracle()
    a32 = rnd(100 + M, (M, K))
    w = q8(rnd(101 + N, (N, K), 0.02))
    ab = O.f32_to_bf16(a32).reshape(M, K)
    ref = ref_q8(bf16_to_f32(ab).reshape(M, K), w, K, N, nt=True)
    for path in (MFMA, SKINNY) if M <= 128 else (MFMA,):
        c = hip.matmul(ab, abi.BF16, w, abi.Q8_0, abi.F32, M, N, K, flags=hip.B_NT, path=path)
        assert_f32_close(c, ref, what=f"q8 bf16-act path {path}")
    ah = O.f32_to_fp16(a32).reshape(M, K)
    ref = ref_q8(ah.view(np.float16).astype(np.float32), w, K, N, nt=True)
    c = hip.matmul(ah, abi.F16, w, abi.Q8_0, abi.F32, M, N, K, flags=hip.B_NT, path=MFMA)
    assert_f32_close(c, ref, what="q8 f16-act")


@pytest.mark.parametrize("cfg", [0, 1, 2, 3, 5, 6, 10, 11, 12])
@pytest.mark.parametrize("a_dt", [abi.F32, abi.BF16, abi.F16])
def test_q8_dl_every_config(env, cfg, a_dt):
    """Direct-to-LDS Q8 GEMM (raw 36-byte blocks in LDS, dequantized per
    fragment) with each tile configuration forced, ragged M and N, bias +
    GELU. bf16 activations go through the f16 cast first; f32 activations
    run the register-staged kernel (the configuration does not apply)."""
    env.set("SAM3_HIP_DLQ8_CFG", str(cfg))
    O = oracle()
    M, N, K = 300, 200, 576
    a32 = rnd(220, (M, K))
    w = q8(rnd(221, (N, K), 0.02))
    bias = rnd(222, N, 0.1)
    if a_dt == abi.F32:
        a, a_ref = a32, a32
    elif a_dt == abi.BF16:
        a = O.f32_to_bf16(a32).reshape(M, K)
        a_ref = O.bf16_to_f32(a).reshape(M, K)
    else:
        a = O.f32_to_fp16(a32).reshape(M, K)
        a_ref = O.fp16_to_f32(a).reshape(M, K)
    c = hip.matmul(a, a_dt, w, abi.Q8_0, abi.F32, M, N, K, bias=bias,
                   flags=hip.B_NT | hip.BIAS | hip.GELU, path=MFMA)
    ref = ref_q8(np.asarray(a_ref, np.float32), w, K, N, nt=True, bias=bias, gelu=True)
    assert_f32_close(c, ref, what=f"dlq8 cfg {cfg} a={a_dt}")


@pytest.mark.parametrize("cfg", [10, 11, 12])
def test_q8_pipelined_same_bits_as_dlq8(env, cfg):
    """The pipelined Q8 kernel (gemm_dlpq) dequantizes each weight fragment
    with gemm_dlq8's arithmetic and accumulates the k-steps in the same
    order, so every output has gemm_dlq8's bits, whatever the tiles;
    ragged M and N, K of 16 k-steps, weight rows with tiny scales (their
    row factor) among them."""
    O = oracle()
    M, N, K = 1000, 520, 1024
    a = O.f32_to_fp16(rnd(230, (M, K))).reshape(M, K)
    wf = rnd(231, (N, K), 0.02)
    wf[7] *= np.float32(1e-6)
    w = q8(wf)
    bias = rnd(232, N, 0.1)
    env.set("SAM3_HIP_Q8_EXPAND", 0)
    outs = []
    for c in (2, cfg):
        env.set("SAM3_HIP_DLQ8_CFG", str(c))
        outs.append(hip.matmul(a, abi.F16, w, abi.Q8_0, abi.F32, M, N, K, bias=bias,
                               flags=hip.B_NT | hip.BIAS, path=MFMA))
    assert np.array_equal(outs[0].view(np.uint32), outs[1].view(np.uint32))
    ref = ref_q8(O.fp16_to_f32(a).reshape(M, K), w, K, N, nt=True, bias=bias)
    assert_f32_close(outs[1], ref, what=f"dlpq cfg {cfg}")


def test_q8_dl_one_hot_rows():
    """One-hot A rows select W rows: the result is q*scale rounded through
    f16 (scale rounded to f16, product rounded to f16), within 2 f16 ulps of
    the exact dequantized weight."""
    O = oracle()
    K, N = 256, 136
    w = q8(rnd(225, (N, K), 0.02))
    deq = O.q8_dequantize(w, N * K).reshape(N, K)
    rows = list(range(0, 256, 8))
    a = np.eye(K, dtype=np.float32)[rows]
    a = np.concatenate([a, np.zeros((200 - len(rows), K), np.float32)])
    c = hip.matmul(a, abi.F32, w, abi.Q8_0, abi.F32, 200, N, K, flags=hip.B_NT, path=MFMA)
    got, ref = c[:len(rows)], deq[:, rows].T
    assert np.all(np.abs(got - ref) <= 2 * np.spacing(np.abs(ref).astype(np.float16)).astype(np.float32) + 1e-12)
    assert np.all(c[len(rows):] == 0)


@pytest.mark.parametrize("M,N,K", [(128, 96, 256), (64, 100, 64), (200, 64, 72), (256, 100, 128)])
def test_q8_kn_kernel_contract(M, N, K):
    """B Q8_0 [K,N] with blocks over the flat index (the layout
    cpu_kernel_matmul_q8 and tests/test_matmul_q8.c use), through the node
    kernel: unpacked to f16 then the tiled GEMM, or the generic kernel."""
    a = rnd(110 + M, (M, K))
    b = q8(rnd(111 + N, (K, N), 0.02))
    ref = ref_q8(a, b, K, N, nt=False)
    c = hip.matmul(a, abi.F32, b, abi.Q8_0, abi.F32, M, N, K)
    assert_f32_close(c, ref, what=f"q8 kn {M}x{N}x{K}")
    g = hip.matmul(a, abi.F32, b, abi.Q8_0, abi.F32, M, N, K, path=GENERIC)
    assert np.array_equal(bits32(g), bits32(ref))


@pytest.mark.parametrize("M", [1, 8, 32, 77])
@pytest.mark.parametrize("K,N", [(256, 256), (256, 2048), (1024, 1024), (1024, 4096), (4096, 1024)])
def test_skinny_q8_config4(M, K, N):
    """Config 4: prompt-decoder / text-encoder shapes on the skinny kernel."""
    assert hip.matmul_path(abi.F32, abi.Q8_0, abi.F32, M, N, K, hip.B_NT) == SKINNY
    a = rnd(120 + M, (M, K))
    w = q8(rnd(121 + N + K, (N, K), 0.02))
    c = hip.matmul(a, abi.F32, w, abi.Q8_0, abi.F32, M, N, K, flags=hip.B_NT)
    assert_f32_close(c, ref_q8(a, w, K, N, nt=True), what=f"skinny M={M} K={K} N={N}")


def test_skinny_bias_gelu_and_ragged_n():
    M, N, K = 5, 37, 96
    a = rnd(130, (M, K))
    w = q8(rnd(131, (N, K), 0.05))
    bias = rnd(132, N, 0.1)
    c = hip.matmul(a, abi.F32, w, abi.Q8_0, abi.F32, M, N, K, bias=bias,
                   flags=hip.B_NT | hip.BIAS | hip.GELU, path=SKINNY)
    assert_f32_close(c, ref_q8(a, w, K, N, nt=True, bias=bias, gelu=True), what="skinny epi")


STREAM_CFGS = [(mr, nt) for mr in (1, 4, 8, 16, 32) for nt in (1, 2, 4)]


@pytest.mark.parametrize("K", [256, 1536])
@pytest.mark.parametrize("mr,nt", STREAM_CFGS)
def test_stream_kernel_every_shape(env, mr, nt, K):
    """q8_stream (K % 256 == 0) with each workgroup shape forced: M split
    over ceil(M / mr) workgroups, ragged N (not a multiple of 16*nt), one
    8-block chunk (K 256) or three 16-block chunks (K 1536; 8-block chunks
    for mr 32), fused bias + GELU."""
    env.set("SAM3_HIP_SK_CFG", f"{mr},{nt}")
    M, N = 37, 200
    a = rnd(170, (M, K))
    w = q8(rnd(171, (N, K), 0.02))
    bias = rnd(172, N, 0.1)
    c = hip.matmul(a, abi.F32, w, abi.Q8_0, abi.F32, M, N, K, bias=bias,
                   flags=hip.B_NT | hip.BIAS | hip.GELU, path=SKINNY)
    assert_f32_close(c, ref_q8(a, w, K, N, nt=True, bias=bias, gelu=True),
                     what=f"stream mr={mr} nt={nt}")


@pytest.mark.parametrize("K", [768, 1024])
@pytest.mark.parametrize("a_dt", [abi.BF16, abi.F16])
@pytest.mark.parametrize("mr,nt", [(1, 1), (8, 2), (32, 4)])
def test_stream_kernel_16bit_activations(env, a_dt, mr, nt, K):
    env.set("SAM3_HIP_SK_CFG", f"{mr},{nt}")
    O = oracle()
    M, N = 20, 72
    a32 = rnd(175, (M, K))
    if a_dt == abi.BF16:
        a16 = O.f32_to_bf16(a32)
        a_ref = O.bf16_to_f32(a16)
    else:
        a16 = O.f32_to_fp16(a32)
        a_ref = O.fp16_to_f32(a16)
    w = q8(rnd(176, (N, K), 0.02))
    c = hip.matmul(a16, a_dt, w, abi.Q8_0, abi.F32, M, N, K, flags=hip.B_NT, path=SKINNY)
    assert_f32_close(c, ref_q8(np.asarray(a_ref, np.float32).reshape(M, K), w, K, N, nt=True),
                     what=f"stream {a_dt} mr={mr} nt={nt}")


def test_stream_kernel_one_hot_exact():
    """One-hot A through q8_stream selects dequantized weights exactly:
    q is exact in f16, 1.0 is exact, the scale is applied in f32."""
    O = oracle()
    K, N = 512, 80
    w = q8(rnd(178, (N, K), 0.02))
    deq = O.q8_dequantize(w, N * K).reshape(N, K)
    rows = [0, 1, 255, 256, 300, 511]
    a = np.eye(K, dtype=np.float32)[rows]
    c = hip.matmul(a, abi.F32, w, abi.Q8_0, abi.F32, len(rows), N, K, flags=hip.B_NT,
                   path=SKINNY)
    assert np.array_equal(c, deq[:, rows].T)


@pytest.mark.parametrize("shared_a", [False, True])
def test_q8_batched_stream(shared_a):
    """sam3_hip_matmul_q8_batched: distinct weights per slice in one launch,
    against the oracle slice by slice (stride_a = 0 shares the activations)."""
    B, M, N, K = 5, 8, 96, 512
    a = rnd(180, (1 if shared_a else B, M, K))
    ws = [q8(rnd(181 + s, (N, K), 0.02)) for s in range(B)]
    wbytes = ws[0].nbytes
    da = hip.DeviceBuffer.of(a)
    dw = hip.DeviceBuffer.of(np.concatenate(ws))
    dc = hip.DeviceBuffer(B * M * N * 4)
    hip.q8_batched_dev(abi.F32, da.ptr, dw.ptr, dc.ptr, B, M, N, K,
                       0 if shared_a else M * K, wbytes, M * N)
    hip.synchronize()
    c = dc.download(np.float32, (B, M, N))
    for s in range(B):
        ref = ref_q8(a[0 if shared_a else s], ws[s], K, N, nt=True)
        assert_f32_close(c[s], ref, what=f"q8 batched slice {s}")


@pytest.mark.parametrize("M,K", [(2, 1024), (24, 1024), (77, 1024)])
def test_q8_batched_shared_f32_cast_once(M, K):
    """Shared f32 activations of a batched skinny launch are cast to f16
    once before the launch; the kernel rounds f32 activations to f16 the
    same way, so the result has the same bits as passing the activations
    as f16 (both batched, so the same workgroup shape runs). One row is
    not cast: it runs on the f32 GEMV (test_q8_gemv_f32_one_row)."""
    B, N = 4, 128
    a = rnd(185, (M, K))
    ws = [q8(rnd(186 + s, (N, K), 0.02)) for s in range(B)]
    dw = hip.DeviceBuffer.of(np.concatenate(ws))
    outs = []
    for dt, host in ((abi.F32, a), (abi.F16, a.astype(np.float16).view(np.uint16))):
        da, dc = hip.DeviceBuffer.of(np.ascontiguousarray(host)), hip.DeviceBuffer(B * M * N * 4)
        hip.q8_batched_dev(dt, da.ptr, dw.ptr, dc.ptr, B, M, N, K, 0, ws[0].nbytes, M * N)
        hip.synchronize()
        outs.append(dc.download(np.float32, (B, M, N)))
        da.free()
        dc.free()
    dw.free()
    assert np.array_equal(outs[0].view(np.uint32), outs[1].view(np.uint32))
    for s in range(B):
        assert_f32_close(outs[0][s], ref_q8(a, ws[s], K, N, nt=True), what=f"slice {s}")


@pytest.mark.parametrize("K,N", [(256, 2048), (1024, 1024), (1024, 3072), (4096, 1024),
                                 (512, 80)])
def test_q8_gemv_f32_one_row(env, K, N):
    """One f32 activation row (q8_gemv): products a * q * scale in f32, no
    rounding to f16, so within a few f32 ulps of the oracle's sums (the
    order differs); bias + GELU and a residual in the epilogue; as one
    launch and as a batch of weight copies sharing the row (K > 256; a
    batch of K = 256 runs the tiled f16 GEMM); rows far outside the f16
    range need no factor. With SAM3_HIP_GEMV_F32=0 the
    f16 MFMA stream runs instead, within the f16 bound."""
    O = oracle()
    B = 3
    for scale in (1.0, 1e6, 1e-7):
        a = rnd(700 + K, (1, K)) * np.float32(scale)
        ws = [q8(rnd(701 + s, (N, K), 0.02)) for s in range(B)]
        bias = rnd(704, N, 0.1)
        refs = [ref_q8(a, w, K, N, nt=True) for w in ws]
        tol = 1e-5 * np.sqrt(K / 256)
        c = hip.matmul(a, abi.F32, ws[0], abi.Q8_0, abi.F32, 1, N, K, flags=hip.B_NT)
        err = np.max(np.abs(c - refs[0])) / np.max(np.abs(refs[0]))
        assert err <= tol, (scale, err)
        cb = hip.matmul(a, abi.F32, ws[0], abi.Q8_0, abi.F32, 1, N, K, bias=bias,
                        flags=hip.B_NT | hip.BIAS | hip.GELU)
        assert_f32_close(cb, O.gelu(O.bias_add(refs[0], bias, "f32"), "f32").reshape(1, N),
                         what=f"gemv bias gelu {scale}")
        dw = hip.DeviceBuffer.of(np.concatenate(ws))
        da, dc = hip.DeviceBuffer.of(a), hip.DeviceBuffer(B * N * 4)
        hip.q8_batched_dev(abi.F32, da.ptr, dw.ptr, dc.ptr, B, 1, N, K, 0, ws[0].nbytes, N)
        hip.synchronize()
        cbat = dc.download(np.float32, (B, 1, N))
        for s_ in (da, dw, dc):
            s_.free()
        if K == 256:
            # a batch of K = 256 weights runs the tiled f16 GEMM instead
            for s_ in range(B):
                assert_f32_close(cbat[s_], refs[s_], what=f"batched K=256 slice {s_} {scale}")
            continue
        assert np.array_equal(cbat[0].view(np.uint32), c.view(np.uint32))
        for s_ in range(B):
            e = np.max(np.abs(cbat[s_] - refs[s_])) / np.max(np.abs(refs[s_]))
            assert e <= tol, (scale, s_, e)
    env.set("SAM3_HIP_GEMV_F32", 0)
    c16 = hip.matmul(a, abi.F32, ws[0], abi.Q8_0, abi.F32, 1, N, K, flags=hip.B_NT)
    assert_f32_close(c16, refs[0], what="f16 stream")


@pytest.mark.parametrize("K,N,B,shared", [(1024, 1024, 20, True), (4096, 1024, 5, False),
                                           (512, 256, 70, True), (512, 2048, 9, False),
                                           (1024, 2048, 20, True), (256, 256, 130, False),
                                           (256, 2048, 17, True), (768, 1024, 37, False),
                                           (1536, 2048, 19, True)])
def test_q8_gemv_tasks_persistent_batch(env, K, N, B, shared):
    """A batch of one-row GEMVs with at least 256 (copy, 64- or 128-row
    group) tasks runs on the persistent q8_gemv_tasks (one workgroup per
    CU, workgroups taking one or several tasks; 128-row groups up to
    K = 1024): the same arithmetic as the one-workgroup-per-task GEMV, so
    the same bits as each copy launched on its own and (K > 256) as
    SAM3_HIP_GEMV_TASKS=0, or within a few ulps where the chunks split k
    over the waves differently; bias and GELU in the epilogue;
    the activations shared (stride 0) or one row per copy; within f32
    rounding of the oracle."""
    O = oracle()
    a = rnd(720 + K, (1 if shared else B, K))
    ws = [q8(rnd(721 + s_, (N, K), 0.02)) for s_ in range(B)]
    bias = rnd(722, N, 0.1)
    dw = hip.DeviceBuffer.of(np.concatenate(ws))
    da, db = hip.DeviceBuffer.of(a), hip.DeviceBuffer.of(bias)

    def run():
        dc = hip.DeviceBuffer(B * N * 4)
        hip.q8_batched_dev(abi.F32, da.ptr, dw.ptr, dc.ptr, B, 1, N, K, 0 if shared else K,
                           ws[0].nbytes, N, bias_ptr=db.ptr, flags=hip.BIAS | hip.GELU)
        hip.synchronize()
        c = dc.download(np.float32, (B, N))
        dc.free()
        return c

    c = run()
    # 128-row tasks in 8-block chunks run up to K = 1024 when N / 128
    # groups make 256 tasks; a launch of one copy (and the per-task GEMV)
    # takes 16-block chunks when K % 512 == 0: the same sums split over
    # the waves otherwise, so a few ulps apart
    same = not (K <= 1024 and K % 512 == 0 and (N // 128) * B >= 256)
    if K > 256:
        # (without the persistent kernel a batch of K = 256 runs the
        # tiled f16 GEMM)
        env.set("SAM3_HIP_GEMV_TASKS", 0)
        c0 = run()
        if same:
            assert np.array_equal(c.view(np.uint32), c0.view(np.uint32))
        else:
            assert np.max(np.abs(c - c0)) <= 1e-5 * np.max(np.abs(c0))
    for s_ in range(B):
        row = a[0 if shared else s_].reshape(1, K)
        one = hip.matmul(row, abi.F32, ws[s_], abi.Q8_0, abi.F32, 1, N, K, bias=bias,
                         flags=hip.B_NT | hip.BIAS | hip.GELU).reshape(N)
        if same:
            assert np.array_equal(c[s_].view(np.uint32), one.view(np.uint32)), s_
        else:
            assert np.max(np.abs(c[s_] - one)) <= 1e-5 * np.max(np.abs(one)), s_
        ref = O.gelu(O.bias_add(ref_q8(row, ws[s_], K, N, nt=True), bias, "f32"), "f32")
        assert_f32_close(c[s_].reshape(1, N), np.asarray(ref).reshape(1, N), what=f"task batch {s_}")
    for b_ in (da, db, dw):
        b_.free()


@pytest.mark.parametrize("M,K,N,B,shared", [(8, 256, 1024, 32, True), (8, 1024, 1024, 33, False),
                                             (2, 512, 2048, 16, True), (13, 256, 256, 130, False),
                                             (16, 2048, 1024, 32, True), (5, 1024, 4096, 8, False),
                                             (4, 768, 2048, 19, False), (11, 768, 1024, 37, True)])
def test_q8_stream_tasks_persistent_batch(env, M, K, N, B, shared):
    """A batch of 2-16 f32 activation rows over weight copies with at
    least 256 (copy, 128-row group) tasks runs on the persistent
    q8_stream_tasks after the row-scaled f16 copy of the rows: every row
    within the f16-operand bound of the oracle (one row scaled past the
    f16 range, its factor undone in the epilogue), bias and GELU in the
    epilogue, the activations shared (stride 0) or one set per copy; and
    close to the path that runs without it (SAM3_HIP_GEMV_TASKS=0: the
    tiled GEMM, whose q * scale is rounded to f16, or the per-task
    q8_stream)."""
    O = oracle()
    a = rnd(730 + M, (1 if shared else B, M, K))
    a[:, M // 2] *= np.float32(1e6)
    ws = [q8(rnd(731 + s_, (N, K), 0.02)) for s_ in range(B)]
    bias = rnd(732, N, 0.1)
    dw = hip.DeviceBuffer.of(np.concatenate(ws))
    da, db = hip.DeviceBuffer.of(a), hip.DeviceBuffer.of(bias)

    def run():
        dc = hip.DeviceBuffer(B * M * N * 4)
        hip.q8_batched_dev(abi.F32, da.ptr, dw.ptr, dc.ptr, B, M, N, K, 0 if shared else M * K,
                           ws[0].nbytes, M * N, bias_ptr=db.ptr, flags=hip.BIAS | hip.GELU)
        hip.synchronize()
        c = dc.download(np.float32, (B, M, N))
        dc.free()
        return c

    c = run()
    for s_ in range(B):
        rows = a[0 if shared else s_]
        ref = O.gelu(O.bias_add(ref_q8(rows, ws[s_], K, N, nt=True), bias, "f32"), "f32")
        ref = np.asarray(ref).reshape(M, N)
        for m in range(M):
            # rows of very different scales: each against its own size
            assert_f32_close(c[s_, m:m + 1], ref[m:m + 1], what=f"task batch {s_} row {m}")
    env.set("SAM3_HIP_GEMV_TASKS", 0)
    c0 = run()
    for m in range(M):
        assert_f32_close(c[:, m], c0[:, m], what=f"tasks against the other path, row {m}")
    for b_ in (da, db, dw):
        b_.free()


def test_q8_batched_falls_back_per_slice():
    """M > 128 is not a skinny problem: one launch per slice, same result."""
    B, M, N, K = 2, 160, 64, 256
    a = rnd(190, (B, M, K))
    ws = [q8(rnd(191 + s, (N, K), 0.02)) for s in range(B)]
    da, dw = hip.DeviceBuffer.of(a), hip.DeviceBuffer.of(np.concatenate(ws))
    dc = hip.DeviceBuffer(B * M * N * 4)
    hip.q8_batched_dev(abi.F32, da.ptr, dw.ptr, dc.ptr, B, M, N, K, M * K, ws[0].nbytes, M * N)
    hip.synchronize()
    c = dc.download(np.float32, (B, M, N))
    for s in range(B):
        assert_f32_close(c[s], ref_q8(a[s], ws[s], K, N, nt=True), what=f"fallback slice {s}")


def test_q8_nt_ragged_k_blocks_straddle_rows():
    """W [N,K] with K % 32 != 0: blocks run over the flat index and cross
    row boundaries (src/core/quant.c quantizes the tensor flat)."""
    M, N, K = 70, 40, 72
    a = rnd(140, (M, K))
    w = q8(rnd(141, (N, K), 0.02))
    ref = ref_q8(a, w, K, N, nt=True)
    assert_f32_close(hip.matmul(a, abi.F32, w, abi.Q8_0, abi.F32, M, N, K, flags=hip.B_NT),
                     ref, what="q8 nt ragged")
    g = hip.matmul(a, abi.F32, w, abi.Q8_0, abi.F32, M, N, K, flags=hip.B_NT, path=GENERIC)
    assert np.array_equal(bits32(g), bits32(ref))


def test_q8_one_hot_rows_exact_dequant():
    """A = e_k rows select dequantized weight rows: the skinny path's
    q*scale in f32 is exact for one-hot A (1.0 is exact in f16)."""
    O = oracle()
    K, N = 128, 48
    w = q8(rnd(150, (N, K), 0.02))
    deq = O.q8_dequantize(w, N * K).reshape(N, K)
    rows = [0, 31, 32, 127]
    a = np.eye(K, dtype=np.float32)[rows]
    c = hip.matmul(a, abi.F32, w, abi.Q8_0, abi.F32, len(rows), N, K, flags=hip.B_NT,
                   path=SKINNY)
    assert np.array_equal(c, deq[:, rows].T)


def test_q8_paths_agree():
    M, N, K = 96, 160, 512
    a = rnd(160, (M, K))
    w = q8(rnd(161, (N, K), 0.02))
    outs = [hip.matmul(a, abi.F32, w, abi.Q8_0, abi.F32, M, N, K, flags=hip.B_NT, path=p)
            for p in (MFMA, SKINNY, GENERIC)]
    assert_f32_close(outs[0], outs[2], what="mfma vs generic")
    assert_f32_close(outs[1], outs[2], what="skinny vs generic")


# ------------------------------------------------------- batched attention
@pytest.mark.parametrize("B,S,D", [(3, 64, 64), (2, 100, 64), (4, 576, 64)])
def test_batched_attention_matmuls(B, S, D):
    """QK^T ([B,S,D] x [B,S,D]^T) and PV ([B,S,S] x [B,S,D]) per slice,
    as gh_multihead_attention builds them (graph_helpers.c:808-843)."""
    O = oracle()
    q = O.f32_to_bf16(rnd(170, (B, S, D)) / 8).reshape(B, S, D)
    k = O.f32_to_bf16(rnd(171, (B, S, D)) / 8).reshape(B, S, D)
    v = O.f32_to_bf16(rnd(172, (B, S, D)) / 8).reshape(B, S, D)
    s = hip.batched(abi.BF16, q, k, B, S, S, D, b_nt=True)
    assert_bf16_close(s, O.matmul_bf16_batched(q, k, b_nt=True, threads=8), what="QK^T")
    p = O.f32_to_bf16(rnd(173, (B, S, S)) / 8).reshape(B, S, S)
    o = hip.batched(abi.BF16, p, v, B, S, D, S, b_nt=False)
    assert_bf16_close(o, O.matmul_bf16_batched(p, v, b_nt=False, threads=8), what="PV")


@pytest.mark.parametrize("dt", [abi.BF16, abi.F16], ids=["bf16", "f16"])
@pytest.mark.parametrize("B,S", [(1296, 576), (16, 5184), (300, 384)])
def test_batched_scores_persistent_kernel(env, dt, B, S):
    """Q K^T with K = 64 over many slices (the ViT's windowed and global
    attention scores) runs the persistent one-k-step kernel: the same bits
    as the per-tile kernel (SAM3_HIP_DL_CFG=24), and a sample of slices
    against the oracle."""
    O = oracle()
    D = 64
    q = rnd(175, (B, S, D)) / 8
    k = rnd(176, (B, S, D)) / 8
    if dt == abi.BF16:
        q, k = (O.f32_to_bf16(x).reshape(x.shape) for x in (q, k))
    else:
        q, k = q.astype(np.float16), k.astype(np.float16)
    env.unset("SAM3_HIP_DL_CFG")
    got = hip.batched(dt, q, k, B, S, S, D, b_nt=True)
    env.set("SAM3_HIP_DL_CFG", 24)
    ref_tile = hip.batched(dt, q, k, B, S, S, D, b_nt=True)
    env.unset("SAM3_HIP_DL_CFG")
    assert np.array_equal(got.view(np.uint16), ref_tile.view(np.uint16))
    pick = np.unique(np.array([0, B // 2, B - 1]))
    if dt == abi.BF16:
        ref = O.matmul_bf16_batched(q[pick], k[pick], b_nt=True, threads=8)
        assert_bf16_close(got[pick], ref, what=f"QK^T {B}x{S}")
    else:
        qf, kf = q[pick].astype(np.float64), k[pick].astype(np.float64)
        ref = np.einsum("bsd,btd->bst", qf, kf).astype(np.float16)
        assert_f16_close(got[pick].view(np.uint16), ref.view(np.uint16), what=f"QK^T f16 {B}x{S}")


@pytest.mark.parametrize("dt", [abi.BF16, abi.F16], ids=["bf16", "f16"])
@pytest.mark.parametrize("B,S,D", [(120, 576, 64), (16, 5184, 64), (90, 384, 128)])
def test_batched_pv_transposing_reads(env, dt, B, S, D):
    """P V with V stored [keys, head dim] (B as [K, N], N <= 128) over many
    slices runs the direct-to-LDS kernel that reads V's fragments with
    transposing LDS reads: the same bits as the register-staged [K, N]
    kernel (taken when SAM3_HIP_DL_CFG is set), and a sample of slices
    against the oracle."""
    O = oracle()
    pm = rnd(185, (B, S, S)) / 8
    v = rnd(186, (B, S, D)) / 8
    if dt == abi.BF16:
        pm, v = (O.f32_to_bf16(x).reshape(x.shape) for x in (pm, v))
    else:
        pm, v = pm.astype(np.float16), v.astype(np.float16)
    env.unset("SAM3_HIP_DL_CFG")
    got = hip.batched(dt, pm, v, B, S, D, S, b_nt=False)
    env.set("SAM3_HIP_DL_CFG", 2)
    staged = hip.batched(dt, pm, v, B, S, D, S, b_nt=False)
    env.unset("SAM3_HIP_DL_CFG")
    assert np.array_equal(got.view(np.uint16), staged.view(np.uint16))
    pick = np.unique(np.array([0, B // 2, B - 1]))
    if dt == abi.BF16:
        ref = O.matmul_bf16_batched(pm[pick], v[pick], b_nt=False, threads=8)
        assert_bf16_close(got[pick], ref, what=f"PV {B}x{S}x{D}")
    else:
        ref = np.matmul(pm[pick].astype(np.float64), v[pick].astype(np.float64)).astype(np.float16)
        assert_f16_close(got[pick].view(np.uint16), ref.view(np.uint16), what=f"PV f16 {B}x{S}x{D}")


@pytest.mark.parametrize("dt,ct,M,N,K", [
    (abi.BF16, abi.BF16, 5184, 4096, 1024),
    (abi.BF16, abi.F32, 5000, 2560, 320),
    (abi.F16, abi.F16, 5000, 2560, 320),
    (abi.F16, abi.F32, 1000, 16384, 128),
], ids=["fc1-bf16", "ragged-bf16-f32", "ragged-f16", "wide-f16-f32"])
def test_wide_kn_weight_transposing_reads(env, dt, ct, M, N, K):
    """A 16-bit product with W stored [K, N] and N a multiple of 256 runs
    the 192x256 direct-to-LDS tile that reads W's fragments with
    transposing LDS reads (rows past M, when M is not a multiple of 192,
    read zeros and are not stored): the same bits as the register-staged
    [K, N] kernel (taken when SAM3_HIP_DL_CFG is set), and a row sample
    against the oracle."""
    O = oracle()
    a = rnd(187, (M, K))
    w = rnd(188, (K, N), 0.05)
    if dt == abi.BF16:
        a, w = (O.f32_to_bf16(x).reshape(x.shape) for x in (a, w))
        dec = bf16_to_f32
    else:
        a, w = a.astype(np.float16), w.astype(np.float16)
        dec = lambda x: x.astype(np.float32)
    env.unset("SAM3_HIP_DL_CFG")
    got = hip.matmul(a, dt, w, dt, ct, M, N, K, path=MFMA)
    env.set("SAM3_HIP_DL_CFG", 2)
    staged = hip.matmul(a, dt, w, dt, ct, M, N, K, path=MFMA)
    env.unset("SAM3_HIP_DL_CFG")
    assert np.array_equal(got.view(np.uint8), staged.view(np.uint8))
    rows = _row_sample(M, n=24)
    if ct == abi.F32:
        ref = O.matmul_f32(dec(a[rows]), dec(w), 8)
        assert_f32_close(got[rows], ref, what=f"[K,N] {M}x{N}x{K} f32 out")
    elif dt == abi.BF16:
        assert_bf16_close(got[rows], ref_linear("bf16", a[rows], w), what=f"[K,N] {M}x{N}x{K}")
    else:
        assert_f16_close(got[rows].view(np.uint16), ref_linear("f16", a[rows].view(np.uint16), w.view(np.uint16)),
                         what=f"[K,N] f16 {M}x{N}x{K}")


# -------------------------------------------- full-size shapes, row sample
def _row_sample(M, n=48, seed=7):
    rng = np.random.default_rng(seed)
    return np.unique(np.concatenate([[0, M - 1], rng.integers(0, M, n)]))


@pytest.mark.parametrize("which", ["fc1", "fc2"])
def test_config2_bf16_full_size_rows(which):
    """Config 2 at full size on the tiled path; rows are independent, so
    a row sample of A against the same W is checked with the oracle."""
    O = oracle()
    M, (K, N) = 5184, ((1024, 4096) if which == "fc1" else (4096, 1024))
    a = O.f32_to_bf16(rnd(180, (M, K))).reshape(M, K)
    w = O.f32_to_bf16(rnd(181, (N, K), 0.02)).reshape(N, K)
    bias = O.f32_to_bf16(rnd(182, N, 0.01))
    c = hip.matmul(a, abi.BF16, w, abi.BF16, abi.BF16, M, N, K, bias=bias,
                   flags=hip.B_NT | hip.BIAS | hip.GELU)
    rows = _row_sample(M)
    ref = ref_linear("bf16", a[rows], w, bias, True, b_nt=True)
    g, r = bf16_to_f32(c[rows]), bf16_to_f32(ref)
    assert np.abs(g - r).max() <= 2e-2, f"max abs {np.abs(g - r).max()}"


def test_config1_q8_full_size_rows():
    M, N, K = 5184, 1024, 1024
    a = rnd(0, (M, K))
    w = q8(rnd(1, (N, K), 0.02))
    c = hip.matmul(a, abi.F32, w, abi.Q8_0, abi.F32, M, N, K, flags=hip.B_NT)
    rows = _row_sample(M)
    assert_f32_close(c[rows], ref_q8(a[rows], w, K, N, nt=True), what="config 1")


# ------------------------------------------------------------- edge cases
def test_degenerate_sizes():
    a = np.zeros((1, 1), np.float32)
    lib = hip.load()
    # M == 0 or N == 0 is a no-op
    assert lib.sam3_hip_matmul(abi.F32, 1, abi.F32, 1, abi.F32, 1, 0, 4, 4, None, 0, None) == abi.OK
    # K == 0: C = 0 (the reference zeroes C and adds nothing)
    da, db, dc = hip.DeviceBuffer(16), hip.DeviceBuffer(16), hip.DeviceBuffer.of(np.ones(4, np.float32))
    hip.matmul_dev(abi.F32, da.ptr, abi.F32, db.ptr, abi.F32, dc.ptr, 2, 2, 0)
    hip.synchronize()
    assert np.all(dc.download(np.float32, 4) == 0)
    c = hip.matmul(np.float32([[2.0]]), abi.F32, np.float32([[3.0]]), abi.F32, abi.F32, 1, 1, 1)
    assert c[0, 0] == 6.0
    del a


def test_one_by_n_and_n_by_one():
    O = oracle()
    a = rnd(190, (1, 300))
    b = rnd(191, (300, 1))
    c = hip.matmul(a, abi.F32, b, abi.F32, abi.F32, 1, 1, 300)
    assert_f32_close(c, O.matmul_f32(a, b), what="1x1")
