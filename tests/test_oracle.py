"""Pins the CPU oracle (oracle/sam3_oracle.c) before it is trusted.

Three kinds of evidence, so that a dropped term, a wrong sign/index or a
transposed operand fails at least one:
  1. golden vectors written by the real reference (tests/golden/), bit-exact;
  2. direct bit-exact comparison with oracle/_ref/libsam3ref.so (the
     reference's sources compiled in place) on fresh seeded inputs, when
     that library is built (skipped on the GPU box, which has no sources);
  3. closed forms: the reference tests' known answers, identity and
     one-hot products, exhaustive conversion sweeps, float64 brute force.
"""
from pathlib import Path

import numpy as np
import pytest

from oracle_bind import Oracle, Ref, have_ref
from sam3_amd import abi, synth

GOLD = np.load(Path(__file__).parent / "golden" / "matmul_golden.npz")


@pytest.fixture(scope="module")
def O():
    return Oracle()


@pytest.fixture(scope="module")
def R():
    if not have_ref():
        pytest.skip("oracle/_ref not built (reference sources absent)")
    r = Ref()
    yield r
    r.close()


def bits32(x):
    return np.ascontiguousarray(x, np.float32).view(np.uint32)


# ------------------------------------------------------------- transpose
TR_SHAPES = [(1, 1), (1, 7), (7, 1), (13, 37), (64, 96), (129, 257)]


@pytest.mark.parametrize("R_,C_", TR_SHAPES)
def test_transpose_is_numpy_transpose(O, R_, C_):
    """oracle_transpose_u16 / _f32 (cpu_transpose.c:355-366's 2-D swap)
    move every element bit for bit to [c][r]: arbitrary bit patterns
    (NaN payloads included) against numpy's .T."""
    rng = np.random.default_rng(R_ * 1000 + C_)
    x16 = rng.integers(0, 1 << 16, (R_, C_), dtype=np.uint32).astype(np.uint16)
    assert np.array_equal(O.transpose_u16(x16), x16.T)
    x32 = rng.integers(0, 1 << 32, (R_, C_), dtype=np.uint64).astype(np.uint32)
    got = O.transpose_f32(x32.view(np.float32))
    assert np.array_equal(got.view(np.uint32), x32.T)


@pytest.mark.parametrize("R_,C_", TR_SHAPES)
def test_transpose_matches_reference_kernel(O, R, R_, C_):
    """The same against the reference's own cpu_kernel_transpose on a 2-D
    TRANSPOSE node (its default last-two-axes swap), 16-bit and f32."""
    rng = np.random.default_rng(R_ * 7 + C_)
    x16 = rng.integers(0, 1 << 16, (R_, C_), dtype=np.uint32).astype(np.uint16)
    rc, ref = R.run("cpu_kernel_transpose", abi.OP_TRANSPOSE, [(abi.BF16, [R_, C_], x16)],
                    abi.BF16, (C_, R_), np.uint16, threads=3)
    assert rc == 0 and np.array_equal(O.transpose_u16(x16), ref)
    x32 = rng.integers(0, 1 << 32, (R_, C_), dtype=np.uint64).astype(np.uint32).view(np.float32)
    rc, ref = R.run("cpu_kernel_transpose", abi.OP_TRANSPOSE, [(abi.F32, [R_, C_], x32)],
                    abi.F32, (C_, R_), np.float32, threads=3)
    assert rc == 0
    assert np.array_equal(O.transpose_f32(x32).view(np.uint32), ref.view(np.uint32))


# ---------------------------------------------------------------- golden
def test_golden_q8_quantize(O):
    qx = GOLD["quant_x"]
    assert np.array_equal(O.q8_quantize(qx), GOLD["quant_blocks"])
    assert np.array_equal(bits32(O.q8_dequantize(GOLD["quant_blocks"], qx.size)),
                          bits32(GOLD["quant_deq"]))


@pytest.mark.parametrize("name", ["q8_a", "q8_b", "q8_c", "q8_t"])
def test_golden_q8_matmul(O, name):
    M, K, N = GOLD[f"{name}_shape"]
    for threads in (1, 3):
        c = O.matmul_q8(GOLD[f"{name}_a"], GOLD[f"{name}_b"], int(K), int(N), threads)
        assert np.array_equal(bits32(c), bits32(GOLD[f"{name}_c"]))


def test_golden_q8_nt(O):
    M, K, N = (int(v) for v in GOLD["q8nt_shape"])
    c = O.matmul_q8_nt(GOLD["q8nt_a"], GOLD["q8nt_w"], K, N, threads=2)
    assert np.array_equal(bits32(c), bits32(GOLD["q8nt_c"]))


def test_golden_dense(O):
    assert np.array_equal(O.matmul_bf16(GOLD["bf16_a"], GOLD["bf16_b"], 2), GOLD["bf16_c"])
    assert np.array_equal(O.matmul_f16(GOLD["f16_a"], GOLD["f16_b"], 2), GOLD["f16_c"])
    assert np.array_equal(bits32(O.matmul_f32(GOLD["f32_a"], GOLD["f32_b"])), bits32(GOLD["f32_c"]))
    assert np.array_equal(bits32(O.matmul_f32(GOLD["f32b_a"], GOLD["f32b_b"], 4)),
                          bits32(GOLD["f32b_c"]))


def test_golden_epilogues(O):
    x, bias = GOLD["ep_x"], GOLD["ep_bias"]
    assert np.array_equal(bits32(O.bias_add(x, bias, "f32")), bits32(GOLD["ep_add_f32"]))
    xb, bb = O.f32_to_bf16(x).reshape(x.shape), O.f32_to_bf16(bias)
    assert np.array_equal(O.bias_add(xb, bb, "bf16"), GOLD["ep_add_bf16"])
    xh, bh = O.f32_to_fp16(x).reshape(x.shape), O.f32_to_fp16(bias)
    assert np.array_equal(O.bias_add(xh, bh, "f16"), GOLD["ep_add_f16"])
    gx = GOLD["gelu_x"]
    assert np.array_equal(bits32(O.gelu(gx, "f32")), bits32(GOLD["gelu_f32"]))
    assert np.array_equal(O.gelu(O.f32_to_bf16(gx), "bf16"), GOLD["gelu_bf16"])
    assert np.array_equal(O.gelu(O.f32_to_fp16(gx), "f16"), GOLD["gelu_f16"])


def test_golden_conversions(O):
    p = GOLD["cvt_f32"]
    assert np.array_equal(O.f32_to_bf16(p), GOLD["cvt_bf16"])
    assert np.array_equal(O.f32_to_fp16(p), GOLD["cvt_fp16"])


# ------------------------------------------------------ reference (_ref)
def test_ref_conversions_exhaustive(O, R):
    allp = np.arange(65536, dtype=np.uint16)
    assert np.array_equal(bits32(O.bf16_to_f32(allp)),
                          bits32(R.cast(allp, abi.BF16, abi.F32, np.float32)))
    assert np.array_equal(bits32(O.fp16_to_f32(allp)),
                          bits32(R.cast(allp, abi.F16, abi.F32, np.float32)))
    rng = np.random.default_rng(5)
    pats = rng.integers(0, 2 ** 32, 1 << 20, dtype=np.uint64).astype(np.uint32).view(np.float32)
    assert np.array_equal(O.f32_to_bf16(pats), R.cast(pats, abi.F32, abi.BF16, np.uint16))
    assert np.array_equal(O.f32_to_fp16(pats), R.cast(pats, abi.F32, abi.F16, np.uint16))


@pytest.mark.parametrize("M,K,N", [(33, 160, 64), (8, 64, 33), (1, 1024, 96), (70, 96, 1)])
def test_ref_q8(O, R, M, K, N):
    a = synth.randn(100 + M, (M, K))
    w = synth.randn(200 + N, (K, N), 0.02)
    b = R.q8_quantize(w)
    assert np.array_equal(O.q8_quantize(w), b)
    assert np.array_equal(bits32(O.matmul_q8(a, b, K, N, 4)), bits32(R.matmul_q8(a, b, K, N, 4)))


def test_ref_q8_nt_columns(O, R):
    M, K, N = 9, 192, 17
    a = synth.randn(300, (M, K))
    w = synth.randn(301, (N, K), 0.05)
    wb = O.q8_quantize(w)
    c = O.matmul_q8_nt(a, wb, K, N)
    row = K // 32 * 36
    for n in range(N):
        assert np.array_equal(bits32(c[:, n:n + 1]), bits32(R.matmul_q8(a, wb[n * row:(n + 1) * row], K, 1)))


@pytest.mark.parametrize("M,K,N", [(17, 130, 9), (64, 64, 64)])
def test_ref_dense(O, R, M, K, N):
    a32 = synth.randn(400 + K, (M, K))
    b32 = synth.randn(500 + N, (K, N))
    ab, bb = O.f32_to_bf16(a32).reshape(M, K), O.f32_to_bf16(b32).reshape(K, N)
    assert np.array_equal(O.matmul_bf16(ab, bb, 3), R.matmul_bf16(ab, bb, 3))
    ah, bh = O.f32_to_fp16(a32).reshape(M, K), O.f32_to_fp16(b32).reshape(K, N)
    assert np.array_equal(O.matmul_f16(ah, bh, 3), R.matmul_f16(ah, bh, 3))
    assert np.array_equal(bits32(O.matmul_f32(a32, b32, 3)), bits32(R.matmul_f32(a32, b32, 3)))


def test_ref_dispatch_q8_routing(R):
    """tests/test_dispatch_q8.c:28-81: F32 x Q8_0 routes to the Q8 kernel;
    a BF16 x Q8_0 node is refused with SAM3_EDTYPE (cpu_dispatch.c:643-655)."""
    M, K, N = 4, 32, 4
    a = (np.arange(M * K, dtype=np.float32) * np.float32(0.01)).reshape(M, K)
    w = (np.arange(K * N, dtype=np.float32) * np.float32(0.01)).reshape(K, N)
    b = R.q8_quantize(w)
    rc, c = R.run("dispatch", abi.OP_MATMUL, [(abi.F32, [M, K], a), (abi.Q8_0, [K, N], b)],
                  abi.F32, (M, N), np.float32)
    assert rc == abi.OK and np.count_nonzero(c) > 0
    ab = np.zeros((M, K), np.uint16)
    rc, _ = R.run("dispatch", abi.OP_MATMUL, [(abi.BF16, [M, K], ab), (abi.Q8_0, [K, N], b)],
                  abi.BF16, (M, N), np.uint16)
    assert rc == abi.EDTYPE


# ------------------------------------------------------------ closed forms
def test_known_answer_f32(O):
    """tests/test_cpu_kernels.c:474-500: [1,2,3;4,5,6]@[7,8;9,10;11,12]."""
    a = np.array([[1, 2, 3], [4, 5, 6]], np.float32)
    b = np.array([[7, 8], [9, 10], [11, 12]], np.float32)
    assert O.matmul_f32(a, b).tolist() == [[58, 64], [139, 154]]


def test_identity_all_dtypes(O):
    a = synth.randn(7, (12, 12))
    eye = np.eye(12, dtype=np.float32)
    assert np.array_equal(O.matmul_f32(a, eye), a)
    ab = O.f32_to_bf16(a).reshape(12, 12)
    assert np.array_equal(O.matmul_bf16(ab, O.f32_to_bf16(eye).reshape(12, 12)), ab)
    ah = O.f32_to_fp16(a).reshape(12, 12)
    assert np.array_equal(O.matmul_f16_acc32(ah, O.f32_to_fp16(eye).reshape(12, 12)), ah)


def test_q8_invariants(O):
    x = synth.randn(8, 32 * 40, 0.3)
    blk = O.q8_quantize(x).reshape(-1, 36)
    scale = blk[:, :4].copy().view(np.float32).ravel()
    q = blk[:, 4:].view(np.int8).astype(np.int32)
    amax = np.abs(x.reshape(-1, 32)).max(1)
    assert np.array_equal(scale, (amax / np.float32(127.0)).astype(np.float32))
    assert np.abs(q).max() <= 127
    # the element reaching amax quantizes to +-127
    idx = np.abs(x.reshape(-1, 32)).argmax(1)
    assert np.all(np.abs(q[np.arange(len(idx)), idx]) == 127)
    # tests/test_quant.c:36-59 block counts / sizes
    assert [O.lib.oracle_q8_block_count(n) for n in (32, 64, 1024, 1, 33, 63)] == [1, 2, 32, 1, 2, 2]
    assert [O.lib.oracle_q8_nbytes(n) for n in (32, 64, 33)] == [36, 72, 72]
    # zero block -> scale 0 and zero data (tests/test_quant.c:80-94)
    z = O.q8_quantize(np.zeros(32, np.float32))
    assert np.all(z == 0)
    # hand-built blocks dequantize exactly (tests/test_metal.c:950-1011)
    hb = np.zeros((2, 36), np.uint8)
    hb[0, :4] = np.frombuffer(np.float32(0.5).tobytes(), np.uint8)
    hb[0, 4:] = np.arange(32, dtype=np.int8).view(np.uint8)
    hb[1, :4] = np.frombuffer(np.float32(0.25).tobytes(), np.uint8)
    hb[1, 4:] = (-(np.arange(32) + 1)).astype(np.int8).view(np.uint8)
    exp = np.concatenate([np.arange(32) * 0.5, -(np.arange(32) + 1) * 0.25]).astype(np.float32)
    assert np.array_equal(O.q8_dequantize(hb.ravel(), 64), exp)


def test_q8_one_hot_rows_pick_dequantized_weights(O):
    """A = e_k picks row k of deq(B) exactly: 1*q*s == q*s in f32."""
    K, N = 96, 70
    w = synth.randn(9, (K, N), 0.02)
    b = O.q8_quantize(w)
    deq = O.q8_dequantize(b, K * N).reshape(K, N)
    a = np.eye(K, dtype=np.float32)[[0, 5, 31, 32, 95]]
    assert np.array_equal(O.matmul_q8(a, b, K, N), deq[[0, 5, 31, 32, 95]])
    wn = synth.randn(10, (N, K), 0.02)
    bn = O.q8_quantize(wn)
    deqn = O.q8_dequantize(bn, K * N).reshape(N, K)
    assert np.array_equal(O.matmul_q8_nt(a, bn, K, N), deqn[:, [0, 5, 31, 32, 95]].T)


def test_q8_brute_force_float64(O):
    M, K, N = 6, 128, 24
    a = synth.randn(11, (M, K))
    w = synth.randn(12, (N, K), 0.02)
    bn = O.q8_quantize(w)
    deq = O.q8_dequantize(bn, N * K).reshape(N, K).astype(np.float64)
    exact = a.astype(np.float64) @ deq.T
    got = O.matmul_q8_nt(a, bn, K, N)
    assert np.max(np.abs(got - exact)) <= 1e-5 * np.max(np.abs(exact))


def test_f16_acc32_pins(O):
    """No reference kernel accumulates fp16 in f32, so: (1) small-integer
    operands make every product and partial sum exact, giving an integer
    closed form that fails on any index/transposition slip; (2) float64
    brute force at K=4096 with a bound an fp16 accumulator cannot meet."""
    rng = np.random.default_rng(3)
    M, K, N = 9, 64, 11
    ai = rng.integers(-4, 5, (M, K)).astype(np.float32)
    bi = rng.integers(-4, 5, (K, N)).astype(np.float32)
    got = O.fp16_to_f32(O.matmul_f16_acc32(O.f32_to_fp16(ai).reshape(M, K),
                                           O.f32_to_fp16(bi).reshape(K, N))).reshape(M, N)
    assert np.array_equal(got, ai @ bi)
    M, K, N = 4, 4096, 6
    a = O.f32_to_fp16(synth.randn(13, (M, K))).reshape(M, K)
    b = O.f32_to_fp16(synth.randn(14, (K, N), 0.02)).reshape(K, N)
    exact = (O.fp16_to_f32(a).reshape(M, K).astype(np.float64) @
             O.fp16_to_f32(b).reshape(K, N).astype(np.float64))
    got = O.fp16_to_f32(O.matmul_f16_acc32(a, b)).reshape(M, N)
    ulp = np.spacing(np.abs(exact).astype(np.float16)).astype(np.float64)
    assert np.all(np.abs(got - exact) <= 0.5 * ulp + 1e-6 * np.abs(exact).max())
    ref16 = O.fp16_to_f32(O.matmul_f16(a, b)).reshape(M, N)
    assert np.max(np.abs(ref16 - exact)) > np.max(np.abs(got - exact))


def test_batched_equals_slices(O):
    B, M, K, N = 3, 20, 16, 24
    a = O.f32_to_bf16(synth.randn(15, (B, M, K))).reshape(B, M, K)
    b_kn = O.f32_to_bf16(synth.randn(16, (B, K, N))).reshape(B, K, N)
    c = O.matmul_bf16_batched(a, b_kn, b_nt=False)
    for s in range(B):
        assert np.array_equal(c[s], O.matmul_bf16(a[s], b_kn[s]))
    b_nk = np.ascontiguousarray(np.transpose(b_kn, (0, 2, 1)))
    assert np.array_equal(O.matmul_bf16_batched(a, b_nk, b_nt=True), c)


# ------------------------------------------------------------------- SDPA
def test_golden_sdpa(O):
    q, k, v, m = GOLD["sdpa_q"], GOLD["sdpa_k"], GOLD["sdpa_v"], GOLD["sdpa_mask"]
    for threads in (1, 4):
        assert np.array_equal(bits32(O.sdpa(q, k, v, None, threads)), bits32(GOLD["sdpa_out"]))
        assert np.array_equal(bits32(O.sdpa(q, k, v, m, threads)), bits32(GOLD["sdpa_out_mask"]))


def test_ref_sdpa(O, R):
    q = synth.randn(81, (2, 50, 64)) / 2
    k = synth.randn(82, (2, 129, 64)) / 2
    v = synth.randn(83, (2, 129, 64))
    m = synth.randn(84, (50, 129))
    for mask in (None, m):
        assert np.array_equal(bits32(O.sdpa(q, k, v, mask, 3)), bits32(R.sdpa(q, k, v, mask, 2)))


def test_sdpa_closed_forms(O):
    """Zero queries give equal weights (the mean of V); one key gives that
    V row; a mask of -inf on all keys but one selects that key's V row
    exactly; random inputs match a float64 softmax."""
    BH, Sk, D = 2, 40, 64
    v = synth.randn(85, (BH, Sk, D))
    k = synth.randn(86, (BH, Sk, D))
    q0 = np.zeros((BH, 5, D), np.float32)
    mean = v.astype(np.float64).mean(axis=1, keepdims=True)
    assert np.allclose(O.sdpa(q0, k, v), np.broadcast_to(mean, (BH, 5, D)), atol=1e-6)
    one = O.sdpa(q0[:, :1], k[:, :1], v[:, :1])
    assert np.array_equal(one, v[:, :1])
    mask = np.full((5, Sk), -np.inf, np.float32)
    pick = [3, 0, 39, 17, 17]
    for i, j in enumerate(pick):
        mask[i, j] = 0.0
    q = synth.randn(87, (BH, 5, D))
    sel = O.sdpa(q, k, v, mask)
    for i, j in enumerate(pick):
        assert np.array_equal(sel[:, i], v[:, j])
    s = np.einsum("bqd,bkd->bqk", q.astype(np.float64), k.astype(np.float64)) / 8.0
    p = np.exp(s - s.max(axis=2, keepdims=True))
    ref = np.einsum("bqk,bkd->bqd", p / p.sum(axis=2, keepdims=True), v.astype(np.float64))
    assert np.max(np.abs(O.sdpa(q, k, v) - ref)) < 1e-5


# ------------------------------------------------------------- LayerNorm
def _kind_cast(O, x, kind):
    if kind == "f32":
        return np.ascontiguousarray(x, np.float32)
    conv = O.f32_to_bf16 if kind == "bf16" else O.f32_to_fp16
    return conv(x).reshape(np.shape(x))


def test_golden_layernorm(O):
    out = O.layernorm(GOLD["ln_x"], GOLD["ln_gamma"], GOLD["ln_beta"], "f32", threads=3)
    assert np.array_equal(bits32(out), bits32(GOLD["ln_out"]))


@pytest.mark.parametrize("kind", ["f32", "bf16", "f16"])
@pytest.mark.parametrize("affine", [2, 1, 0])
def test_ref_layernorm(O, R, kind, affine):
    x = synth.randn(91, (29, 160), 2.0, -1.0)
    g, b = synth.randn(92, (160,)), synth.randn(93, (160,))
    xi, gi, bi = (_kind_cast(O, t, kind) for t in (x, g, b))
    args = (gi if affine >= 1 else None, bi if affine >= 2 else None)
    a = O.layernorm(xi, *args, kind=kind, threads=4)
    r = R.layernorm(xi, *args, kind=kind)
    assert np.array_equal(a.view(np.uint8), r.view(np.uint8))


def test_layernorm_closed_forms(O):
    """Rows come out with mean 0 and variance var/(var + eps) (float64),
    a constant row gives exactly beta, and gamma/beta apply per column."""
    x = synth.randn(94, (16, 256), 3.0, 2.0)
    y = O.layernorm(x).astype(np.float64)
    assert np.max(np.abs(y.mean(axis=1))) < 1e-6
    var = x.astype(np.float64).var(axis=1)
    assert np.allclose(y.var(axis=1), var / (var + 1e-5), atol=1e-5)
    const = np.full((3, 64), 7.25, np.float32)
    beta = synth.randn(95, (64,))
    out = O.layernorm(const, np.ones(64, np.float32), beta)
    assert np.array_equal(bits32(out), bits32(np.broadcast_to(beta, (3, 64))))


# ------------------------------------------------------------------ RoPE
def test_golden_rope(O):
    out = O.rope(GOLD["rope_x"], GOLD["rope_cos"], GOLD["rope_sin"], "f32")
    assert np.array_equal(bits32(out), bits32(GOLD["rope_out"]))


@pytest.mark.parametrize("kind", ["f32", "bf16", "f16"])
def test_ref_rope(O, R, kind):
    x = _kind_cast(O, synth.randn(96, (2, 11, 4, 32)), kind)
    c, s = synth.randn(97, (11, 16)), synth.randn(98, (11, 16))
    assert np.array_equal(O.rope(x, c, s, kind).view(np.uint8), R.rope(x, c, s, kind).view(np.uint8))


def test_rope_closed_forms(O):
    """cos 1 / sin 0 is the identity; cos 0 / sin 1 maps (x0, x1) to
    (-x1, x0) exactly; a rotation keeps each pair's norm (float64)."""
    x = synth.randn(99, (1, 5, 2, 8))
    one, zero = np.ones((5, 4), np.float32), np.zeros((5, 4), np.float32)
    assert np.array_equal(bits32(O.rope(x, one, zero)), bits32(x))
    y = O.rope(x, zero, one)
    assert np.array_equal(y[..., 0::2], -x[..., 1::2]) and np.array_equal(y[..., 1::2], x[..., 0::2])
    ang = synth.randn(100, (5, 4))
    y = O.rope(x, np.cos(ang).astype(np.float32), np.sin(ang).astype(np.float32)).astype(np.float64)
    n0 = np.hypot(x[..., 0::2].astype(np.float64), x[..., 1::2])
    assert np.allclose(np.hypot(y[..., 0::2], y[..., 1::2]), n0, rtol=1e-6)


# ---- Conv2D (cpu_conv2d.c and its 16-bit twins) ----

CONV_KEYS = ("p1", "s2g2", "patch", "asym")


@pytest.mark.parametrize("key", CONV_KEYS)
def test_golden_conv2d(O, key):
    x, w, y = GOLD[f"conv_{key}_x"], GOLD[f"conv_{key}_w"], GOLD[f"conv_{key}_y"]
    st, ph, gr, pw = (int(v) for v in GOLD[f"conv_{key}_p"])
    got = O.conv2d(x, w, st, ph, pw if pw else None, gr, out_hw=y.shape[1:3], threads=3)
    assert np.array_equal(bits32(got), bits32(y))


@pytest.mark.parametrize("kind", ["bf16", "f16"])
def test_golden_conv2d_16bit(O, kind):
    x, w, y = (GOLD[f"conv_p1_{kind}_{t}"] for t in "xwy")
    assert np.array_equal(O.conv2d(x, w, 1, 1, kind=kind), y)


@pytest.mark.parametrize("shape", [((1, 9, 7, 8), (6, 3, 3, 8), 1, 1, 1),
                                   ((2, 10, 10, 6), (4, 3, 3, 3), 2, 1, 2),
                                   ((1, 28, 28, 3), (16, 14, 14, 3), 14, 0, 1),
                                   ((1, 5, 5, 4), (4, 1, 1, 1), 1, 0, 4),
                                   ((1, 8, 8, 64), (32, 3, 3, 64), 1, 1, 1)],
                         ids=["p1", "s2g2", "patch14", "depthwise", "c64"])
@pytest.mark.parametrize("kind", ["f32", "bf16", "f16"])
def test_ref_conv2d(O, R, shape, kind):
    xs, ws, st, ph, gr = shape
    x, w = synth.randn(101, xs), synth.randn(102, ws, 0.2)
    if kind != "f32":
        cv = O.f32_to_bf16 if kind == "bf16" else O.f32_to_fp16
        x, w = cv(x).reshape(xs), cv(w).reshape(ws)
    rc, y = R.conv2d(x, w, st, ph, None, gr, kind)
    assert rc == 0
    assert np.array_equal(O.conv2d(x, w, st, ph, groups=gr, kind=kind).view(np.uint8),
                          y.view(np.uint8))


def conv_f64(x, w, stride, ph, pw, groups):
    """Direct float64 convolution (definition of NHWC x OHWI)."""
    x, w = x.astype(np.float64), w.astype(np.float64)
    N, H, W, C = x.shape
    OC, KH, KW, cg = w.shape
    OH, OW = (H + 2 * ph - KH) // stride + 1, (W + 2 * pw - KW) // stride + 1
    xp = np.zeros((N, H + 2 * ph, W + 2 * pw, C))
    xp[:, ph:ph + H, pw:pw + W] = x
    og = OC // groups
    y = np.zeros((N, OH, OW, OC))
    for oh in range(OH):
        for ow in range(OW):
            patch = xp[:, oh * stride:oh * stride + KH, ow * stride:ow * stride + KW]
            for g in range(groups):
                pg = patch[..., g * cg:(g + 1) * cg].reshape(N, -1)
                wg = w[g * og:(g + 1) * og].reshape(og, -1)
                y[:, oh, ow, g * og:(g + 1) * og] = pg @ wg.T
    return y


def test_conv2d_closed_forms(O):
    """A centre-tap identity kernel with padding 1 returns x exactly; a
    1x1 conv is the matmul of the pixels; stride = kernel patchifies; all
    match a float64 direct convolution within f32 accumulation error."""
    x = synth.randn(103, (2, 6, 5, 4))
    eye = np.zeros((4, 3, 3, 4), np.float32)
    eye[:, 1, 1, :] = np.eye(4, dtype=np.float32)
    assert np.array_equal(bits32(O.conv2d(x, eye, 1, 1)), bits32(x))
    w1 = synth.randn(104, (7, 1, 1, 4))
    y = O.conv2d(x, w1).astype(np.float64)
    ref = x.reshape(-1, 4).astype(np.float64) @ w1.reshape(7, 4).T.astype(np.float64)
    assert np.allclose(y.reshape(-1, 7), ref, rtol=1e-5, atol=1e-6)
    for (xs, ws, st, ph, pw, gr) in [((1, 12, 12, 3), (5, 4, 4, 3), 4, 0, 0, 1),
                                     ((1, 7, 9, 6), (6, 3, 3, 2), 2, 1, 2, 3)]:
        xx, ww = synth.randn(105, xs), synth.randn(106, ws)
        got = O.conv2d(xx, ww, st, ph, pw, gr).astype(np.float64)
        assert np.allclose(got, conv_f64(xx, ww, st, ph, pw, gr), rtol=1e-5, atol=1e-5)


# ---- ConvTranspose2D and MaxPool2D (cpu_conv_transpose2d.c, cpu_maxpool2d.c) ----

@pytest.mark.parametrize("key", ["k2", "k3"])
def test_golden_conv_transpose2d(O, key):
    x, w, y = GOLD[f"convt_{key}_x"], GOLD[f"convt_{key}_w"], GOLD[f"convt_{key}_y"]
    st, pd = (int(v) for v in GOLD[f"convt_{key}_p"])
    assert np.array_equal(bits32(O.conv_transpose2d(x, w, st, pd, threads=3)), bits32(y))


@pytest.mark.parametrize("k,st", [(2, 2), (3, 2)])
def test_golden_maxpool2d(O, k, st):
    assert np.array_equal(bits32(O.maxpool2d(GOLD["maxpool_x"], k, st)),
                          bits32(GOLD[f"maxpool_{k}{st}_y"]))


@pytest.mark.parametrize("shape", [((1, 5, 6, 8), (4, 2, 2, 8), 2, 0),
                                   ((2, 4, 4, 3), (5, 3, 3, 3), 2, 1),
                                   ((1, 4, 5, 6), (3, 3, 3, 6), 1, 1)])
def test_ref_conv_transpose2d(O, R, shape):
    xs, ws, st, pd = shape
    x, w = synth.randn(110, xs), synth.randn(111, ws, 0.2)
    rc, y = R.conv_transpose2d(x, w, st, pd)
    assert rc == 0
    assert np.array_equal(bits32(O.conv_transpose2d(x, w, st, pd)), bits32(y))


def test_conv_transpose2d_closed_forms(O):
    """stride = kernel, no padding: each output pixel is one input pixel
    times one tap's [OC, C] slice (float64); an overlapping transposed
    conv equals the scatter-add definition (float64)."""
    x, w = synth.randn(112, (1, 3, 4, 5)), synth.randn(113, (6, 2, 2, 5))
    y = O.conv_transpose2d(x, w, 2, 0).astype(np.float64)
    ref = np.einsum("nhwc,okjc->nhkwjo", x.astype(np.float64), w.astype(np.float64))
    assert np.allclose(y, ref.reshape(1, 6, 8, 6), rtol=1e-5, atol=1e-6)
    x, w = synth.randn(114, (1, 3, 3, 2)), synth.randn(115, (2, 3, 3, 2))
    st, pd = 2, 1
    full = np.zeros((1, (3 - 1) * st + 3, (3 - 1) * st + 3, 2))
    for h in range(3):
        for ww in range(3):
            full[0, h * st:h * st + 3, ww * st:ww * st + 3] += np.einsum(
                "c,okjc->kjo", x[0, h, ww].astype(np.float64), w.astype(np.float64))
    ref = full[:, pd:full.shape[1] - pd, pd:full.shape[2] - pd]
    assert np.allclose(O.conv_transpose2d(x, w, st, pd), ref, rtol=1e-5, atol=1e-6)


def test_maxpool2d_closed_forms(O):
    x = synth.randn(116, (2, 8, 6, 3))
    ref = x.reshape(2, 4, 2, 3, 2, 3).max(axis=(2, 4))
    assert np.array_equal(O.maxpool2d(x, 2, 2), ref)
