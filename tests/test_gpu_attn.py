"""GPU parity of the fused attention kernels (SAM3_OP_SDPA) against the CPU
oracle, through the C ABI.

The reference's SDPA (cpu_kernel_sdpa, src/backend/cpu/kernels/
cpu_sdpa.c:216-288) is f32 only; its golden vectors (written by the
reference's own kernel, tests/golden/make_golden.py) and the oracle
restatement (pinned to it bit for bit in tests/test_oracle.py) are the
checkers here:
  - f32 on the MFMA kernel (three bf16 products per step) and on the any-D
    kernel: within the f32 bound of 1e-3 (assert_f32_close);
  - bf16 / f16 inputs: the oracle on the inputs widened to f32, its output
    rounded once to the input type, within 2e-2 (bf16) or 5e-3 (f16)
    absolute, the bounds of the reference's bf16/f16 matmul tests;
  - closed forms that fix the result exactly: a mask that leaves one key
    returns that key's V row bit for bit (16-bit inputs), a fully masked
    row returns zeros, Sk = 0 returns zeros.
"""
import ctypes as C
from pathlib import Path

import numpy as np
import pytest

from gpu_util import assert_bf16_close, assert_f16_close, assert_f32_close, oracle, require_gpu
from sam3_amd import abi, hip, synth

pytestmark = pytest.mark.gpu

GOLD = np.load(Path(__file__).parent / "golden" / "matmul_golden.npz")
MFMA, GENERIC, SMALL = 1, 3, 4


@pytest.fixture(scope="module", autouse=True)
def gpu():
    require_gpu()


def bits32(x):
    return np.ascontiguousarray(x, np.float32).view(np.uint32)


def to_dtype(x, dt):
    """Host array of dtype dt (bf16 as uint16 bits) and its exact f32 value."""
    if dt == abi.F32:
        x = np.ascontiguousarray(x, np.float32)
        return x, x
    if dt == abi.F16:
        h = np.ascontiguousarray(x, np.float32).astype(np.float16)
        return h, h.astype(np.float32)
    b = oracle().f32_to_bf16(x).reshape(x.shape)
    return b, (b.astype(np.uint32) << 16).view(np.float32)


def check(dt, got, ref_f32, what):
    if dt == abi.F32:
        assert_f32_close(got, ref_f32, what=what)
    elif dt == abi.F16:
        assert_f16_close(got.view(np.uint16), ref_f32.astype(np.float16).view(np.uint16), what=what)
    else:
        ref = oracle().f32_to_bf16(ref_f32).reshape(ref_f32.shape)
        assert_bf16_close(got, ref, what=what)


def inputs(seed, BH, Sq, Sk, D, qscale=1.0):
    q = synth.randn(seed, (BH, Sq, D)) * np.float32(qscale)
    k = synth.randn(seed + 1, (BH, Sk, D))
    v = synth.randn(seed + 2, (BH, Sk, D))
    return q, k, v


def run(dt, q, k, v, mask=None, path=0):
    """hip.sdpa on dtype dt; returns (device output, oracle f32 output)."""
    qd, qf = to_dtype(q, dt)
    kd, kf = to_dtype(k, dt)
    vd, vf = to_dtype(v, dt)
    got = hip.sdpa(qd, kd, vd, mask, dtype=dt, path=path)
    return got, oracle().sdpa(qf, kf, vf, mask, 8)


DTS = [abi.F32, abi.BF16, abi.F16]
DT_ID = {abi.F32: "f32", abi.BF16: "bf16", abi.F16: "f16"}


# ----------------------------------------------------------- golden vectors
@pytest.mark.parametrize("path", [0, MFMA, GENERIC, SMALL])
def test_sdpa_golden(path):
    """The reference's own outputs (cpu_kernel_sdpa, 4-D, ragged Sk = 70)."""
    q, k, v, m = GOLD["sdpa_q"], GOLD["sdpa_k"], GOLD["sdpa_v"], GOLD["sdpa_mask"]
    got = hip.sdpa(q, k, v, None, dtype=abi.F32, path=path)
    assert_f32_close(got, GOLD["sdpa_out"], what=f"golden sdpa path {path}")
    got = hip.sdpa(q, k, v, m, dtype=abi.F32, path=path)
    assert_f32_close(got, GOLD["sdpa_out_mask"], what=f"golden sdpa+mask path {path}")


def test_sdpa_generic_f32_close_to_reference_order():
    """The any-D kernel keeps f32 throughout: far inside the bound."""
    q, k, v, m = GOLD["sdpa_q"], GOLD["sdpa_k"], GOLD["sdpa_v"], GOLD["sdpa_mask"]
    got = hip.sdpa(q, k, v, m, dtype=abi.F32, path=GENERIC)
    ref = GOLD["sdpa_out_mask"].astype(np.float64)
    assert np.max(np.abs(got - ref)) <= 2e-5 * np.max(np.abs(ref))


# ------------------------------------------------------- shapes and dtypes
SHAPES = [(8, 576, 576), (3, 37, 70), (2, 1, 1), (2, 129, 65), (1, 200, 1000),
          (1, 128, 63), (2, 256, 5184)]


@pytest.mark.parametrize("dt", DTS, ids=lambda d: DT_ID[d])
@pytest.mark.parametrize("BH,Sq,Sk", SHAPES)
def test_sdpa_mfma_shapes(dt, BH, Sq, Sk):
    q, k, v = inputs(900 + Sq + Sk, BH, Sq, Sk, 64)
    got, ref = run(dt, q, k, v, path=MFMA)
    check(dt, got, ref, f"sdpa {DT_ID[dt]} {BH}x{Sq}x{Sk}")


@pytest.mark.parametrize("dt", DTS, ids=lambda d: DT_ID[d])
@pytest.mark.parametrize("Sk", [70, 576, 1001])
def test_sdpa_mask(dt, Sk):
    """Additive f32 mask shared by the heads; Sk = 70 and 1001 take the
    scalar mask loads (rows not 16-byte aligned)."""
    BH, Sq = 3, 150
    q, k, v = inputs(950 + Sk, BH, Sq, Sk, 64)
    mask = synth.randn(960 + Sk, (Sq, Sk), 2.0)
    mask[::7, ::3] = -np.inf
    got, ref = run(dt, q, k, v, mask, path=MFMA)
    check(dt, got, ref, f"sdpa mask {DT_ID[dt]} Sk={Sk}")


@pytest.mark.parametrize("dt", [abi.BF16, abi.F16], ids=lambda d: DT_ID[d])
@pytest.mark.parametrize("BH,Sq,Sk,masked", [(3, 150, 70, True), (2, 129, 65, False),
                                             (8, 576, 576, False), (1, 200, 1000, True),
                                             (2, 256, 5184, False), (2, 1, 1, False)])
def test_sdpa_v_tiles_by_dma_same_bits(env, dt, BH, Sq, Sk, masked):
    """16-bit V tiles by direct-to-LDS loads read with ds_read_b64_tr_b16
    (the default) give the same MFMA operands as V staged through
    registers into a transposed tile (SAM3_HIP_ATTN_VDMA=0): the same bits,
    ragged key tails and masks included."""
    q, k, v = inputs(980 + Sq + Sk, BH, Sq, Sk, 64)
    mask = None
    if masked:
        mask = synth.randn(990 + Sk, (Sq, Sk), 2.0)
        mask[::5, ::3] = -np.inf
    qd, _ = to_dtype(q, dt)
    kd, _ = to_dtype(k, dt)
    vd, _ = to_dtype(v, dt)
    env.unset("SAM3_HIP_ATTN_VDMA")
    dma = hip.sdpa(qd, kd, vd, mask, dtype=dt, path=MFMA)
    env.set("SAM3_HIP_ATTN_VDMA", 0)
    staged = hip.sdpa(qd, kd, vd, mask, dtype=dt, path=MFMA)
    assert np.array_equal(np.asarray(dma).view(np.uint16), np.asarray(staged).view(np.uint16))


@pytest.mark.parametrize("dt", DTS, ids=lambda d: DT_ID[d])
def test_sdpa_sharp_softmax(dt):
    """Scores with a spread of ~100 (q scaled by 12): the running max and
    the rescale of earlier tiles carry the result."""
    q, k, v = inputs(970, 4, 256, 700, 64, qscale=12.0)
    got, ref = run(dt, q, k, v, path=MFMA)
    check(dt, got, ref, f"sdpa sharp {DT_ID[dt]}")


@pytest.mark.parametrize("dt", DTS, ids=lambda d: DT_ID[d])
@pytest.mark.parametrize("D", [16, 32, 48, 80, 128, 256, 320])
def test_sdpa_any_head_dim(dt, D):
    """The any-D kernel, for the decoder's head sizes and beyond."""
    q, k, v = inputs(980 + D, 3, 45, 133, D)
    mask = synth.randn(990 + D, (45, 133))
    got, ref = run(dt, q, k, v, mask)
    check(dt, got, ref, f"sdpa D={D} {DT_ID[dt]}")


@pytest.mark.parametrize("dt", DTS, ids=lambda d: DT_ID[d])
def test_sdpa_paths_agree(dt):
    q, k, v = inputs(995, 2, 300, 333, 64)
    a, ref = run(dt, q, k, v, path=MFMA)
    b, _ = run(dt, q, k, v, path=GENERIC)
    check(dt, a, ref, "mfma")
    check(dt, b, ref, "generic")


# --------------------------------------------------------- closed forms
@pytest.mark.parametrize("dt", [abi.BF16, abi.F16], ids=lambda d: DT_ID[d])
@pytest.mark.parametrize("path", [MFMA, GENERIC])
def test_sdpa_single_key_mask_selects_v_row(dt, path):
    """A mask of -inf on every key but one gives weight exactly 1 to that
    key: the output is its V row, bit for bit."""
    BH, Sq, Sk, D = 2, 70, 200, 64
    q, k, v = inputs(1000, BH, Sq, Sk, D)
    pick = (np.arange(Sq) * 37 + 5) % Sk
    mask = np.full((Sq, Sk), -np.inf, np.float32)
    mask[np.arange(Sq), pick] = 0.0
    qd, _ = to_dtype(q, dt)
    kd, _ = to_dtype(k, dt)
    vd, _ = to_dtype(v, dt)
    got = hip.sdpa(qd, kd, vd, mask, dtype=dt, path=path)
    assert np.array_equal(got, vd[:, pick, :])


@pytest.mark.parametrize("dt", DTS, ids=lambda d: DT_ID[d])
@pytest.mark.parametrize("path", [MFMA, GENERIC])
def test_sdpa_fully_masked_rows_are_zero(dt, path):
    """A row whose scores are all -inf has row_sum 0 and stays zero
    (cpu_sdpa.c:143-158); the other rows are unaffected."""
    BH, Sq, Sk, D = 2, 40, 90, 64
    q, k, v = inputs(1010, BH, Sq, Sk, D)
    mask = np.zeros((Sq, Sk), np.float32)
    mask[[0, 13, 39]] = -np.inf
    got, ref = run(dt, q, k, v, mask, path=path)
    f = got if dt == abi.F32 else (got.astype(np.float32) if dt == abi.F16 else
                                   (got.astype(np.uint32) << 16).view(np.float32))
    assert np.all(f[:, [0, 13, 39]] == 0)
    check(dt, got, ref, "partially masked")


def test_sdpa_no_keys_and_no_queries():
    q = synth.randn(1020, (2, 5, 64))
    empty = np.zeros((2, 0, 64), np.float32)
    assert not hip.sdpa(q, empty, empty, dtype=abi.F32).any()
    assert hip.sdpa(empty, q, q, dtype=abi.F32).shape == (2, 0, 64)


def test_sdpa_kernel_choice_errors():
    q = synth.randn(1030, (1, 4, 32))
    with pytest.raises(hip.HipError):
        hip.sdpa(q, q, q, dtype=abi.F32, path=MFMA)   # D = 32: no MFMA kernel
    big = np.zeros((1, 2, 513), np.float32)
    with pytest.raises(hip.HipError):
        hip.sdpa(big, big, big, dtype=abi.F32)


# ------------------------------------------------------ few-keys kernel
SMALL_SAME = [(2, 1, 1), (16, 1, 1), (16, 8, 8), (16, 32, 32), (3, 37, 64), (1, 100, 17)]


@pytest.mark.parametrize("masked", [False, True], ids=["nomask", "mask"])
@pytest.mark.parametrize("BH,Sq,Sk", SMALL_SAME)
def test_sdpa_small_same_bits_as_generic(BH, Sq, Sk, masked):
    """Up to 64 keys the few-keys kernel takes the any-D kernel's steps in
    the same order (one 64-key tile there), so the outputs agree bit for
    bit; both are checked against the oracle."""
    q, k, v = inputs(1100 + Sq + Sk, BH, Sq, Sk, 64)
    mask = None
    if masked:
        mask = synth.randn(1101, (Sq, Sk))
        mask[np.triu_indices(Sq, 1, Sk)] = np.float32(-1e9)
    a = hip.sdpa(q, k, v, mask, dtype=abi.F32, path=SMALL)
    b = hip.sdpa(q, k, v, mask, dtype=abi.F32, path=GENERIC)
    assert np.array_equal(bits32(a), bits32(b))
    assert_f32_close(a, oracle().sdpa(q, k, v, mask, 8), what=f"small {BH}x{Sq}x{Sk}")


@pytest.mark.parametrize("Sq,Sk,want", [(1, 1, GENERIC), (8, 8, GENERIC), (32, 32, MFMA),
                                        (77, 77, SMALL), (3, 100, SMALL), (200, 300, MFMA)])
def test_sdpa_best_kernel_by_size(Sq, Sk, want):
    """f32, D = 64: path 0 takes the one-wave-per-row kernel up to 64
    scores per head, the few-keys kernel from 65 keys to 128, the MFMA
    kernel otherwise; its bits are that kernel's."""
    q, k, v = inputs(1140 + Sq, 16, Sq, Sk, 64)
    best = hip.sdpa(q, k, v, None, dtype=abi.F32)
    forced = hip.sdpa(q, k, v, None, dtype=abi.F32, path=want)
    assert np.array_equal(bits32(best), bits32(forced))


@pytest.mark.parametrize("masked", [False, True], ids=["nomask", "mask"])
@pytest.mark.parametrize("BH,Sq,Sk", [(16, 77, 77), (2, 129, 65), (1, 200, 128), (5, 3, 100)])
def test_sdpa_small_many_keys(BH, Sq, Sk, masked):
    """65-128 keys: the softmax over all keys at once (the any-D kernel
    rescales per 64-key tile), within the f32 bound of the oracle."""
    q, k, v = inputs(1110 + Sq + Sk, BH, Sq, Sk, 64, qscale=2.0)
    mask = None
    if masked:
        c = np.arange(Sk)
        mask = np.where(c[None, :] > np.arange(Sq)[:, None] + (Sk - Sq), np.float32(-1e9),
                        np.float32(0.0)).astype(np.float32)
    got = hip.sdpa(q, k, v, mask, dtype=abi.F32, path=SMALL)
    assert_f32_close(got, oracle().sdpa(q, k, v, mask, 8), what=f"small {BH}x{Sq}x{Sk}")


def test_sdpa_small_single_key_and_masked_rows():
    """One unmasked key: weight exactly 1, the output is that V row bit for
    bit; rows with every key masked are zero."""
    BH, Sq, Sk, D = 3, 50, 100, 64
    q, k, v = inputs(1120, BH, Sq, Sk, D)
    pick = (np.arange(Sq) * 37 + 5) % Sk
    mask = np.full((Sq, Sk), -np.inf, np.float32)
    mask[np.arange(Sq), pick] = 0.0
    mask[[7, 49]] = -np.inf
    got = hip.sdpa(q, k, v, mask, dtype=abi.F32, path=SMALL)
    keep = np.setdiff1d(np.arange(Sq), [7, 49])
    assert np.array_equal(bits32(got[:, keep]), bits32(v[:, pick[keep], :]))
    assert np.all(got[:, [7, 49]] == 0)


def test_sdpa_small_kernel_limits():
    q = synth.randn(1130, (1, 4, 64))
    k = synth.randn(1131, (1, 129, 64))
    with pytest.raises(hip.HipError):
        hip.sdpa(q, k, k, dtype=abi.F32, path=SMALL)   # 129 keys
    q32 = synth.randn(1132, (1, 4, 32))
    with pytest.raises(hip.HipError):
        hip.sdpa(q32, q32, q32, dtype=abi.F32, path=SMALL)   # D = 32
    qb, _ = to_dtype(q, abi.BF16)
    with pytest.raises(hip.HipError):
        hip.sdpa(qb, qb, qb, dtype=abi.BF16, path=SMALL)   # f32 only


# ------------------------------------------------- node kernel and backend
def _dev_tensor(keep, dt, dims, arr):
    buf = hip.DeviceBuffer.of(arr)
    keep.append(buf)
    t = abi.make_tensor(dt, list(dims), buf.ptr, arr.nbytes)
    keep.append(t)
    return t


@pytest.mark.parametrize("dt", DTS, ids=lambda d: DT_ID[d])
def test_sdpa_node_kernel_4d(dt):
    """sam3_hip_kernel_sdpa and sam3_hip_dispatch_node on a hand-built
    4-D node [B, H, seq, hd] with a mask, as gh_sdpa builds it
    (graph_helpers.c:688-717)."""
    B, H, Sq, Sk, D = 2, 3, 77, 99, 64
    q, k, v = inputs(1040, B * H, Sq, Sk, D)
    mask = synth.randn(1043, (Sq, Sk))
    qd, qf = to_dtype(q, dt)
    kd, kf = to_dtype(k, dt)
    vd, vf = to_dtype(v, dt)
    ref = oracle().sdpa(qf, kf, vf, mask, 8)
    keep = []
    tq = _dev_tensor(keep, dt, (B, H, Sq, D), qd)
    tk = _dev_tensor(keep, dt, (B, H, Sk, D), kd)
    tv = _dev_tensor(keep, dt, (B, H, Sk, D), vd)
    tm = _dev_tensor(keep, abi.F32, (Sq, Sk), mask)
    to = _dev_tensor(keep, dt, (B, H, Sq, D), np.zeros_like(qd))
    lib = hip.load()
    for fn in (lib.sam3_hip_kernel_sdpa, lib.sam3_hip_dispatch_node):
        node = abi.make_node(abi.OP_SDPA, [tq, tk, tv, tm], to, (D, 0, 0, 0))
        hip.check(fn(C.byref(node), None), "sdpa node")
        hip.synchronize()
        got = keep[-2].download(qd.dtype, qd.shape)
        check(dt, got, ref, f"node {DT_ID[dt]}")
    bad = abi.make_node(abi.OP_SDPA, [tq, tk, tv, tm], tq, (D, 0, 0, 0))
    bad.inputs[3].contents.dtype = abi.BF16
    assert lib.sam3_hip_kernel_sdpa(C.byref(bad), None) == abi.EDTYPE
    for b in keep:
        if isinstance(b, hip.DeviceBuffer):
            b.free()


def test_sdpa_graph_eval_2d():
    """graph_eval runs an f32 SDPA node on the GPU (2-D [seq, hd] form,
    as the mask decoder's per-head calls use it, head_dim 32)."""
    from test_gpu_backend import GraphBuilder, out_array
    be = hip.Backend(0)
    try:
        Sq, Sk, D = 9, 4100, 32
        q, k, v = inputs(1050, 1, Sq, Sk, D)
        G = GraphBuilder()
        tq, _ = G.tensor(abi.F32, (Sq, D), q[0], ephemeral=1)
        tk, _ = G.tensor(abi.F32, (Sk, D), k[0], ephemeral=1)
        tv, _ = G.tensor(abi.F32, (Sk, D), v[0], ephemeral=1)
        to, _ = G.tensor(abi.F32, (Sq, D))
        G.node(abi.OP_SDPA, [tq, tk, tv], to, (D, 0, 0, 0))
        assert be.graph_eval(G.g) == abi.OK
        st = be.stats()
        assert st.gpu_nodes == 1 and st.host_nodes == 0
        got = out_array(to, np.float32, (1, Sq, D))
        assert_f32_close(got, oracle().sdpa(q, k, v, None, 8), what="graph sdpa")
    finally:
        be.close()
