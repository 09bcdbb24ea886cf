"""GPU parity of CONV2D (NHWC x OHWI, cpu_conv2d.c and its 16-bit twins)
and BIAS_ADD against the oracle (bit-exact with the reference's kernels,
tests/test_oracle.py):

  - the direct kernel: f32 bit for bit (the reference's order), 16-bit
    outputs bit for bit (f32 accumulation, one rounding);
  - the implicit GEMM and the column-matrix GEMM: f32 through bf16 hi/lo
    planes within the f32 bound (1e-3; measured ~1e-5), bf16/f16 within
    their output bounds;
  - padding, strides, ragged M (rows past the last tile), OC not a
    multiple of 8, several 64-channel k-steps per tap;
  - graph_eval folds CONV2D -> BIAS_ADD -> GELU into one launch;
  - the ViT patch embedding (1008x1008x3, 14x14 stride 14 -> 72x72x1024)
    at full size, checked on its first patch rows.
"""
import ctypes as C

import numpy as np
import pytest

from gpu_util import assert_bf16_close, assert_f16_close, assert_f32_close, oracle, require_gpu
from sam3_amd import abi, hip, synth

pytestmark = pytest.mark.gpu

DT = {"f32": abi.F32, "bf16": abi.BF16, "f16": abi.F16}
IMPLICIT, IM2COL, DIRECT = 1, 2, 3


@pytest.fixture(scope="module", autouse=True)
def gpu():
    require_gpu()


def cast(x, kind):
    if kind == "f32":
        return np.ascontiguousarray(x, np.float32)
    O = oracle()
    return (O.f32_to_bf16 if kind == "bf16" else O.f32_to_fp16)(x).reshape(x.shape)


def gpu_conv(x, w, stride, ph, pw, groups, kind, path, out_hw=None):
    N, H, W, Cin = x.shape
    OC, KH, KW, _ = w.shape
    p_w = ph if pw is None else pw
    OH, OW = out_hw or ((H + 2 * ph - KH) // stride + 1, (W + 2 * p_w - KW) // stride + 1)
    npt = np.float32 if kind == "f32" else np.uint16
    bx, bw = hip.DeviceBuffer.of(x), hip.DeviceBuffer.of(w)
    by = hip.DeviceBuffer(N * OH * OW * OC * np.dtype(npt).itemsize)
    try:
        tx = abi.make_tensor(DT[kind], [N, H, W, Cin], bx.ptr, x.nbytes)
        tw = abi.make_tensor(DT[kind], list(w.shape), bw.ptr, w.nbytes)
        ty = abi.make_tensor(DT[kind], [N, OH, OW, OC], by.ptr, by.nbytes)
        node = abi.make_node(abi.OP_CONV2D, [tx, tw], ty, (stride, ph, groups, pw or 0))
        lib = hip.load()
        if path:
            hip.check(lib.sam3_hip_conv2d_on_path(path, C.byref(node), None), f"conv path {path}")
        else:
            hip.check(lib.sam3_hip_kernel_conv2d(C.byref(node), None), "conv")
        hip.synchronize()
        return by.download(npt, (N, OH, OW, OC))
    finally:
        for b in (bx, bw, by):
            b.free()


def check(got, ref, kind, exact, what):
    if exact:
        assert np.array_equal(got.view(np.uint8), ref.view(np.uint8)), what
    elif kind == "f32":
        assert_f32_close(got, ref, what=what)
    elif kind == "bf16":
        assert_bf16_close(got, ref, what=what)
    else:
        assert_f16_close(got, ref, what=what)


CASES = {
    # name: (x shape, w shape, stride, pad_h, pad_w, groups, paths)
    "c64_3x3": ((2, 12, 10, 64), (48, 3, 3, 64), 1, 1, None, 1, (IMPLICIT, IM2COL, DIRECT)),
    "c128_1x1": ((1, 16, 16, 128), (64, 1, 1, 128), 1, 0, None, 1, (IMPLICIT, IM2COL)),
    "c64_s2_tail": ((1, 15, 13, 64), (80, 3, 3, 64), 2, 1, None, 1, (IMPLICIT, IM2COL, DIRECT)),
    "c192_oc20": ((1, 9, 9, 192), (20, 3, 3, 192), 1, 1, None, 1, (IMPLICIT, IM2COL)),
    "c64_asym": ((1, 11, 9, 64), (32, 3, 3, 64), 1, 2, 1, 1, (IMPLICIT, IM2COL, DIRECT)),
    "patch14": ((1, 56, 56, 3), (64, 14, 14, 3), 14, 0, None, 1, (IM2COL, DIRECT)),
    "c32_5x5": ((1, 12, 12, 32), (24, 5, 5, 32), 1, 2, None, 1, (IM2COL, DIRECT)),
    "groups2": ((2, 10, 10, 6), (4, 3, 3, 3), 2, 1, None, 2, (DIRECT,)),
    "depthwise": ((1, 9, 9, 16), (16, 3, 3, 1), 1, 1, None, 16, (DIRECT,)),
}


@pytest.mark.parametrize("kind", ["f32", "bf16", "f16"])
@pytest.mark.parametrize("name", sorted(CASES))
def test_conv2d_paths_vs_oracle(name, kind):
    xs, ws, st, ph, pw, gr, paths = CASES[name]
    x = cast(synth.randn(300, xs), kind)
    w = cast(synth.randn(301, ws, 0.1), kind)
    ref = oracle().conv2d(x, w, st, ph, pw, gr, kind=kind)
    for path in paths:
        got = gpu_conv(x, w, st, ph, pw, gr, kind, path)
        check(got, ref, kind, path == DIRECT, f"{name} {kind} path {path}")
    # the default choice
    got = gpu_conv(x, w, st, ph, pw, gr, kind, 0)
    check(got, ref, kind, False, f"{name} {kind} default")


def test_conv2d_path_choice_and_errors():
    lib = hip.load()
    x = np.zeros((1, 16, 16, 64), np.float32)
    bx = hip.DeviceBuffer.of(x)
    try:
        def node(ws, out, params=(1, 1, 1, 0), dt=abi.F32, wdt=None):
            tx = abi.make_tensor(dt, [1, 16, 16, 64], bx.ptr, x.nbytes)
            tw = abi.make_tensor(wdt or dt, list(ws), bx.ptr, 4)
            ty = abi.make_tensor(dt, list(out), bx.ptr, 4)
            return abi.make_node(abi.OP_CONV2D, [tx, tw], ty, params), (tx, tw, ty)
        n, keep = node((64, 3, 3, 64), (1, 16, 16, 64))
        assert lib.sam3_hip_conv2d_path(C.byref(n)) == IMPLICIT
        n, keep = node((8, 3, 3, 64), (1, 16, 16, 8))
        assert lib.sam3_hip_conv2d_path(C.byref(n)) == DIRECT        # under 2^22 MACs
        n, keep = node((64, 3, 3, 32), (1, 16, 16, 64))               # 32 * 1 != 64
        assert lib.sam3_hip_kernel_conv2d(C.byref(n), None) == abi.EINVAL
        n, keep = node((64, 3, 3, 64), (1, 16, 16, 32))               # output channels
        assert lib.sam3_hip_kernel_conv2d(C.byref(n), None) == abi.EINVAL
        n, keep = node((64, 3, 3, 64), (1, 16, 16, 64), wdt=abi.BF16)  # mixed dtypes
        assert lib.sam3_hip_kernel_conv2d(C.byref(n), None) == abi.EDTYPE
        n, keep = node((64, 3, 3, 32), (1, 16, 16, 64), params=(1, 1, 2, 0))  # groups 2
        assert lib.sam3_hip_conv2d_on_path(IMPLICIT, C.byref(n), None) == abi.EINVAL
    finally:
        bx.free()


@pytest.mark.parametrize("kind", ["f32", "bf16"])
@pytest.mark.parametrize("gelu", [False, True])
def test_graph_conv_bias_gelu_fused(kind, gelu):
    """CONV2D -> BIAS_ADD (-> GELU) as gh_conv2d + the neck build them
    (graph_helpers.c:1341-1396, necks.c:345-365): one GEMM launch with the
    bias and GELU in its epilogue."""
    from sam3_amd import graph
    O = oracle()
    xs, ws = (1, 18, 18, 64), (96, 3, 3, 64)
    x = cast(synth.randn(310, xs), kind)
    w = cast(synth.randn(311, ws, 0.1), kind)
    b = cast(synth.randn(312, (96,), 0.5), kind)
    G = graph.Graph()
    tx, tw, tb = G.tensor(DT[kind], xs, x), G.tensor(DT[kind], ws, w), G.tensor(DT[kind], (96,), b)
    ty = G.node(abi.OP_CONV2D, [tx, tw], G.tensor(DT[kind], (1, 18, 18, 96)), (1, 1, 1, 0))
    ty = G.node(abi.OP_BIAS_ADD, [ty, tb], G.tensor(DT[kind], (1, 18, 18, 96)))
    if gelu:
        ty = G.node(abi.OP_GELU, [ty], G.tensor(DT[kind], (1, 18, 18, 96)))
    be = hip.Backend(0)
    try:
        assert be.graph_eval(G.g) == abi.OK
        st = be.stats()
    finally:
        be.close()
    assert st.host_nodes == 0 and st.gpu_nodes == 1 and st.fused_nodes == (2 if gelu else 1)
    npt = np.float32 if kind == "f32" else np.uint16
    got = np.ctypeslib.as_array(C.cast(ty.data, C.POINTER(C.c_float if kind == "f32" else C.c_uint16)),
                                shape=(18 * 18 * 96,)).astype(npt).copy()
    conv = O.conv2d(x, w, 1, 1, kind=kind).reshape(-1, 96)
    ref = O.bias_add(conv, b, kind)
    if gelu:
        ref = O.gelu(ref, kind)
    check(got.reshape(-1, 96), ref.reshape(-1, 96), kind, False, f"conv+bias gelu={gelu}")


def test_patch_embedding_full_size():
    """sam3_vit's patch embedding (image_encoder.c:560-600): image
    [1, 1008, 1008, 3] f32, weight [1024, 14, 14, 3], stride 14, no pad ->
    [1, 72, 72, 1024]. Patches do not overlap, so the first 3 patch rows
    of the output are the conv of the image's first 42 pixel rows, which
    the oracle computes."""
    x = synth.randn(320, (1, 1008, 1008, 3))
    w = synth.randn(321, (1024, 14, 14, 3), 0.02)
    got = gpu_conv(x, w, 14, 0, None, 1, "f32", 0)
    assert got.shape == (1, 72, 72, 1024)
    ref = oracle().conv2d(np.ascontiguousarray(x[:, :42]), w, 14, 0)
    assert_f32_close(got[:, :3], ref, what="patch embed rows 0-2")
    assert np.isfinite(got).all()


def test_neck_conv3x3_full_size():
    """The neck's 3x3 conv at the 4x scale (necks.c:345-365): [1, 288,
    288, 256] -> 256 channels, pad 1, f32 on the implicit GEMM; output rows
    0-4 need input rows 0-5, which a 7-row crop of the input holds."""
    x = synth.randn(330, (1, 288, 288, 256))
    w = synth.randn(331, (256, 3, 3, 256), 0.02)
    got = gpu_conv(x, w, 1, 1, None, 1, "f32", IMPLICIT)
    ref = oracle().conv2d(np.ascontiguousarray(x[:, :7]), w, 1, 1)
    assert_f32_close(got[:, :5], ref[:, :5], what="neck 3x3 rows 0-4")


# ---------------------------------------------- ConvTranspose2D and MaxPool2D
CONVT_GEMM, CONVT_DIRECT = 1, 3


def gpu_node(op, ins, out_shape, params):
    """Run one node kernel on device copies of f32 arrays."""
    bufs = [hip.DeviceBuffer.of(np.ascontiguousarray(a, np.float32)) for a in ins]
    by = hip.DeviceBuffer(int(np.prod(out_shape)) * 4)
    try:
        ts = [abi.make_tensor(abi.F32, list(a.shape), b.ptr, a.nbytes) for a, b in zip(ins, bufs)]
        ty = abi.make_tensor(abi.F32, list(out_shape), by.ptr, by.nbytes)
        node = abi.make_node(op, ts, ty, params)
        return (node, ts, ty), bufs, by
    except Exception:
        for b in bufs + [by]:
            b.free()
        raise


@pytest.mark.parametrize("shape", [((1, 12, 10, 64), (32, 2, 2, 64), 2, 0, (CONVT_GEMM, CONVT_DIRECT)),
                                   ((2, 9, 7, 24), (16, 2, 2, 24), 2, 0, (CONVT_GEMM, CONVT_DIRECT)),
                                   ((1, 5, 6, 8), (4, 3, 3, 8), 2, 1, (CONVT_DIRECT,)),
                                   ((1, 4, 5, 6), (3, 3, 3, 6), 1, 1, (CONVT_DIRECT,))],
                         ids=["k2_c64", "k2_ragged", "k3_s2_p1", "k3_s1"])
def test_conv_transpose2d_vs_oracle(shape):
    xs, ws, st, pd, paths = shape
    x, w = synth.randn(400, xs), synth.randn(401, ws, 0.1)
    ref = oracle().conv_transpose2d(x, w, st, pd)
    lib = hip.load()
    for path in paths:
        (node, ts, ty), bufs, by = gpu_node(abi.OP_CONV_TRANSPOSE2D, [x, w], ref.shape, (st, pd, 0, 0))
        try:
            hip.check(lib.sam3_hip_conv_transpose2d_on_path(path, C.byref(node), None), "convT")
            hip.synchronize()
            got = by.download(np.float32, ref.shape)
        finally:
            for b in bufs + [by]:
                b.free()
        if path == CONVT_DIRECT:
            assert np.array_equal(got.view(np.uint32), ref.view(np.uint32)), "direct"
        else:
            assert_f32_close(got, ref, what="convT gemm")


def test_maxpool2d_bit_exact():
    x = synth.randn(410, (2, 17, 13, 40))
    x[0, 0, 0, :3] = np.nan
    x[1, 5, 6, 7] = np.nan
    lib = hip.load()
    for k, st in ((2, 2), (3, 2), (2, 1)):
        ref = oracle().maxpool2d(x, k, st)
        (node, ts, ty), bufs, by = gpu_node(abi.OP_MAXPOOL2D, [x], ref.shape, (k, st, 0, 0))
        try:
            hip.check(lib.sam3_hip_kernel_maxpool2d(C.byref(node), None), "maxpool")
            hip.synchronize()
            got = by.download(np.float32, ref.shape)
        finally:
            for b in bufs + [by]:
                b.free()
        assert np.array_equal(got.view(np.uint32), ref.view(np.uint32)), (k, st)


def test_neck_stage_4x_in_graph():
    """The neck's 4x scale (necks.c:330-365): ConvTranspose2D 2x2 s2
    (+bias) -> GELU -> ConvTranspose2D 2x2 s2 (+bias) -> Conv2D 1x1
    (+bias) -> Conv2D 3x3 pad 1 (+bias), on a 12x12x128 map (scaled-down
    channels), all on the GPU with the bias and GELU folded; against the
    oracle's kernels in f32."""
    from sam3_amd import graph
    O = oracle()
    x = synth.randn(420, (1, 12, 12, 128))
    w1, b1 = synth.randn(421, (64, 2, 2, 128), 0.05), synth.randn(422, (64,), 0.1)
    w2, b2 = synth.randn(423, (32, 2, 2, 64), 0.05), synth.randn(424, (32,), 0.1)
    w3, b3 = synth.randn(425, (64, 1, 1, 32), 0.1), synth.randn(426, (64,), 0.1)
    w4, b4 = synth.randn(427, (64, 3, 3, 64), 0.05), synth.randn(428, (64,), 0.1)
    G = graph.Graph()
    F = abi.F32
    t = G.tensor(F, x.shape, x)
    t = G.node(abi.OP_CONV_TRANSPOSE2D, [t, G.tensor(F, w1.shape, w1)], G.tensor(F, (1, 24, 24, 64)), (2, 0, 0, 0))
    t = G.node(abi.OP_BIAS_ADD, [t, G.tensor(F, (64,), b1)], G.tensor(F, (1, 24, 24, 64)))
    t = G.node(abi.OP_GELU, [t], G.tensor(F, (1, 24, 24, 64)))
    t = G.node(abi.OP_CONV_TRANSPOSE2D, [t, G.tensor(F, w2.shape, w2)], G.tensor(F, (1, 48, 48, 32)), (2, 0, 0, 0))
    t = G.node(abi.OP_BIAS_ADD, [t, G.tensor(F, (32,), b2)], G.tensor(F, (1, 48, 48, 32)))
    t = G.node(abi.OP_CONV2D, [t, G.tensor(F, w3.shape, w3)], G.tensor(F, (1, 48, 48, 64)), (1, 0, 1, 0))
    t = G.node(abi.OP_BIAS_ADD, [t, G.tensor(F, (64,), b3)], G.tensor(F, (1, 48, 48, 64)))
    t = G.node(abi.OP_CONV2D, [t, G.tensor(F, w4.shape, w4)], G.tensor(F, (1, 48, 48, 64)), (1, 1, 1, 0))
    t = G.node(abi.OP_BIAS_ADD, [t, G.tensor(F, (64,), b4)], G.tensor(F, (1, 48, 48, 64)))
    be = hip.Backend(0)
    try:
        assert be.graph_eval(G.g) == abi.OK
        st = be.stats()
    finally:
        be.close()
    assert st.host_nodes == 0 and st.downloads == 1
    got = np.ctypeslib.as_array(C.cast(t.data, C.POINTER(C.c_float)), shape=(1, 48, 48, 64)).copy()
    r = O.conv_transpose2d(x, w1, 2, 0)
    r = O.gelu(O.bias_add(r.reshape(-1, 64), b1, "f32"), "f32").reshape(1, 24, 24, 64)
    r = O.bias_add(O.conv_transpose2d(r, w2, 2, 0).reshape(-1, 32), b2, "f32").reshape(1, 48, 48, 32)
    r = O.bias_add(O.conv2d(r, w3, 1, 0).reshape(-1, 64), b3, "f32").reshape(1, 48, 48, 64)
    r = O.bias_add(O.conv2d(r, w4, 1, 1).reshape(-1, 64), b4, "f32").reshape(1, 48, 48, 64)
    assert_f32_close(got, r, what="neck 4x stage")
