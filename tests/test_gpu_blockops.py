"""GPU parity of the ViT block ops (LAYERNORM, ROPE, SLICE, TRANSPOSE,
RESHAPE) and of a whole ViT block evaluated by the HIP backend's
graph_eval, against the oracle (pinned to the reference in
tests/test_oracle.py) and the reference's own CPU kernels.

  - ROPE, SLICE, TRANSPOSE, RESHAPE: bit for bit;
  - LAYERNORM: f32 within 1e-5 (mean and variance are summed in another
    order than the reference's left-to-right loop), bf16/f16 within their
    output bounds;
  - a ViT block (windowed and global) built node for node as
    image_encoder.c:755-916 builds it, run entirely on the GPU (no node is
    handed back to the host) and compared with the reference's
    cpu_dispatch_node loop over the same graph: f32 bound 1e-3.
"""
import ctypes as C
import itertools

import numpy as np
import pytest

from gpu_util import assert_bf16_close, assert_f16_close, assert_f32_close, oracle, require_gpu
from sam3_amd import abi, graph, hip, synth

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def gpu():
    require_gpu()


def kind_cast(x, kind):
    if kind == "f32":
        return np.ascontiguousarray(x, np.float32)
    O = oracle()
    conv = O.f32_to_bf16 if kind == "bf16" else O.f32_to_fp16
    return conv(x).reshape(np.shape(x))


DT = {"f32": abi.F32, "bf16": abi.BF16, "f16": abi.F16}


class Dev:
    """Device tensors for node-kernel calls; frees on exit."""

    def __init__(self):
        self.bufs, self.keep = [], []

    def t(self, dt, arr, dims=None):
        arr = np.ascontiguousarray(arr)
        b = hip.DeviceBuffer.of(arr)
        self.bufs.append(b)
        t = abi.make_tensor(dt, list(arr.shape if dims is None else dims), b.ptr, arr.nbytes)
        self.keep.append(t)
        return t, b

    def __enter__(self):
        return self

    def __exit__(self, *a):
        for b in self.bufs:
            b.free()


def run_node(fn, op, ins, out, params=(0, 0, 0, 0)):
    node = abi.make_node(op, ins, out, params)
    hip.check(fn(C.byref(node), None), f"op {op}")
    hip.synchronize()


# ------------------------------------------------------------- LayerNorm
@pytest.mark.parametrize("kind", ["f32", "bf16", "f16"])
@pytest.mark.parametrize("rows,cols", [(5184, 1024), (37, 96), (29, 160), (7, 3000), (3, 1), (130, 256),
                                       (64, 1536), (9, 512), (5, 2048), (11, 768)])
@pytest.mark.parametrize("affine", [2, 0])
def test_layernorm(kind, rows, cols, affine):
    O, lib = oracle(), hip.load()
    x = kind_cast(synth.randn(300 + cols, (rows, cols), 2.0, 0.5), kind)
    g = kind_cast(synth.randn(301, (cols,)), kind) if affine else None
    b = kind_cast(synth.randn(302, (cols,)), kind) if affine else None
    ref = O.layernorm(x, g, b, kind, threads=8)
    with Dev() as d:
        ins = [d.t(DT[kind], x)[0]] + ([d.t(DT[kind], g)[0], d.t(DT[kind], b)[0]] if affine else [])
        to, bo = d.t(DT[kind], np.zeros_like(x))
        for fn in (lib.sam3_hip_kernel_layernorm, lib.sam3_hip_dispatch_node):
            run_node(fn, abi.OP_LAYERNORM, ins, to)
            got = bo.download(x.dtype, x.shape)
            if kind == "f32":
                err = np.abs(got.astype(np.float64) - ref)
                assert err.max() <= 1e-5 * (1 + np.abs(ref).max()), err.max()
            elif kind == "bf16":
                assert_bf16_close(got, ref, what="layernorm bf16")
            else:
                assert_f16_close(got, ref, what="layernorm f16")


# ------------------------------------------------------------------ RoPE
@pytest.mark.parametrize("kind", ["f32", "bf16", "f16"])
@pytest.mark.parametrize("shape", [(81, 576, 16, 64), (1, 5184, 16, 64), (2, 9, 3, 16), (1, 1, 1, 2)])
def test_rope_bit_exact(kind, shape):
    O, lib = oracle(), hip.load()
    b, s, h, hd = shape
    x = kind_cast(synth.randn(310 + s, shape), kind)
    ang = synth.randn(311, (s, hd // 2), 3.0)
    c, sn = np.cos(ang).astype(np.float32), np.sin(ang).astype(np.float32)
    ref = O.rope(x, c, sn, kind)
    with Dev() as d:
        tx, _ = d.t(DT[kind], x)
        tc, _ = d.t(abi.F32, c)
        ts, _ = d.t(abi.F32, sn)
        to, bo = d.t(DT[kind], np.zeros_like(x))
        for fn in (lib.sam3_hip_kernel_rope, lib.sam3_hip_dispatch_node):
            run_node(fn, abi.OP_ROPE, [tx, tc, ts], to, (hd, 0, 0, 0))
            assert np.array_equal(bo.download(x.dtype, x.shape).view(np.uint8), ref.view(np.uint8))


# ------------------------------------------------------- slice, permute
@pytest.mark.parametrize("dt,npt", [(abi.F32, np.float32), (abi.BF16, np.uint16), (abi.I8, np.int8)])
@pytest.mark.parametrize("shape,axis,start,end", [((5184, 3072), 1, 1024, 2048), ((4, 10, 6), 1, 3, 8),
                                                   ((4, 10, 6), 0, 1, 4), ((4, 10, 6), 2, 5, 6),
                                                   ((7,), 0, 2, 5)])
def test_slice_exact(dt, npt, shape, axis, start, end):
    lib = hip.load()
    x = (synth.randn(320, shape) * 50).astype(npt)
    ref = np.take(x, np.arange(start, end), axis=axis)
    with Dev() as d:
        tx, _ = d.t(dt, x)
        to, bo = d.t(dt, np.zeros_like(ref))
        for fn in (lib.sam3_hip_kernel_slice, lib.sam3_hip_dispatch_node):
            run_node(fn, abi.OP_SLICE, [tx], to, (axis, start, end, 0))
            assert np.array_equal(bo.download(npt, ref.shape), ref)


PERM_CASES = ([((2, 3, 4, 5), p) for p in itertools.permutations(range(4))] +
              [((3, 5, 7), p) for p in itertools.permutations(range(3))] +
              [((6, 9), (1, 0)), ((9, 24, 9, 24 * 64), (0, 2, 1, 3)), ((81, 576, 16, 64), (0, 2, 1, 3)),
               ((5,), (0,))])


@pytest.mark.parametrize("dt,npt", [(abi.F32, np.float32), (abi.F16, np.float16), (abi.I8, np.int8)])
@pytest.mark.parametrize("shape,axes", PERM_CASES, ids=lambda v: str(v))
def test_permute_exact(dt, npt, shape, axes):
    lib = hip.load()
    x = (synth.randn(330, shape) * 50).astype(npt)
    ref = np.ascontiguousarray(x.transpose(axes))
    with Dev() as d:
        tx, _ = d.t(dt, x)
        to, bo = d.t(dt, np.zeros_like(ref))
        params = tuple(axes) + (0,) * (4 - len(axes))
        for fn in (lib.sam3_hip_kernel_transpose, lib.sam3_hip_dispatch_node):
            run_node(fn, abi.OP_TRANSPOSE, [tx], to, params)
            assert np.array_equal(bo.download(npt, ref.shape), ref)


def test_permute_matches_reference_kernel():
    """cpu_kernel_transpose itself on a 4-D case (the reference through
    oracle/_ref, when built)."""
    from oracle_bind import Ref, have_ref
    if not have_ref():
        pytest.skip("oracle/_ref not built")
    R = Ref()
    x = synth.randn(331, (3, 4, 5, 6))
    lib = hip.load()
    for axes in [(0, 2, 1, 3), (3, 1, 0, 2), (1, 0, 3, 2)]:
        ref = R.permute(x, abi.F32, axes)
        with Dev() as d:
            tx, _ = d.t(abi.F32, x)
            to, bo = d.t(abi.F32, np.zeros_like(ref))
            run_node(lib.sam3_hip_kernel_transpose, abi.OP_TRANSPOSE, [tx], to, axes)
            assert np.array_equal(bo.download(np.float32, ref.shape), ref)
    R.close()


def test_reshape_is_a_view():
    lib = hip.load()
    with Dev() as d:
        tx, bx = d.t(abi.F32, np.arange(24, dtype=np.float32))
        to = abi.make_tensor(abi.F32, [2, 3, 4], 0, 96)
        hip.check(lib.sam3_hip_kernel_reshape(C.byref(abi.make_node(abi.OP_RESHAPE, [tx], to))),
                  "reshape")
        assert to.data == bx.ptr and list(to.strides)[:3] == [12, 4, 1]


# ------------------------------------------------------- ViT block graph
def block_weights(G, seed, e, mlp):
    def w(i, shape, std):
        return G.tensor(abi.F32, shape, synth.randn(seed + i, shape, std))
    return {
        "ln1_w": w(1, (e,), 1.0), "ln1_b": w(2, (e,), 0.1),
        "qkv_w": w(3, (3 * e, e), 0.05), "qkv_b": w(4, (3 * e,), 0.02),
        "proj_w": w(5, (e, e), 0.05), "proj_b": w(6, (e,), 0.02),
        "ln2_w": w(7, (e,), 1.0), "ln2_b": w(8, (e,), 0.1),
        "fc1_w": w(9, (mlp, e), 0.05), "fc1_b": w(10, (mlp,), 0.02),
        "fc2_w": w(11, (e, mlp), 0.05), "fc2_b": w(12, (e,), 0.02),
    }


def build_block(grid, window, e, heads, mlp, is_global, seed):
    G = graph.Graph()
    x = G.tensor(abi.F32, (grid * grid, e), synth.randn(seed, (grid * grid, e)), ephemeral=1)
    p = block_weights(G, seed + 100, e, mlp)
    side = grid if is_global else window
    c, s = graph.rope_tables(side, e // heads)
    tc, ts = G.tensor(abi.F32, c.shape, c), G.tensor(abi.F32, s.shape, s)
    out = graph.vit_block(G, x, p, heads, grid, window, is_global, tc, ts)
    return G, out


def reference_eval(R, g, pool):
    """The reference CPU backend's graph_eval loop (cpu_backend.c:134-148):
    cpu_dispatch_node on each node in order. One substitution: the x86
    scalar build writes only the first rows/N outputs of a last-dim
    broadcast ADD (cpu_elementwise.c:357-384 splits the work by rows,
    add_f32_scalar :65-75 walks elements), so such a node runs the
    reference's same-shape add against the bias tiled to full size, which
    is what its NEON and AVX2 paths compute."""
    scratch = (C.c_char * 64)()
    keep = []
    for i in range(g.n_nodes):
        n = g.nodes[i]
        node = n
        if n.op == abi.OP_ADD and n.n_inputs == 2:
            a, b = n.inputs[0].contents, n.inputs[1].contents
            na = int(np.prod(list(a.dims)[:a.n_dims]))
            nb = int(np.prod(list(b.dims)[:b.n_dims]))
            if nb != na and b.dtype == abi.F32 and nb == a.dims[a.n_dims - 1]:
                bias = np.ctypeslib.as_array(C.cast(b.data, C.POINTER(C.c_float)), shape=(nb,))
                tiled = np.ascontiguousarray(np.tile(bias, na // nb))
                tb = abi.make_tensor(abi.F32, [na], tiled.ctypes.data, tiled.nbytes)
                node = abi.make_node(abi.OP_ADD, [a, tb], n.output.contents)
                keep += [tiled, tb, node]
        rc = R.lib.cpu_dispatch_node(C.byref(node), C.byref(scratch), pool)
        if rc != 0:
            return rc
    return 0


def out_array(t, shape):
    return np.ctypeslib.as_array(C.cast(t.data, C.POINTER(C.c_float)), shape=shape).copy()


@pytest.mark.parametrize("is_global", [False, True], ids=["windowed", "global"])
@pytest.mark.parametrize("e,heads", [(128, 2), (64, 2)], ids=["hd64", "hd32"])
def test_vit_block_graph_all_on_gpu(is_global, e, heads):
    """A ViT block (grid 8, window 4) through the HIP backend's graph_eval:
    every node runs on the GPU, and the block output matches the
    reference's CPU kernels run over the same graph."""
    from oracle_bind import Ref, have_ref
    if not have_ref():
        pytest.skip("oracle/_ref not built")
    grid, window, mlp = 8, 4, 4 * e
    Gh, oh = build_block(grid, window, e, heads, mlp, is_global, 400)
    Gr, orf = build_block(grid, window, e, heads, mlp, is_global, 400)
    be = hip.Backend(0)
    try:
        assert be.graph_eval(Gh.g) == abi.OK
        st = be.stats()
        assert st.host_nodes == 0, f"{st.host_nodes} nodes ran on the host"
        assert st.downloads == 1      # the block output only; intermediates stay
        got = out_array(oh, (grid * grid, e))
    finally:
        be.close()
    R = Ref()
    assert reference_eval(R, Gr.g, R.pool(8)) == 0
    ref = out_array(orf, (grid * grid, e))
    R.close()
    assert_f32_close(got, ref, what=f"vit block e={e} global={is_global}")


@pytest.mark.parametrize("wkind", ["f32", "q8"])
@pytest.mark.parametrize("via_reshape", [False, True])
def test_layernorm_written_as_gemm_operand(env, wkind, via_reshape):
    """LAYERNORM -> (RESHAPE ->) linear, as gh_mlp and the global-attention
    qkv build it: the LN writes the operand its one GEMM reads (bf16
    hi/lo planes for f32 weights, f16 for Q8_0 weights) instead of its f32
    output. That is the same arithmetic as LN then split/cast, so the
    result equals the unfused graph's bit for bit; both match LN + matmul
    of the oracle."""
    M, K, N = 1024, 512, 768
    O = oracle()
    x = synth.randn(800, (M, K), 2.0, 0.5)
    gam, bet = synth.randn(801, (K,)), synth.randn(802, (K,), 0.1)
    w = synth.randn(803, (N, K), 0.05)
    bias = synth.randn(804, (N,), 0.02)

    def run(mode):
        if mode is None:
            env.unset("SAM3_HIP_LN_OPERAND")
        else:
            env.set("SAM3_HIP_LN_OPERAND", mode)
        G = graph.Graph()
        tx = G.tensor(abi.F32, (M, K), x)
        t = G.layernorm(tx, G.tensor(abi.F32, (K,), gam), G.tensor(abi.F32, (K,), bet))
        if via_reshape:
            t = G.reshape(G.reshape(t, [1, M, K]), [M, K])
        tw = (G.tensor(abi.Q8_0, (N, K), O.q8_quantize(w)) if wkind == "q8"
              else G.tensor(abi.F32, (N, K), w))
        y = G.linear(t, tw, G.tensor(abi.F32, (N,), bias))
        be = hip.Backend(0)
        try:
            assert be.graph_eval(G.g) == abi.OK
            st = be.stats()
        finally:
            be.close()
        return np.ctypeslib.as_array(C.cast(y.data, C.POINTER(C.c_float)), shape=(M, N)).copy(), st

    fused, st = run(None)
    plain, st0 = run("0")
    assert st.operand_writes == 1 and st0.operand_writes == 0
    assert st.host_nodes == 0
    assert np.array_equal(fused.view(np.uint32), plain.view(np.uint32))
    ln = O.layernorm(x, gam, bet, "f32", threads=8)
    wd = O.q8_dequantize(O.q8_quantize(w), N * K).reshape(N, K) if wkind == "q8" else w
    ref = ln.astype(np.float64) @ wd.T.astype(np.float64) + bias
    assert_f32_close(fused, ref.astype(np.float32), what=f"LN -> linear {wkind}")


@pytest.mark.parametrize("wkind", ["f32", "q8"])
def test_gemm_written_as_next_gemm_operand(env, wkind):
    """gh_mlp (graph_helpers.c:1258-1276) after a LayerNorm: fc1's result,
    after its folded bias and GELU, is read only by fc2, which converts
    its A first (bf16 hi/lo planes for f32 weights, f16 for Q8_0 weights).
    fc1's epilogue writes that operand directly: the bias and GELU stay in
    f32 and the split / cast is the one the unfused graph applies to fc1's
    f32 output, so the result is the same bit for bit; both match the
    oracle's LN + MLP."""
    M, E, H = 1024, 256, 1024
    O = oracle()
    x = synth.randn(820, (M, E), 2.0, 0.5)
    gam, bet = synth.randn(821, (E,)), synth.randn(822, (E,), 0.1)
    w1, b1 = synth.randn(823, (H, E), 0.05), synth.randn(824, (H,), 0.02)
    w2, b2 = synth.randn(825, (E, H), 0.03), synth.randn(826, (E,), 0.02)

    def wt(G, w):
        return (G.tensor(abi.Q8_0, w.shape, O.q8_quantize(w)) if wkind == "q8"
                else G.tensor(abi.F32, w.shape, w))

    def run(mode):
        if mode is None:
            env.unset("SAM3_HIP_GEMM_OPERAND")
        else:
            env.set("SAM3_HIP_GEMM_OPERAND", mode)
        G = graph.Graph()
        t = G.layernorm(G.tensor(abi.F32, (M, E), x), G.tensor(abi.F32, (E,), gam),
                        G.tensor(abi.F32, (E,), bet))
        y = G.mlp(t, wt(G, w1), G.tensor(abi.F32, (H,), b1), wt(G, w2), G.tensor(abi.F32, (E,), b2))
        be = hip.Backend(0)
        try:
            assert be.graph_eval(G.g) == abi.OK
            st = be.stats()
        finally:
            be.close()
        return np.ctypeslib.as_array(C.cast(y.data, C.POINTER(C.c_float)), shape=(M, E)).copy(), st

    fused, st = run(None)
    plain, st0 = run("0")
    # LN2 -> fc1 always; fc1 -> fc2 only when enabled
    assert st.operand_writes == 2 and st0.operand_writes == 1
    assert st.host_nodes == 0 and st.downloads == 1
    assert np.array_equal(fused.view(np.uint32), plain.view(np.uint32))
    ln = O.layernorm(x, gam, bet, "f32", threads=8).astype(np.float64)

    def deq(w):
        return (O.q8_dequantize(O.q8_quantize(w), w.size).reshape(w.shape) if wkind == "q8"
                else w).astype(np.float64)
    h = O.gelu((ln @ deq(w1).T + b1).astype(np.float32), "f32").astype(np.float64)
    ref = h @ deq(w2).T + b2
    assert_f32_close(fused, ref.astype(np.float32), what=f"LN -> MLP {wkind}")


@pytest.mark.parametrize("wkind", ["f32", "q8"])
def test_permute_written_as_gemm_operand(env, wkind):
    """The attention head merge (gh_multihead_attention_rope, [B,H,N,D] ->
    [B,N,H,D] -> [B*N, H*D] -> out projection): an f32 TRANSPOSE that keeps
    its last axis and feeds only a GEMM's A writes that GEMM's operand
    (bf16 planes / f16) while permuting, the same split / cast the GEMM
    applies otherwise, so the result is the same bit for bit."""
    B, H, N, D, E = 2, 4, 256, 64, 256
    O = oracle()
    x = synth.randn(840, (B, H, N, D))
    w, bias = synth.randn(841, (E, H * D), 0.05), synth.randn(842, (E,), 0.02)

    def run(mode):
        if mode is None:
            env.unset("SAM3_HIP_PERMUTE_OPERAND")
        else:
            env.set("SAM3_HIP_PERMUTE_OPERAND", mode)
        G = graph.Graph()
        t = G.permute(G.tensor(abi.F32, x.shape, x), (0, 2, 1, 3))
        tw = (G.tensor(abi.Q8_0, w.shape, O.q8_quantize(w)) if wkind == "q8"
              else G.tensor(abi.F32, w.shape, w))
        y = G.linear(G.reshape(t, [B * N, H * D]), tw, G.tensor(abi.F32, (E,), bias))
        be = hip.Backend(0)
        try:
            assert be.graph_eval(G.g) == abi.OK
            st = be.stats()
        finally:
            be.close()
        return np.ctypeslib.as_array(C.cast(y.data, C.POINTER(C.c_float)), shape=(B * N, E)).copy(), st

    fused, st = run(None)
    plain, st0 = run("0")
    assert st.operand_writes == 1 and st0.operand_writes == 0
    assert st.host_nodes == 0 and st.downloads == 1
    assert np.array_equal(fused.view(np.uint32), plain.view(np.uint32))
    a = x.transpose(0, 2, 1, 3).reshape(B * N, H * D).astype(np.float64)
    wd = (O.q8_dequantize(O.q8_quantize(w), w.size).reshape(w.shape) if wkind == "q8"
          else w).astype(np.float64)
    assert_f32_close(fused, (a @ wd.T + bias).astype(np.float32), what=f"permute -> linear {wkind}")


def test_qkv_slice_rope_split_chain(env):
    """gh_multihead_attention_rope's q / k / v preparation: SLICE of the
    fused qkv rows -> RESHAPE [B,S,H,D] -> (ROPE -> RESHAPE -> RESHAPE) ->
    TRANSPOSE (0,2,1,3) runs in one kernel reading the qkv rows in place
    (no slice copies, no separate RoPE or permute pass), one launch for
    all three chains. Same bits as the
    node-by-node run (SAM3_HIP_QKV_CHAIN=0), and equal to RoPE by the
    reference's pair formula in float32 (products and sums rounded
    separately) followed by the head split."""
    side, H, D = 6, 4, 32
    B, S, E = 2, side * side, H * D
    qkv = synth.randn(860, (B * S, 3 * E))
    c, sn = graph.rope_tables(side, D)

    def run(mode):
        if mode is None:
            env.unset("SAM3_HIP_QKV_CHAIN")
        else:
            env.set("SAM3_HIP_QKV_CHAIN", mode)
        G = graph.Graph()
        x = G.tensor(abi.F32, (B * S, 3 * E), qkv)
        ct, st_ = G.tensor(abi.F32, c.shape, c), G.tensor(abi.F32, sn.shape, sn)
        sq, sk, sv = (G.slice(x, 1, i * E, (i + 1) * E) for i in range(3))
        four = [B, S, H, D]
        q = G.reshape(G.rope(G.reshape(sq, four), ct, st_), [B * S, E])
        k = G.reshape(G.rope(G.reshape(sk, four), ct, st_), [B * S, E])
        outs = [G.permute(G.reshape(t, four), (0, 2, 1, 3)) for t in (q, k, sv)]
        be = hip.Backend(0)
        try:
            assert be.graph_eval(G.g) == abi.OK
            st = be.stats()
        finally:
            be.close()
        return [np.ctypeslib.as_array(C.cast(t.data, C.POINTER(C.c_float)), shape=(B, H, S, D)).copy()
                for t in outs], st

    fused, st = run(None)
    plain, st0 = run("0")
    assert st.host_nodes == 0 and st.downloads == 3
    assert st.gpu_nodes == 1 and st0.gpu_nodes > 3
    for f, p in zip(fused, plain):
        assert np.array_equal(f.view(np.uint32), p.view(np.uint32))

    def rope_ref(v):
        v = v.reshape(B, S, H, D // 2, 2)
        cc, ss = c[None, :, None, :], sn[None, :, None, :]
        x0, x1 = v[..., 0], v[..., 1]
        o0 = (x0 * cc).astype(np.float32) - (x1 * ss).astype(np.float32)
        o1 = (x0 * ss).astype(np.float32) + (x1 * cc).astype(np.float32)
        return np.stack([o0, o1], -1).reshape(B, S, H, D)

    parts = [qkv[:, i * E:(i + 1) * E].reshape(B, S, H, D) for i in range(3)]
    refs = [rope_ref(parts[0]), rope_ref(parts[1]), parts[2]]
    for f, r in zip(fused, refs):
        assert np.array_equal(f.view(np.uint32), r.transpose(0, 2, 1, 3).astype(np.float32).view(np.uint32))


@pytest.mark.parametrize("cfg", [None, "20", "24", "2"], ids=["auto", "dlp256", "dlp192x128", "dl64"])
@pytest.mark.parametrize("geom", [(3, 8, 4, 64), (2, 12, 5, 32), (3, 8, 2, 128)],
                         ids=["s64h4d64", "s144h5d32", "s64h2d128"])
@pytest.mark.parametrize("wkind", ["f32", "q8"])
def test_qkv_projection_stores_attention_operands(env, wkind, geom, cfg):
    """gh_multihead_attention_rope after its LayerNorm (graph_helpers.c:
    721-882): LN -> linear qkv (+ bias) -> the q / k / v chains (SLICE ->
    RESHAPE -> ROPE -> ... -> TRANSPOSE 0,2,1,3). The qkv GEMM's epilogue
    stores the three head-split operands itself, RoPE applied to q and k
    after the bias, so the qkv rows are never written and the chain
    kernel does not run. Same bits as the chain kernel on the GEMM's f32
    result (SAM3_HIP_QKV_FOLD=0) on every tile shape (SAM3_HIP_DL_CFG;
    the non-pipelined "2" is replaced by the pipelined 128x128 tile), and
    equal to LN + matmul + RoPE of the oracle within f32 tolerance.
    Shapes: partial M and N tiles, head sizes of 32 (a wave's columns
    span two heads) and 128 (half a head)."""
    B, side, H, D = geom
    S, E, Ein = side * side, H * D, 256
    M = B * S
    O = oracle()
    x = synth.randn(870, (M, Ein), 2.0, 0.5)
    gam, bet = synth.randn(871, (Ein,)), synth.randn(872, (Ein,), 0.1)
    w = synth.randn(873, (3 * E, Ein), 0.05)
    bias = synth.randn(874, (3 * E,), 0.02)
    c, sn = graph.rope_tables(side, D)
    if cfg is None:
        env.unset("SAM3_HIP_DL_CFG")
    else:
        env.set("SAM3_HIP_DL_CFG", cfg)

    def run(mode):
        if mode is None:
            env.unset("SAM3_HIP_QKV_FOLD")
        else:
            env.set("SAM3_HIP_QKV_FOLD", mode)
        G = graph.Graph()
        tx = G.tensor(abi.F32, (M, Ein), x)
        t = G.layernorm(tx, G.tensor(abi.F32, (Ein,), gam), G.tensor(abi.F32, (Ein,), bet))
        tw = (G.tensor(abi.Q8_0, (3 * E, Ein), O.q8_quantize(w)) if wkind == "q8"
              else G.tensor(abi.F32, (3 * E, Ein), w))
        qkv = G.linear(t, tw, G.tensor(abi.F32, (3 * E,), bias))
        ct, st_ = G.tensor(abi.F32, c.shape, c), G.tensor(abi.F32, sn.shape, sn)
        sq, sk, sv = (G.slice(qkv, 1, i * E, (i + 1) * E) for i in range(3))
        four = [B, S, H, D]
        q = G.reshape(G.rope(G.reshape(sq, four), ct, st_), [M, E])
        k = G.reshape(G.rope(G.reshape(sk, four), ct, st_), [M, E])
        outs = [G.permute(G.reshape(t, four), (0, 2, 1, 3)) for t in (q, k, sv)]
        be = hip.Backend(0)
        try:
            assert be.graph_eval(G.g) == abi.OK
            st = be.stats()
        finally:
            be.close()
        return [np.ctypeslib.as_array(C.cast(t.data, C.POINTER(C.c_float)), shape=(B, H, S, D)).copy()
                for t in outs], st

    fused, st = run(None)
    plain, st0 = run("0")
    assert st.host_nodes == 0 and st0.host_nodes == 0
    assert st.gpu_nodes == st0.gpu_nodes - 1, (st.gpu_nodes, st0.gpu_nodes)
    for f, p in zip(fused, plain):
        assert np.array_equal(f.view(np.uint32), p.view(np.uint32))

    ln = O.layernorm(x, gam, bet, "f32", threads=8)
    wd = O.q8_dequantize(O.q8_quantize(w), w.size).reshape(w.shape) if wkind == "q8" else w
    y = (ln.astype(np.float64) @ wd.T.astype(np.float64) + bias).astype(np.float32)

    def rope_ref(v):
        v = v.reshape(B, S, H, D // 2, 2)
        cc, ss = c[None, :, None, :], sn[None, :, None, :]
        x0, x1 = v[..., 0], v[..., 1]
        o0 = (x0 * cc).astype(np.float32) - (x1 * ss).astype(np.float32)
        o1 = (x0 * ss).astype(np.float32) + (x1 * cc).astype(np.float32)
        return np.stack([o0, o1], -1).reshape(B, S, H, D)

    parts = [y[:, i * E:(i + 1) * E].reshape(B, S, H, D) for i in range(3)]
    refs = [rope_ref(parts[0]), rope_ref(parts[1]), parts[2]]
    for f, r, name in zip(fused, refs, "qkv"):
        assert_f32_close(f, r.transpose(0, 2, 1, 3), what=f"qkv epilogue {name} {wkind} {geom}")


@pytest.mark.parametrize("S", [1, 8, 77])
def test_skinny_qkv_stores_attention_operands(env, S):
    """The text encoder's attention operands (text_encoder.c:588-652, no
    RoPE): x -> linear qkv (Q8_0, + bias) on the streaming skinny kernel ->
    SLICE -> RESHAPE -> TRANSPOSE (0,2,1,3) for q, k and v. The skinny
    GEMM's epilogue stores the head-split operands itself: same bits as
    the chain kernel on its f32 result (SAM3_HIP_QKV_FOLD=0), and the
    oracle's Q8 matmul within f32 tolerance."""
    H, D, Ein = 16, 64, 1024
    E = H * D
    O = oracle()
    x = synth.randn(880 + S, (S, Ein))
    w = synth.randn(881, (3 * E, Ein), 0.02)
    bias = synth.randn(882, (3 * E,), 0.02)
    wq = O.q8_quantize(w)

    def run(mode):
        if mode is None:
            env.unset("SAM3_HIP_QKV_FOLD")
        else:
            env.set("SAM3_HIP_QKV_FOLD", mode)
        G = graph.Graph()
        tx = G.tensor(abi.F32, (S, Ein), x)
        qkv = G.linear(tx, G.tensor(abi.Q8_0, (3 * E, Ein), wq), G.tensor(abi.F32, (3 * E,), bias))
        four = [1, S, H, D]
        outs = [G.permute(G.reshape(G.slice(qkv, 1, i * E, (i + 1) * E), four), (0, 2, 1, 3))
                for i in range(3)]
        be = hip.Backend(0)
        try:
            assert be.graph_eval(G.g) == abi.OK
            st = be.stats()
        finally:
            be.close()
        return [np.ctypeslib.as_array(C.cast(t.data, C.POINTER(C.c_float)), shape=(1, H, S, D)).copy()
                for t in outs], st

    fused, st = run(None)
    plain, st0 = run("0")
    assert st.host_nodes == 0 and st0.host_nodes == 0
    assert st.gpu_nodes == 1 and st0.gpu_nodes == 2, (st.gpu_nodes, st0.gpu_nodes)
    for f, p in zip(fused, plain):
        assert np.array_equal(f.view(np.uint32), p.view(np.uint32))
    wd = O.q8_dequantize(wq, w.size).reshape(w.shape)
    y = (x.astype(np.float64) @ wd.T.astype(np.float64) + bias).astype(np.float32)
    for i, (f, name) in enumerate(zip(fused, "qkv")):
        ref = y[:, i * E:(i + 1) * E].reshape(1, S, H, D).transpose(0, 2, 1, 3)
        assert_f32_close(f, ref, what=f"skinny qkv epilogue {name} S={S}")


@pytest.mark.parametrize("dt", [abi.F32, abi.BF16, abi.F16], ids=["f32", "bf16", "f16"])
@pytest.mark.parametrize("B,H,S", [(1, 16, 1), (1, 16, 77), (2, 3, 300)])
def test_sdpa_stores_heads_merged(env, dt, B, H, S):
    """SDPA -> TRANSPOSE (0,2,1,3), the head merge of
    gh_multihead_attention_rope when no GEMM takes the result as its
    operand (the text encoder's skinny output projection): the attention
    kernel stores the merged rows itself, one launch instead of two.
    Same bits as the SDPA node followed by the permute kernel
    (SAM3_HIP_SDPA_MERGE=0), masked, on the MFMA kernel (D = 64) and the
    any-D kernel (D = 32)."""
    def to_dtype(x):
        if dt == abi.F32:
            return np.ascontiguousarray(x, np.float32)
        if dt == abi.F16:
            return np.ascontiguousarray(x, np.float32).astype(np.float16).view(np.uint16)
        return oracle().f32_to_bf16(x).reshape(x.shape)

    for D in (64, 32):
        q, k, v = (synth.randn(890 + i, (B, H, S, D)) for i in range(3))
        c = np.arange(S)
        mask = np.where(c[None, :] > c[:, None], np.float32(-1e9), np.float32(0)).astype(np.float32)
        nbytes = B * S * H * D * (4 if dt == abi.F32 else 2)

        def run(mode):
            if mode is None:
                env.unset("SAM3_HIP_SDPA_MERGE")
            else:
                env.set("SAM3_HIP_SDPA_MERGE", mode)
            G = graph.Graph()
            tq, tk, tv = (G.tensor(dt, x.shape, to_dtype(x)) for x in (q, k, v))
            o = G.permute(G.sdpa(tq, tk, tv, G.tensor(abi.F32, mask.shape, mask)), (0, 2, 1, 3))
            be = hip.Backend(0)
            try:
                assert be.graph_eval(G.g) == abi.OK
                st = be.stats()
            finally:
                be.close()
            got = np.ctypeslib.as_array(C.cast(o.data, C.POINTER(C.c_uint8)), shape=(nbytes,)).copy()
            return got, st

        fused, st = run(None)
        plain, st0 = run("0")
        assert st.gpu_nodes == 1 and st0.gpu_nodes == 2, (D, st.gpu_nodes, st0.gpu_nodes)
        assert np.array_equal(fused, plain), D


@pytest.mark.parametrize("wkind", ["f32", "q8"])
def test_sdpa_stores_heads_merged_gemm_operand(env, wkind):
    """gh_multihead_attention_rope's SDPA -> TRANSPOSE (0,2,1,3) ->
    RESHAPE -> output projection (the ViT block's path): the attention
    kernel stores the merged rows directly as the projection's operand
    (bf16 planes for f32 weights, f16 for Q8_0 weights) instead of f32
    rows that a permute kernel then converts: one launch fewer, the same
    bits as that permute (SAM3_HIP_SDPA_MERGE=0), and the oracle's
    attention + matmul within f32 tolerance."""
    B, H, S, D, N = 4, 4, 64, 64, 512
    E = H * D
    O = oracle()
    q, k, v = (synth.randn(895 + i, (B, H, S, D)) for i in range(3))
    w = synth.randn(898, (N, E), 0.05)
    bias = synth.randn(899, (N,), 0.02)

    def run(mode):
        if mode is None:
            env.unset("SAM3_HIP_SDPA_MERGE")
        else:
            env.set("SAM3_HIP_SDPA_MERGE", mode)
        G = graph.Graph()
        tq, tk, tv = (G.tensor(abi.F32, x.shape, x) for x in (q, k, v))
        a = G.reshape(G.permute(G.sdpa(tq, tk, tv), (0, 2, 1, 3)), [B * S, E])
        tw = (G.tensor(abi.Q8_0, (N, E), O.q8_quantize(w)) if wkind == "q8"
              else G.tensor(abi.F32, (N, E), w))
        y = G.linear(a, tw, G.tensor(abi.F32, (N,), bias))
        be = hip.Backend(0)
        try:
            assert be.graph_eval(G.g) == abi.OK
            st = be.stats()
        finally:
            be.close()
        return np.ctypeslib.as_array(C.cast(y.data, C.POINTER(C.c_float)), shape=(B * S, N)).copy(), st

    fused, st = run(None)
    plain, st0 = run("0")
    assert st.host_nodes == 0 and st0.host_nodes == 0
    assert st.gpu_nodes == st0.gpu_nodes - 1, (st.gpu_nodes, st0.gpu_nodes)
    assert st.operand_writes == st0.operand_writes == 1
    assert np.array_equal(fused.view(np.uint32), plain.view(np.uint32))
    att = O.sdpa(q.reshape(B * H, S, D), k.reshape(B * H, S, D), v.reshape(B * H, S, D), None, 8)
    a = att.reshape(B, H, S, D).transpose(0, 2, 1, 3).reshape(B * S, E).astype(np.float64)
    wd = O.q8_dequantize(O.q8_quantize(w), w.size).reshape(w.shape) if wkind == "q8" else w
    assert_f32_close(fused, (a @ wd.T.astype(np.float64) + bias).astype(np.float32),
                     what=f"sdpa -> merged operand -> linear {wkind}")


@pytest.mark.parametrize("wkind", ["f32", "q8"])
def test_residual_add_folded_into_gemm(env, wkind):
    """x + linear(LN(x)) as the ViT block builds its residuals
    (image_encoder.c:755-916): the ADD of the earlier f32 tensor is done in
    the GEMM epilogue after the bias, one f32 rounding as the ADD node
    does, so the result is the same bit for bit as the unfolded graph."""
    M, E = 1024, 512
    O = oracle()
    x = synth.randn(870, (M, E))
    gam, bet = synth.randn(871, (E,)), synth.randn(872, (E,), 0.1)
    w, bias = synth.randn(873, (E, E), 0.04), synth.randn(874, (E,), 0.02)

    def run(mode):
        if mode is None:
            env.unset("SAM3_HIP_RESIDUAL_FOLD")
        else:
            env.set("SAM3_HIP_RESIDUAL_FOLD", mode)
        G = graph.Graph()
        tx = G.tensor(abi.F32, (M, E), x)
        t = G.layernorm(tx, G.tensor(abi.F32, (E,), gam), G.tensor(abi.F32, (E,), bet))
        tw = (G.tensor(abi.Q8_0, w.shape, O.q8_quantize(w)) if wkind == "q8"
              else G.tensor(abi.F32, w.shape, w))
        y = G.add(tx, G.linear(t, tw, G.tensor(abi.F32, (E,), bias)))
        be = hip.Backend(0)
        try:
            assert be.graph_eval(G.g) == abi.OK
            st = be.stats()
        finally:
            be.close()
        return np.ctypeslib.as_array(C.cast(y.data, C.POINTER(C.c_float)), shape=(M, E)).copy(), st

    fused, st = run(None)
    plain, st0 = run("0")
    assert st.fused_nodes == st0.fused_nodes + 1 and st.gpu_nodes == st0.gpu_nodes - 1
    assert st.host_nodes == 0 and st.downloads == 1
    assert np.array_equal(fused.view(np.uint32), plain.view(np.uint32))
    ln = O.layernorm(x, gam, bet, "f32", threads=8).astype(np.float64)
    wd = (O.q8_dequantize(O.q8_quantize(w), w.size).reshape(w.shape) if wkind == "q8"
          else w).astype(np.float64)
    assert_f32_close(fused, (x + ln @ wd.T + bias).astype(np.float32), what=f"x + linear {wkind}")


@pytest.mark.parametrize("wkind", ["f32", "q8"])
def test_unpartition_and_residual_folded_into_gemm(env, wkind):
    """The windowed block's output projection: linear on window rows ->
    gh_window_unpartition (RESHAPE -> TRANSPOSE (0,2,1,3) -> RESHAPE) ->
    x + that. The epilogue stores each C row at its unpartitioned row and
    adds x there, so the three nodes and the ADD run inside the GEMM; same
    bits as the node-by-node run, and equal to the oracle's reference."""
    grid, ws, E = 24, 8, 256
    nw = grid // ws
    M = grid * grid
    O = oracle()
    a = synth.randn(880, (M, E))
    x = synth.randn(881, (M, E))
    gam, bet = synth.randn(884, (E,)), synth.randn(885, (E,), 0.1)
    w, bias = synth.randn(882, (E, E), 0.04), synth.randn(883, (E,), 0.02)

    def run(mode):
        if mode is None:
            env.unset("SAM3_HIP_UNPARTITION_FOLD")
        else:
            env.set("SAM3_HIP_UNPARTITION_FOLD", mode)
        G = graph.Graph()
        tw = (G.tensor(abi.Q8_0, w.shape, O.q8_quantize(w)) if wkind == "q8"
              else G.tensor(abi.F32, w.shape, w))
        t = G.layernorm(G.tensor(abi.F32, (M, E), a), G.tensor(abi.F32, (E,), gam),
                        G.tensor(abi.F32, (E,), bet))
        aw = G.linear(t, tw, G.tensor(abi.F32, (E,), bias))
        un = G.window_unpartition(G.reshape(aw, [nw * nw, ws * ws, E]), ws, grid)
        y = G.add(G.tensor(abi.F32, (M, E), x), un)
        be = hip.Backend(0)
        try:
            assert be.graph_eval(G.g) == abi.OK
            st = be.stats()
        finally:
            be.close()
        return np.ctypeslib.as_array(C.cast(y.data, C.POINTER(C.c_float)), shape=(M, E)).copy(), st

    fused, st = run(None)
    plain, st0 = run("0")
    assert st.host_nodes == 0 and st.downloads == 1
    assert st.gpu_nodes == 2 and st0.gpu_nodes == 4  # LN + GEMM, or LN, GEMM, permute, ADD
    assert np.array_equal(fused.view(np.uint32), plain.view(np.uint32))
    wd = (O.q8_dequantize(O.q8_quantize(w), w.size).reshape(w.shape) if wkind == "q8"
          else w).astype(np.float64)
    ln = O.layernorm(a, gam, bet, "f32", threads=8).astype(np.float64)
    lin = ln @ wd.T + bias
    un_ref = lin.reshape(nw, nw, ws, ws * E).transpose(0, 2, 1, 3).reshape(M, E)
    assert_f32_close(fused, (x + un_ref).astype(np.float32), what=f"unpartition fold {wkind}")


@pytest.mark.parametrize("wkind", ["f32", "q8"])
def test_partition_folded_into_layernorm(env, wkind):
    """The windowed block's LN1 -> gh_window_partition -> qkv linear: the
    LayerNorm writes the GEMM's operand (bf16 planes / f16) with its rows
    already in window order, so the partition permute does not run; same
    bits as the node-by-node run, and equal to the oracle's LN ->
    partition -> linear."""
    grid, ws, E, N = 24, 8, 256, 768
    nw = grid // ws
    M = grid * grid
    O = oracle()
    x = synth.randn(890, (M, E), 2.0, 0.5)
    gam, bet = synth.randn(891, (E,)), synth.randn(892, (E,), 0.1)
    w, bias = synth.randn(893, (N, E), 0.04), synth.randn(894, (N,), 0.02)

    def run(mode):
        if mode is None:
            env.unset("SAM3_HIP_PARTITION_FOLD")
        else:
            env.set("SAM3_HIP_PARTITION_FOLD", mode)
        G = graph.Graph()
        t = G.layernorm(G.tensor(abi.F32, (M, E), x), G.tensor(abi.F32, (E,), gam),
                        G.tensor(abi.F32, (E,), bet))
        xw = G.window_partition(t, ws, grid)
        tw = (G.tensor(abi.Q8_0, w.shape, O.q8_quantize(w)) if wkind == "q8"
              else G.tensor(abi.F32, w.shape, w))
        y = G.linear(G.reshape(xw, [M, E]), tw, G.tensor(abi.F32, (N,), bias))
        be = hip.Backend(0)
        try:
            assert be.graph_eval(G.g) == abi.OK
            st = be.stats()
        finally:
            be.close()
        return np.ctypeslib.as_array(C.cast(y.data, C.POINTER(C.c_float)), shape=(M, N)).copy(), st

    fused, st = run(None)
    plain, st0 = run("0")
    assert st.host_nodes == 0 and st.downloads == 1
    assert st.gpu_nodes == 2 and st0.gpu_nodes == 3  # LN + GEMM, or LN, permute, GEMM
    assert np.array_equal(fused.view(np.uint32), plain.view(np.uint32))
    ln = O.layernorm(x, gam, bet, "f32", threads=8).astype(np.float64)
    part = ln.reshape(nw, ws, nw, ws * E).transpose(0, 2, 1, 3).reshape(M, E)
    wd = (O.q8_dequantize(O.q8_quantize(w), w.size).reshape(w.shape) if wkind == "q8"
          else w).astype(np.float64)
    assert_f32_close(fused, (part @ wd.T + bias).astype(np.float32), what=f"LN -> partition {wkind}")


def test_blocks_chained_across_evals():
    """The image encoder's block loop (image_encoder.c:736-915): blocks in
    separate graph_evals, each graph's output the next graph's input. With
    no_readback on the first graph its output stays on the device and is
    read there by the second (no upload of x); the result equals one graph
    of both blocks, and equals it again when the first graph reads back."""
    grid, window, e, heads, mlp = 8, 4, 128, 2, 512
    x0 = synth.randn(950, (grid * grid, e))
    c, s = graph.rope_tables(window, e // heads)

    def two_graphs(no_readback):
        G1, G2 = graph.Graph(), graph.Graph()
        x = G1.tensor(abi.F32, (grid * grid, e), x0, ephemeral=1)
        y1 = graph.vit_block(G1, x, block_weights(G1, 960, e, mlp), heads, grid, window, False,
                             G1.tensor(abi.F32, c.shape, c), G1.tensor(abi.F32, s.shape, s))
        G1.g.no_readback = no_readback
        G2.keep.append(y1)
        y2 = graph.vit_block(G2, y1, block_weights(G2, 970, e, mlp), heads, grid, window, False,
                             G2.tensor(abi.F32, c.shape, c), G2.tensor(abi.F32, s.shape, s))
        be = hip.Backend(0)
        try:
            assert be.graph_eval(G1.g) == abi.OK
            st1 = be.stats()
            assert be.graph_eval(G2.g) == abi.OK
            st2 = be.stats()
        finally:
            be.close()
        return out_array(y2, (grid * grid, e)), st1, st2

    G = graph.Graph()
    x = G.tensor(abi.F32, (grid * grid, e), x0, ephemeral=1)
    y1 = graph.vit_block(G, x, block_weights(G, 960, e, mlp), heads, grid, window, False,
                         G.tensor(abi.F32, c.shape, c), G.tensor(abi.F32, s.shape, s))
    y2 = graph.vit_block(G, y1, block_weights(G, 970, e, mlp), heads, grid, window, False,
                         G.tensor(abi.F32, c.shape, c), G.tensor(abi.F32, s.shape, s))
    be = hip.Backend(0)
    try:
        assert be.graph_eval(G.g) == abi.OK
        st = be.stats()
        one = out_array(y2, (grid * grid, e))
    finally:
        be.close()
    assert st.downloads == 1
    assert st.uploads == 27                   # x, 2 x 12 weights, the 2 RoPE tables
    fwd, st1, st2 = two_graphs(True)
    assert st1.downloads == 0 and st2.downloads == 1
    assert st1.uploads == 15 and st2.uploads == 12   # block 2 reads x on the device
    back, _, _ = two_graphs(False)
    assert np.array_equal(fwd.view(np.uint32), one.view(np.uint32))
    assert np.array_equal(back.view(np.uint32), one.view(np.uint32))


def _block_full(wkind, seed, deq_ref=False, is_global=False):
    """The windowed (or global) ViT-L block at its production shape (grid
    72, window 24, e 1024, 16 heads, MLP 4096), f32 or Q8_0 linear weights (the
    reference graph gets the dequantized Q8_0 weights in f32: its own Q8
    path through gh_linear's transpose is a no-op, cpu_transpose.c:
    355-366)."""
    O = oracle()
    grid, window, e, heads, mlp = 72, 24, 1024, 16, 4096
    G = graph.Graph()
    x = G.tensor(abi.F32, (grid * grid, e), synth.randn(seed, (grid * grid, e)), ephemeral=1)
    p = {}
    shapes = {"ln1_w": ((e,), 1.0), "ln1_b": ((e,), 0.1), "qkv_w": ((3 * e, e), 0.05),
              "qkv_b": ((3 * e,), 0.02), "proj_w": ((e, e), 0.05), "proj_b": ((e,), 0.02),
              "ln2_w": ((e,), 1.0), "ln2_b": ((e,), 0.1), "fc1_w": ((mlp, e), 0.05),
              "fc1_b": ((mlp,), 0.02), "fc2_w": ((e, mlp), 0.05), "fc2_b": ((e,), 0.02)}
    for i, (name, (shape, std)) in enumerate(shapes.items()):
        w = synth.randn(seed + 100 + i, shape, std)
        if len(shape) == 2 and wkind == "q8":
            blocks = O.q8_quantize(w)
            if deq_ref:
                p[name] = G.tensor(abi.F32, shape, O.q8_dequantize(blocks, w.size).reshape(shape))
            else:
                p[name] = G.tensor(abi.Q8_0, shape, blocks)
        else:
            p[name] = G.tensor(abi.F32, shape, w)
    c, s = graph.rope_tables(grid if is_global else window, e // heads)
    tc, ts = G.tensor(abi.F32, c.shape, c), G.tensor(abi.F32, s.shape, s)
    out = graph.vit_block(G, x, p, heads, grid, window, is_global, tc, ts)
    return G, out


@pytest.mark.parametrize("wkind", ["f32", "q8"])
def test_vit_block_full_size_windowed(env, wkind):
    """The production windowed block (5184 tokens, the SLOTS = 4 LayerNorm
    and the g = 24 row maps): the default run is bit-identical to the run
    with the partition, unpartition, qkv-epilogue and head-merge folds
    off, and matches the reference's CPU kernels run over the same
    graph."""
    from oracle_bind import Ref, have_ref
    if not have_ref():
        pytest.skip("oracle/_ref not built")
    M, e = 72 * 72, 1024

    def gpu_run(fold):
        for name in ("SAM3_HIP_PARTITION_FOLD", "SAM3_HIP_UNPARTITION_FOLD",
                     "SAM3_HIP_QKV_FOLD", "SAM3_HIP_SDPA_MERGE"):
            if fold:
                env.unset(name)
            else:
                env.set(name, "0")
        G, out = _block_full(wkind, 470)
        be = hip.Backend(0)
        try:
            assert be.graph_eval(G.g) == abi.OK
            st = be.stats()
            assert st.host_nodes == 0
            return out_array(out, (M, e)), st
        finally:
            be.close()

    y, st = gpu_run(True)
    y0, st0 = gpu_run(False)
    assert st.gpu_nodes < st0.gpu_nodes, "the folds did not apply"
    assert np.array_equal(y.view(np.uint32), y0.view(np.uint32))
    Gr, orf = _block_full(wkind, 470, deq_ref=True)
    R = Ref()
    assert reference_eval(R, Gr.g, R.pool(0)) == 0
    ref = out_array(orf, (M, e))
    R.close()
    # Q8_0: each of the block's five chained GEMMs (qkv, proj, fc1, fc2 and
    # the attention it feeds) rounds its activations and q*scale to f16,
    # about 3e-4 normwise each; the block output keeps the 1e-3 normwise
    # bound and cosine, with an elementwise floor of 1.5e-2 * rms(ref)
    # (2e-3 for the f32 weights)
    assert_f32_close(y, ref, floor=1.5e-2 if wkind == "q8" else 2e-3,
                     what=f"full-size windowed block {wkind}")


@pytest.mark.parametrize("wkind", ["f32", "q8"])
def test_vit_block_full_size_global(env, wkind):
    """The production global block (5184 tokens in one sequence: the qkv
    epilogue's RoPE over 5184 positions, attention over 5184 keys storing
    the projection's operand): bit-identical to the run with the
    qkv-epilogue, head-merge and residual folds off, and matching the
    reference's CPU kernels run over the same graph."""
    from oracle_bind import Ref, have_ref
    if not have_ref():
        pytest.skip("oracle/_ref not built")
    M, e = 72 * 72, 1024

    def gpu_run(fold):
        for name in ("SAM3_HIP_QKV_FOLD", "SAM3_HIP_SDPA_MERGE", "SAM3_HIP_RESIDUAL_FOLD"):
            if fold:
                env.unset(name)
            else:
                env.set(name, "0")
        G, out = _block_full(wkind, 480, is_global=True)
        be = hip.Backend(0)
        try:
            assert be.graph_eval(G.g) == abi.OK
            st = be.stats()
            assert st.host_nodes == 0
            return out_array(out, (M, e)), st
        finally:
            be.close()

    y, st = gpu_run(True)
    y0, st0 = gpu_run(False)
    assert st.gpu_nodes == 7 and st0.gpu_nodes > st.gpu_nodes, (st.gpu_nodes, st0.gpu_nodes)
    assert np.array_equal(y.view(np.uint32), y0.view(np.uint32))
    Gr, orf = _block_full(wkind, 480, deq_ref=True, is_global=True)
    R = Ref()
    assert reference_eval(R, Gr.g, R.pool(0)) == 0
    ref = out_array(orf, (M, e))
    R.close()
    assert_f32_close(y, ref, floor=1.5e-2 if wkind == "q8" else 2e-3,
                     what=f"full-size global block {wkind}")
