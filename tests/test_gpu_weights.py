"""Weights in HBM: sam3_hip_backend_map_weights (a `.sam3` data blob
copied to HBM once, then read in place by graph_eval) and
sam3_hip_backend_fuse_rows (the QKV stacking of image_encoder.c:223-254,
dtype-preserving).

  - a mapped range reads back byte for byte at every offset, across
    staging chunks and lanes;
  - a ViT block whose weights come from a `.sam3` file (f32, and Q8_0
    linear weights) gives the same bits with the blob mapped as with
    per-tensor uploads, and (f32) matches the reference's CPU kernels over
    the same graph within 1e-3;
  - fused tensors are the byte concatenation of their parts, in the
    parts' dtype; bad shapes and mixed dtypes return the documented
    errors.
"""
import ctypes as C

import numpy as np
import pytest

from gpu_util import assert_f32_close, oracle, require_gpu
from sam3_amd import abi, graph, hip, synth
from sam3_amd import weights as W

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def gpu():
    require_gpu()


@pytest.mark.parametrize("lanes,chunk_mb,nbytes", [(None, None, 5 * (4 << 20) + 4096 * 3 + 13),
                                                   (3, 1, (5 << 20) + 7), (1, 1, 4097)],
                         ids=["default", "3lanes", "one_lane_small"])
def test_map_weights_reads_back(monkeypatch, lanes, chunk_mb, nbytes):
    if lanes:
        monkeypatch.setenv("SAM3_HIP_UPLOAD_LANES", str(lanes))
        monkeypatch.setenv("SAM3_HIP_UPLOAD_CHUNK_MB", str(chunk_mb))
    host = np.random.default_rng(nbytes).integers(0, 256, nbytes, dtype=np.uint8)
    be = hip.Backend(0)
    try:
        hip.check(be.map_weights(host.ctypes.data, nbytes), "map_weights")
        base = be.weight_ptr(host.ctypes.data)
        assert base
        assert np.array_equal(hip.download_ptr(base, nbytes), host)
        for off in (1, min(12345, nbytes - 2), nbytes - 1):
            assert be.weight_ptr(host.ctypes.data + off) == base + off
        assert be.weight_ptr(host.ctypes.data + nbytes) is None
    finally:
        be.close()


def test_map_weights_errors_and_invalidate():
    host = np.arange(1 << 20, dtype=np.uint8)
    be = hip.Backend(0)
    dev = hip.DeviceBuffer(4096)
    try:
        p = host.ctypes.data
        assert be.map_weights(p, 0) == abi.EINVAL
        assert be.map_weights(None, 16) == abi.EINVAL
        assert be.map_weights(dev.ptr, 4096) == abi.EINVAL
        hip.check(be.map_weights(p + 4096, 8192), "map_weights")
        assert be.map_weights(p, 4097) == abi.EINVAL      # overlaps the mapped range
        assert be.map_weights(p + 8192, 100) == abi.EINVAL
        hip.check(be.map_weights(p, 4096), "map_weights")  # adjacent: fine
        be.cache_invalidate(p + 10000, 1)                  # touches the second range
        assert be.weight_ptr(p + 5000) is None
        assert be.weight_ptr(p + 100)
        hip.check(be.map_weights(p + 4096, host.nbytes - 4096), "map_weights")
        got = hip.download_ptr(be.weight_ptr(p + 4096), host.nbytes - 4096)
        assert np.array_equal(got, host[4096:])
    finally:
        dev.free()
        be.close()


def block_from_file(wf, be, grid, window, e, heads, is_global, seed):
    G = graph.Graph()
    x = G.tensor(abi.F32, (grid * grid, e), synth.randn(seed, (grid * grid, e)), ephemeral=1)
    p = graph.load_vit_layer(G, wf, 0, be)
    c, s = graph.rope_tables(grid if is_global else window, e // heads)
    tc, ts = G.tensor(abi.F32, c.shape, c), G.tensor(abi.F32, s.shape, s)
    out = graph.vit_block(G, x, p, heads, grid, window, is_global, tc, ts)
    return G, out


def out_array(t, shape):
    return np.ctypeslib.as_array(C.cast(t.data, C.POINTER(C.c_float)), shape=shape).copy()


@pytest.mark.parametrize("wkind", ["f32", "q8"])
@pytest.mark.parametrize("is_global", [False, True], ids=["windowed", "global"])
def test_vit_block_from_sam3_file(tmp_path, wkind, is_global):
    grid, window, e, heads, mlp = 8, 4, 128, 2, 512
    quant = oracle().q8_quantize if wkind == "q8" else None
    path = tmp_path / "layer.sam3"
    W.write(path, graph.vit_layer_entries(0, e, mlp, 900, quant))
    with W.WeightFile(path) as wf:
        # mapped blob, q/k/v stacked in HBM
        be = hip.Backend(0)
        try:
            hip.check(be.map_weights(wf.data_base, wf.data_size), "map_weights")
            G, out = block_from_file(wf, be, grid, window, e, heads, is_global, 77)
            assert be.graph_eval(G.g) == abi.OK
            st = be.stats()
            got = out_array(out, (grid * grid, e))
        finally:
            be.close()
        assert st.host_nodes == 0
        assert st.mapped_reads >= 10, st.mapped_reads   # LN, proj, fc1, fc2 weights and biases
        assert st.uploads == 3, st.uploads              # x and the two RoPE tables only
        # no mapping, q/k/v stacked on the host, per-tensor uploads
        be = hip.Backend(0)
        try:
            G2, out2 = block_from_file(wf, None, grid, window, e, heads, is_global, 77)
            assert be.graph_eval(G2.g) == abi.OK
            st2 = be.stats()
            plain = out_array(out2, (grid * grid, e))
        finally:
            be.close()
        assert st2.mapped_reads == 0 and st2.uploads == 15
        assert np.array_equal(got.view(np.uint32), plain.view(np.uint32))
        if wkind == "f32":
            from oracle_bind import Ref, have_ref
            from test_gpu_blockops import reference_eval
            if have_ref():
                G3, out3 = block_from_file(wf, None, grid, window, e, heads, is_global, 77)
                R = Ref()
                assert reference_eval(R, G3.g, R.pool(8)) == 0
                ref = out_array(out3, (grid * grid, e))
                R.close()
                assert_f32_close(got, ref, what=f"vit block from .sam3 global={is_global}")


def test_fuse_rows_q8_from_mapped_blob(tmp_path):
    e = 96
    ents = graph.vit_layer_entries(3, e, 4 * e, 50, oracle().q8_quantize)
    W.write(tmp_path / "l.sam3", ents)
    byname = {n: a for n, _, _, a in ents}
    with W.WeightFile(tmp_path / "l.sam3") as wf:
        be = hip.Backend(0)
        try:
            hip.check(be.map_weights(wf.data_base, wf.data_size), "map_weights")
            keys = ("q_w", "k_w", "v_w")
            names = [graph.VIT_PREFIX + graph.VIT_NAMES[k].format(3) for k in keys]
            parts = [wf.to_tensor(wf.find(n)) for n in names]
            out = abi.Tensor()
            hip.check(be.fuse_rows(parts, out), "fuse_rows")
            assert out.dtype == abi.Q8_0 and out.n_dims == 2
            assert list(out.dims)[:2] == [3 * e, e] and list(out.strides) == [0, 0, 0, 0]
            assert out.nbytes == 3 * abi.q8_nbytes(e * e)
            want = np.concatenate([byname[n] for n in names])
            assert np.array_equal(hip.download_ptr(out.data, out.nbytes), want)
            # host parts (F32 biases) and device parts
            bn = [graph.VIT_PREFIX + graph.VIT_NAMES[k].format(3) for k in ("q_b", "k_b", "v_b")]
            host = [np.ascontiguousarray(byname[n]) for n in bn]
            hp = [abi.make_tensor(abi.F32, [e], h.ctypes.data, h.nbytes) for h in host]
            ob = abi.Tensor()
            hip.check(be.fuse_rows(hp, ob), "fuse_rows host")
            assert ob.dtype == abi.F32 and ob.n_dims == 1 and ob.dims[0] == 3 * e
            assert np.array_equal(hip.download_ptr(ob.data, ob.nbytes, np.float32),
                                  np.concatenate(host))
            dev = [hip.DeviceBuffer.of(h) for h in host]
            dp = [abi.make_tensor(abi.F32, [e], d.ptr, h.nbytes) for d, h in zip(dev, host)]
            od = abi.Tensor()
            hip.check(be.fuse_rows(dp, od), "fuse_rows device")
            assert np.array_equal(hip.download_ptr(od.data, od.nbytes, np.float32),
                                  np.concatenate(host))
            for d in dev:
                d.free()
        finally:
            be.close()


def test_fuse_rows_errors():
    be = hip.Backend(0)
    a = np.zeros(64, np.float32)
    q = np.zeros(abi.q8_nbytes(48), np.uint8)
    try:
        f = abi.make_tensor(abi.F32, [4, 16], a.ctypes.data, a.nbytes)
        g = abi.make_tensor(abi.F32, [2, 32], a.ctypes.data, a.nbytes)
        h = abi.make_tensor(abi.F16, [4, 16], a.ctypes.data, 128)
        q48 = abi.make_tensor(abi.Q8_0, [3, 16], q.ctypes.data, q.nbytes)
        three = abi.make_tensor(abi.F32, [1, 4, 16], a.ctypes.data, a.nbytes)
        out = abi.Tensor()
        assert be.fuse_rows([f, g], out) == abi.EINVAL     # columns differ
        assert be.fuse_rows([f, h], out) == abi.EDTYPE     # dtypes differ
        assert be.fuse_rows([q48, q48], out) == abi.EINVAL  # a block would span two parts
        assert be.fuse_rows([three], out) == abi.EINVAL    # rank 3
        assert be.fuse_rows([], out) == abi.EINVAL
    finally:
        be.close()


def test_prepared_weights_reused_and_dropped():
    """The bf16 planes of constant f32 weights are made once per backend:
    a second eval reuses them (prep_hits) with identical bits, and
    cache_invalidate of one weight's host range drops its planes, so the
    next eval uses the new values (equal to a fresh backend's result)."""
    from test_gpu_blockops import block_weights
    grid, window, e, heads, mlp = 16, 8, 256, 4, 1024

    def build():
        G = graph.Graph()
        x = G.tensor(abi.F32, (grid * grid, e), synth.randn(70, (grid * grid, e)), ephemeral=1)
        p = block_weights(G, 170, e, mlp)
        c, s = graph.rope_tables(window, e // heads)
        tc, ts = G.tensor(abi.F32, c.shape, c), G.tensor(abi.F32, s.shape, s)
        return G, p, graph.vit_block(G, x, p, heads, grid, window, False, tc, ts)

    G, p, out = build()
    be = hip.Backend(0)
    try:
        assert be.graph_eval(G.g) == abi.OK
        y1, st1 = out_array(out, (grid * grid, e)), be.stats()
        assert be.graph_eval(G.g) == abi.OK
        y2, st2 = out_array(out, (grid * grid, e)), be.stats()
        w = p["fc2_w"]
        wa = np.ctypeslib.as_array(C.cast(w.data, C.POINTER(C.c_float)), shape=(e * mlp,))
        wa *= 2.0
        be.cache_invalidate(w.data, w.nbytes)
        assert be.graph_eval(G.g) == abi.OK
        y3, st3 = out_array(out, (grid * grid, e)), be.stats()
    finally:
        be.close()
    assert st1.prep_hits == 0 and st2.prep_hits == 4 and st3.prep_hits == 3
    assert np.array_equal(y1.view(np.uint32), y2.view(np.uint32))
    assert not np.array_equal(y2, y3)
    G4, p4, out4 = build()
    wa4 = np.ctypeslib.as_array(C.cast(p4["fc2_w"].data, C.POINTER(C.c_float)), shape=(e * mlp,))
    wa4 *= 2.0
    be = hip.Backend(0)
    try:
        assert be.graph_eval(G4.g) == abi.OK
        y4 = out_array(out4, (grid * grid, e))
    finally:
        be.close()
    assert np.array_equal(y3.view(np.uint32), y4.view(np.uint32))


@pytest.mark.parametrize("gelu", [False, True])
def test_q8_weights_expanded_once(env, gelu):
    """Inside graph_eval a constant Q8_0 weight of a large-M GEMM is
    expanded once to f16 (q*scale in f32, rounded once) and reused by
    later evals (prep_hits). The direct Q8 kernel (SAM3_HIP_Q8_EXPAND=0,
    which rounds the scale to f16 first) keeps only the weight's row
    factors, also made once (one prep hit in the second eval). Both
    match the reference's dequantized weights in float64; the expanded
    path is at least as close."""
    M, K, N = 2048, 1024, 768
    O = oracle()
    x = synth.randn(900, (M, K))
    wq = O.q8_quantize(synth.randn(901, (N, K), 0.03))
    bias = synth.randn(902, (N,), 0.02)

    def run(mode, evals=2):
        if mode is None:
            env.unset("SAM3_HIP_Q8_EXPAND")
        else:
            env.set("SAM3_HIP_Q8_EXPAND", mode)
        G = graph.Graph()
        t = G.linear(G.tensor(abi.F32, (M, K), x), G.tensor(abi.Q8_0, (N, K), wq),
                     G.tensor(abi.F32, (N,), bias))
        if gelu:
            t = G.unary(abi.OP_GELU, t)
        be = hip.Backend(0)
        stats = []
        try:
            for _ in range(evals):
                assert be.graph_eval(G.g) == abi.OK
                stats.append(be.stats())
        finally:
            be.close()
        return out_array(t, (M, N)), stats

    y, st = run(None)
    y0, st0 = run("0")
    assert st[0].prep_hits == 0 and st[1].prep_hits == 1
    assert st0[0].prep_hits == 0 and st0[1].prep_hits == 1
    assert st[1].host_nodes == 0
    wd = O.q8_dequantize(wq, N * K).reshape(N, K).astype(np.float64)
    ref = x.astype(np.float64) @ wd.T + bias
    if gelu:
        ref = O.gelu(ref.astype(np.float32), "f32").astype(np.float64)
    assert_f32_close(y, np.asarray(ref, np.float32), what=f"Q8 expanded gelu={gelu}")
    assert_f32_close(y0, np.asarray(ref, np.float32), what=f"Q8 direct gelu={gelu}")
    e_exp, e_dir = np.abs(y - ref).max(), np.abs(y0 - ref).max()
    assert e_exp <= 1.05 * e_dir + 1e-6, (e_exp, e_dir)
