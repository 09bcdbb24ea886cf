"""The HIP backend behind sam3.c's vtable: graph_eval over host tensors,
with the gh_linear / gh_mlp chains (TRANSPOSE(W) -> MATMUL -> ADD -> GELU,
src/model/graph_helpers.c:297-320,1258-1276) folded into one GEMM, the
weight cache, and the host dispatcher for ops without a HIP kernel.
Results are compared with the oracle's node-by-node composition."""
import ctypes as C

import numpy as np
import pytest

from gpu_util import (assert_bf16_close, assert_f32_close, oracle, ref_linear, ref_q8,
                      require_gpu)
from sam3_amd import abi, hip, synth

pytestmark = pytest.mark.gpu


@pytest.fixture
def be():
    """A fresh backend per test: the weight cache is keyed by host address
    and these tests free and reuse host buffers without calling
    cache_invalidate (which sam3.c does when it recycles arena memory)."""
    require_gpu()
    b = hip.Backend(0)
    yield b
    b.close()


class GraphBuilder:
    """Hand-built graphs, as the reference tests build nodes by hand
    (tests/test_matmul_q8.c:27-59); keeps every buffer alive."""

    def __init__(self):
        self.g = abi.Graph()
        self.keep = []

    def tensor(self, dtype, dims, arr=None, ephemeral=0):
        if arr is None:
            n = int(np.prod(dims))
            esz = {abi.F32: 4, abi.F16: 2, abi.BF16: 2}[dtype]
            arr = np.zeros(n * esz, np.uint8)
        arr = np.ascontiguousarray(arr)
        self.keep.append(arr)
        t = abi.make_tensor(dtype, list(dims), arr.ctypes.data, arr.nbytes)
        t.ephemeral = ephemeral
        self.keep.append(t)
        return t, arr

    def node(self, op, inputs, output, params=(0, 0, 0, 0)):
        i = self.g.n_nodes
        n = self.g.nodes[i]
        n.op = op
        for k, t in enumerate(inputs):
            n.inputs[k] = C.pointer(t)
        n.n_inputs = len(inputs)
        n.output = C.pointer(output)
        for k, p in enumerate(params):
            n.params[k] = p
        self.g.n_nodes = i + 1


def linear_graph(dt, x, w, bias, gelu):
    """gh_linear (+ GELU): W stored [N,K] as the converter writes it."""
    M, K = x.shape
    N = w.shape[0] if dt != abi.Q8_0 else bias.shape[0]
    G = GraphBuilder()
    adt = abi.F32 if dt == abi.Q8_0 else dt
    tx, _ = G.tensor(adt, (M, K), x, ephemeral=1)
    tw, _ = G.tensor(dt, (N, K), w)
    twt, _ = G.tensor(dt, (K, N), np.zeros(w.nbytes, np.uint8))
    ty, _ = G.tensor(adt, (M, N))
    G.node(abi.OP_TRANSPOSE, [tw], twt)
    G.node(abi.OP_MATMUL, [tx, twt], ty)
    out = ty
    if bias is not None:
        tb, _ = G.tensor(adt, (N,), bias)
        tz, _ = G.tensor(adt, (M, N))
        G.node(abi.OP_ADD, [ty, tb], tz)
        out = tz
    if gelu:
        to, _ = G.tensor(adt, (M, N))
        G.node(abi.OP_GELU, [out], to)
        out = to
    return G, out


def out_array(t, dtype, shape):
    return np.ctypeslib.as_array(C.cast(t.data, C.POINTER(
        C.c_uint16 if dtype == np.uint16 else C.c_float)), shape=shape).copy()


def test_bf16_mlp_chain_folds_into_one_gemm(be):
    O = oracle()
    M, N, K = 300, 256, 192
    x = O.f32_to_bf16(synth.randn(1, (M, K))).reshape(M, K)
    w = O.f32_to_bf16(synth.randn(2, (N, K), 0.05)).reshape(N, K)
    bias = O.f32_to_bf16(synth.randn(3, N, 0.1))
    G, out = linear_graph(abi.BF16, x, w, bias, True)
    assert be.graph_eval(G.g) == abi.OK
    s = be.stats()
    assert (s.gpu_nodes, s.fused_nodes, s.host_nodes) == (1, 3, 0)
    got = out_array(out, np.uint16, (M, N))
    ref = O.gelu(O.bias_add(O.matmul_bf16(x, np.ascontiguousarray(
        O.transpose_u16(w)), 8), bias, "bf16"), "bf16").reshape(M, N)
    assert_bf16_close(got, ref, what="graph bf16 mlp")


def test_q8_linear_with_transpose_runs_nt(be):
    """TRANSPOSE of a Q8_0 weight is a byte no-op on the reference CPU
    backend (dtype size 0); folded here, the matmul reads W[N,K] blocks
    along K directly, which is what gh_linear means."""
    M, N, K = 96, 128, 256
    x = synth.randn(4, (M, K))
    w = oracle().q8_quantize(synth.randn(5, (N, K), 0.02))
    bias = synth.randn(6, N, 0.01)
    G, out = linear_graph(abi.Q8_0, x, w, bias, False)
    assert be.graph_eval(G.g) == abi.OK
    s = be.stats()
    assert (s.gpu_nodes, s.fused_nodes) == (1, 2)
    got = out_array(out, np.float32, (M, N))
    assert_f32_close(got, ref_q8(x, w, K, N, nt=True, bias=bias), what="graph q8 linear")


def test_weight_cache_and_invalidate(be):
    O = oracle()
    M, N, K = 64, 64, 64
    x = O.f32_to_bf16(synth.randn(7, (M, K))).reshape(M, K)
    w = O.f32_to_bf16(synth.randn(8, (N, K), 0.1)).reshape(N, K)
    G, out = linear_graph(abi.BF16, x, w, None, False)
    assert be.graph_eval(G.g) == abi.OK
    first = be.stats()
    assert first.uploads == 2 and first.downloads == 1
    assert be.graph_eval(G.g) == abi.OK
    again = be.stats()
    assert again.cache_hits == 1 and again.uploads == 1   # W cached, X ephemeral
    # the host changes W and invalidates it (backend.h:50-55)
    w2 = O.f32_to_bf16(synth.randn(9, (N, K), 0.1)).reshape(N, K)
    wt = G.g.nodes[0].inputs[0].contents
    C.memmove(wt.data, w2.ctypes.data, w2.nbytes)
    be.cache_invalidate(wt.data, w2.nbytes)
    assert be.graph_eval(G.g) == abi.OK
    assert be.stats().uploads == 2
    got = out_array(out, np.uint16, (M, N))
    assert_bf16_close(got, O.matmul_bf16(x, np.ascontiguousarray(O.transpose_u16(w2))),
                      what="after invalidate")


def test_plain_q8_matmul_kernel_contract(be):
    """MATMUL(A f32 [M,K], B Q8_0 [K,N]) with no transpose: the reference
    kernel contract (blocks over the flat [K,N] index)."""
    M, K, N = 16, 128, 32
    a = synth.randn(10, (M, K))
    b = oracle().q8_quantize(synth.randn(11, (K, N), 0.02))
    G = GraphBuilder()
    ta, _ = G.tensor(abi.F32, (M, K), a)
    tb, _ = G.tensor(abi.Q8_0, (K, N), b)
    tc, _ = G.tensor(abi.F32, (M, N))
    G.node(abi.OP_MATMUL, [ta, tb], tc)
    assert be.graph_eval(G.g) == abi.OK
    assert_f32_close(out_array(tc, np.float32, (M, N)), ref_q8(a, b, K, N, nt=False),
                     what="graph q8 kn")


def test_host_dispatch_for_ops_without_kernel(be):
    """SOFTMAX has no HIP kernel: without a host dispatcher graph_eval
    fails with SAM3_EDTYPE (as cpu_dispatch_node does for a missing
    kernel); with one, the node runs on the host between GPU nodes."""
    M, K, N = 8, 32, 16
    a = synth.randn(12, (M, K))
    b = synth.randn(13, (K, N))
    G = GraphBuilder()
    ta, _ = G.tensor(abi.F32, (M, K), a)
    tb, _ = G.tensor(abi.F32, (K, N), b)
    tc, _ = G.tensor(abi.F32, (M, N))
    ts, _ = G.tensor(abi.F32, (M, N))
    G.node(abi.OP_MATMUL, [ta, tb], tc)
    G.node(abi.OP_SOFTMAX, [tc], ts)
    be.set_host_dispatch(None)
    assert be.graph_eval(G.g) == abi.EDTYPE

    def softmax(node_p, ctx):
        node = C.cast(node_p, C.POINTER(abi.Node)).contents
        x = out_array(node.inputs[0].contents, np.float32, (M, N))
        e = np.exp(x - x.max(1, keepdims=True))
        y = (e / e.sum(1, keepdims=True)).astype(np.float32)
        C.memmove(node.output.contents.data, y.ctypes.data, y.nbytes)
        return abi.OK

    be.set_host_dispatch(softmax)
    try:
        assert be.graph_eval(G.g) == abi.OK
        assert be.stats().host_nodes == 1
        c = oracle().matmul_f32(a, b)
        e = np.exp(c - c.max(1, keepdims=True))
        assert_f32_close(out_array(ts, np.float32, (M, N)), e / e.sum(1, keepdims=True),
                         what="host softmax")
    finally:
        be.set_host_dispatch(None)


def test_alloc_tensor_pinned_arena(be):
    t = abi.Tensor()
    t.dtype, t.n_dims = abi.F32, 2
    t.dims[0], t.dims[1] = 3, 5
    assert be.alloc_tensor(t) == abi.OK
    assert t.data and t.nbytes == 60 and t.data % 256 == 0
    assert list(t.strides)[:2] == [5, 1]
    q = abi.Tensor()
    q.dtype, q.n_dims, q.dims[0] = abi.Q8_0, 1, 64
    assert be.alloc_tensor(q) == abi.EINVAL  # no element size (cpu_backend.c:97-101)
    be.arena_reset()


def _view(big, nbytes, dtype):
    """A host tensor buffer at the start of `big` (same address every time)."""
    return big[:nbytes].view(dtype)


def test_reused_host_address_copies_only_the_tensor_bytes(be):
    """sam3.c recycles arena memory between graphs without cache_invalidate
    (image_encoder.c:737-738). Eval 1 leaves at host address B a residency
    entry for fc1's output, written as fc2's bf16-planes operand (6 bytes per
    element on the device for a 4-byte-per-element host tensor). Eval 2's final
    output is a smaller f32 tensor at the same B: its readback must write
    exactly its own bytes, and the next eval's ephemeral input at B must be
    uploaded with exactly its own bytes."""
    O = oracle()
    M, K, N1, N2, N3 = 256, 256, 512, 256, 128
    big = np.full(M * N1 * 6 + 4096, 0x7F, np.uint8)
    x = synth.randn(11, (M, K))
    w1 = synth.randn(12, (N1, K), 0.05)
    b1 = synth.randn(13, N1, 0.1)
    w2 = synth.randn(14, (N2, N1), 0.05)
    w3 = synth.randn(15, (N3, K), 0.05)

    G = GraphBuilder()
    tx, _ = G.tensor(abi.F32, (M, K), x, ephemeral=1)
    tw1, _ = G.tensor(abi.F32, (N1, K), w1)
    tw1t, _ = G.tensor(abi.F32, (K, N1))
    th, _ = G.tensor(abi.F32, (M, N1))
    tb1, _ = G.tensor(abi.F32, (N1,), b1)
    thb, _ = G.tensor(abi.F32, (M, N1))
    tg = abi.make_tensor(abi.F32, [M, N1], big.ctypes.data, M * N1 * 4)
    G.keep.append(tg)
    tw2, _ = G.tensor(abi.F32, (N2, N1), w2)
    tw2t, _ = G.tensor(abi.F32, (N1, N2))
    ty, _ = G.tensor(abi.F32, (M, N2))
    G.node(abi.OP_TRANSPOSE, [tw1], tw1t)
    G.node(abi.OP_MATMUL, [tx, tw1t], th)
    G.node(abi.OP_ADD, [th, tb1], thb)
    G.node(abi.OP_GELU, [thb], tg)
    G.node(abi.OP_TRANSPOSE, [tw2], tw2t)
    G.node(abi.OP_MATMUL, [tg, tw2t], ty)
    assert be.graph_eval(G.g) == abi.OK
    assert be.stats().operand_writes >= 1, "fc1 did not write fc2's operand form"
    assert (big[M * N1 * 4:] == 0x7F).all(), "eval 1 wrote past its output"

    big[:] = 0x7F
    G2 = GraphBuilder()
    tx2, _ = G2.tensor(abi.F32, (M, K), x, ephemeral=1)
    tw3, _ = G2.tensor(abi.F32, (N3, K), w3)
    tw3t, _ = G2.tensor(abi.F32, (K, N3))
    ty3 = abi.make_tensor(abi.F32, [M, N3], big.ctypes.data, M * N3 * 4)
    G2.keep.append(ty3)
    G2.node(abi.OP_TRANSPOSE, [tw3], tw3t)
    G2.node(abi.OP_MATMUL, [tx2, tw3t], ty3)
    assert be.graph_eval(G2.g) == abi.OK
    assert (big[M * N3 * 4:] == 0x7F).all(), "readback wrote past the output tensor"
    got = _view(big, M * N3 * 4, np.float32).reshape(M, N3).copy()
    assert_f32_close(got, ref_linear("f32", x, w3, b_nt=True), what="eval 2 output")

    # eval 3: an ephemeral input of fewer bytes at B (the host rewrote it)
    x4 = synth.randn(16, (M // 2, K // 2))
    _view(big, x4.nbytes, np.float32)[:] = x4.reshape(-1)
    w4 = synth.randn(17, (64, K // 2), 0.05)
    G3 = GraphBuilder()
    tx4 = abi.make_tensor(abi.F32, [M // 2, K // 2], big.ctypes.data, x4.nbytes)
    tx4.ephemeral = 1
    G3.keep.append(tx4)
    tw4, _ = G3.tensor(abi.F32, (64, K // 2), w4)
    tw4t, _ = G3.tensor(abi.F32, (K // 2, 64))
    ty4, _ = G3.tensor(abi.F32, (M // 2, 64))
    G3.node(abi.OP_TRANSPOSE, [tw4], tw4t)
    G3.node(abi.OP_MATMUL, [tx4, tw4t], ty4)
    assert be.graph_eval(G3.g) == abi.OK
    assert_f32_close(out_array(ty4, np.float32, (M // 2, 64)),
                     ref_linear("f32", x4, w4, b_nt=True), what="eval 3 output")
