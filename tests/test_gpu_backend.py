"""The HIP backend behind sam3.c's vtable: graph_eval over host tensors,
with the gh_linear / gh_mlp chains (TRANSPOSE(W) -> MATMUL -> ADD -> GELU,
src/model/graph_helpers.c:297-320,1258-1276) folded into one GEMM, the
weight cache, and the host dispatcher for ops without a HIP kernel.
Results are compared with the oracle's node-by-node composition."""
import ctypes as C

import numpy as np
import pytest

from gpu_util import assert_bf16_close, assert_f32_close, oracle, ref_q8, require_gpu
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
