"""The text encoder's layer chain (text_encoder.c:559-660) through the HIP
backend's graph_eval: LN -> MHA with the fused QKV weight and the causal
mask -> + x -> LN -> MLP -> + x, several layers per graph_eval, for the
token counts of BASELINE config 4 (seq 1, 8, 32, 77), with Q8_0 or f32
linear weights at the production width (1024, 16 heads, MLP 4096).

Every node must run on the GPU. The output is compared with the
reference's own cpu_dispatch_node loop over the same graph (oracle/_ref);
for Q8_0 weights the reference graph gets the dequantized weights in f32
(its Q8 linear path is the same arithmetic on them, cpu_matmul_q8.c:
124-131). Bounds: f32 weights 1e-3 normwise with a 2e-3 * rms elementwise
floor; Q8_0 weights the same with a 1.5e-2 * rms floor (each of a
layer's four GEMMs rounds activations and q*scale to f16, about 3e-4
normwise each).
"""
import numpy as np
import pytest

from gpu_util import assert_f32_close, oracle, ref_q8, require_gpu
from sam3_amd import abi, graph, hip, synth
from test_gpu_blockops import out_array, reference_eval

pytestmark = pytest.mark.gpu

W, HEADS, MLP = 1024, 16, 4096


@pytest.fixture(scope="module", autouse=True)
def gpu():
    require_gpu()


def build(seq, n_layers, wkind, seed, deq_ref=False):
    O = oracle()
    G = graph.Graph()
    x = G.tensor(abi.F32, (seq, W), synth.randn(seed, (seq, W)), ephemeral=1)
    mask = G.tensor(abi.F32, (seq, seq), graph.causal_mask(seq))
    shapes = {"ln1_w": ((W,), 1.0), "ln1_b": ((W,), 0.1), "qkv_w": ((3 * W, W), 0.03),
              "qkv_b": ((3 * W,), 0.02), "proj_w": ((W, W), 0.03), "proj_b": ((W,), 0.02),
              "ln2_w": ((W,), 1.0), "ln2_b": ((W,), 0.1), "fc1_w": ((MLP, W), 0.03),
              "fc1_b": ((MLP,), 0.02), "fc2_w": ((W, MLP), 0.03), "fc2_b": ((W,), 0.02)}
    for li in range(n_layers):
        p = {}
        for i, (name, (shape, std)) in enumerate(shapes.items()):
            w = synth.randn(seed + 100 * (li + 1) + i, shape, std)
            if len(shape) == 2 and wkind == "q8":
                blocks = O.q8_quantize(w)
                p[name] = (G.tensor(abi.F32, shape, O.q8_dequantize(blocks, w.size).reshape(shape))
                           if deq_ref else G.tensor(abi.Q8_0, shape, blocks))
            else:
                p[name] = G.tensor(abi.F32, shape, w)
        x = graph.text_layer(G, x, p, HEADS, mask)
    return G, x


def test_causal_mask_matches_the_reference_rule():
    m = graph.causal_mask(5)
    assert m[0, 0] == 0 and m[0, 1] == np.float32(-1e9) and m[4, 0] == 0 and m[3, 4] < 0
    assert (np.triu(m, 1) == np.float32(-1e9))[np.triu_indices(5, 1)].all()
    assert (np.tril(m) == 0).all()


@pytest.mark.parametrize("seq", [1, 8, 32, 77])
@pytest.mark.parametrize("wkind", ["q8", "f32"])
def test_text_layers_graph_all_on_gpu(seq, wkind):
    from oracle_bind import Ref, have_ref
    if not have_ref():
        pytest.skip("oracle/_ref not built")
    n_layers = 2
    G, out = build(seq, n_layers, wkind, 1300 + seq)
    be = hip.Backend(0)
    try:
        assert be.graph_eval(G.g) == abi.OK
        st = be.stats()
        assert st.host_nodes == 0, f"{st.host_nodes} nodes ran on the host"
        got = out_array(out, (seq, W))
    finally:
        be.close()
    Gr, orf = build(seq, n_layers, wkind, 1300 + seq, deq_ref=True)
    R = Ref()
    assert reference_eval(R, Gr.g, R.pool(8)) == 0
    ref = out_array(orf, (seq, W))
    R.close()
    assert_f32_close(got, ref, floor=1.5e-2 if wkind == "q8" else 2e-3,
                     what=f"text layers seq {seq} {wkind}")


def test_text_chain_forwarded_between_evals_matches_one_eval():
    """Four layers as two graph_evals of two, the first's output left in HBM
    and wrapped as the second's input (the reference's batched block loop,
    text_encoder.c:559-575), equal bit for bit to the four layers in one
    eval."""
    seq = 77
    G1, out1 = build(seq, 4, "q8", 1400)
    be = hip.Backend(0)
    try:
        assert be.graph_eval(G1.g) == abi.OK
        one = out_array(out1, (seq, W))
    finally:
        be.close()
    O = oracle()
    xd = hip.DeviceBuffer.of(synth.randn(1400, (seq, W)))
    mask_h = graph.causal_mask(seq)
    shapes = {"ln1_w": ((W,), 1.0), "ln1_b": ((W,), 0.1), "qkv_w": ((3 * W, W), 0.03),
              "qkv_b": ((3 * W,), 0.02), "proj_w": ((W, W), 0.03), "proj_b": ((W,), 0.02),
              "ln2_w": ((W,), 1.0), "ln2_b": ((W,), 0.1), "fc1_w": ((MLP, W), 0.03),
              "fc1_b": ((MLP,), 0.02), "fc2_w": ((W, MLP), 0.03), "fc2_b": ((W,), 0.02)}
    Wg = graph.Graph()
    params = []
    for li in range(4):
        p = {}
        for i, (name, (shape, std)) in enumerate(shapes.items()):
            w = synth.randn(1400 + 100 * (li + 1) + i, shape, std)
            p[name] = (Wg.tensor(abi.Q8_0, shape, O.q8_quantize(w)) if len(shape) == 2
                       else Wg.tensor(abi.F32, shape, w))
        params.append(p)
    mask = Wg.tensor(abi.F32, (seq, seq), mask_h)
    x = abi.make_tensor(abi.F32, [seq, W], xd.ptr, seq * W * 4)
    Wg.keep.append(x)
    graphs = []
    for b0 in (0, 2):
        G = graph.Graph()
        G.keep.append(Wg)
        for li in (b0, b0 + 1):
            x = graph.text_layer(G, x, params[li], HEADS, mask)
        G.g.no_readback = b0 == 0
        graphs.append(G)
    be = hip.Backend(0)
    try:
        for G in graphs:
            assert be.graph_eval(G.g) == abi.OK
        two = out_array(x, (seq, W))
    finally:
        be.close()
        xd.free()
    assert np.array_equal(one.view(np.uint32), two.view(np.uint32))


def _eval(G, out, shape):
    be = hip.Backend(0)
    try:
        assert be.graph_eval(G.g) == abi.OK
        st = be.stats()
        assert st.host_nodes == 0
        return out_array(out, shape), st
    finally:
        be.close()


@pytest.mark.parametrize("seq", [1, 8, 32, 77])
def test_layernorm_folded_into_the_gemv_keeps_the_bits(seq, env):
    """The LayerNorms before the qkv and fc1 projections do not run on
    their own when the Q8_0 GEMM that reads them streams on the skinny
    kernel: the GEMM normalizes its input rows with the LayerNorm kernel's
    arithmetic (same sums in the same order, each step rounded the same
    way), so the layers' output must have the same bits as with the
    LayerNorm kernel run first (SAM3_HIP_LN_GEMV_FOLD=0), with two fewer
    kernels per layer."""
    n_layers = 2
    G, out = build(seq, n_layers, "q8", 1500 + seq)
    on, st_on = _eval(G, out, (seq, W))
    env.set("SAM3_HIP_LN_GEMV_FOLD", 0)
    G, out = build(seq, n_layers, "q8", 1500 + seq)
    off, st_off = _eval(G, out, (seq, W))
    assert np.array_equal(on.view(np.uint32), off.view(np.uint32))
    assert st_on.gpu_nodes == st_off.gpu_nodes - 2 * n_layers
    assert st_on.fused_nodes == st_off.fused_nodes + 2 * n_layers


@pytest.mark.parametrize("affine", ["none", "gamma"])
@pytest.mark.parametrize("M,K", [(1, 1024), (5, 2048), (40, 512)])
def test_layernorm_gemv_fold_without_beta(affine, M, K, env):
    """LN -> RESHAPE -> Q8_0 linear with gamma only, or no affine terms:
    folded and unfolded give the same bits, and both match the oracle's
    LayerNorm followed by the Q8_0 product."""
    O = oracle()
    N = 768
    x_h = synth.randn(1600 + M, (M, K)) * np.float32(3.0) + np.float32(0.5)
    g_h = synth.randn(1601, (K,), 1.0)
    w_h = O.q8_quantize(synth.randn(1602, (N, K), 0.03))

    def run():
        G = graph.Graph()
        x = G.tensor(abi.F32, (M, K), x_h)
        gm = G.tensor(abi.F32, (K,), g_h) if affine == "gamma" else None
        w = G.tensor(abi.Q8_0, (N, K), w_h)
        y = G.linear(G.reshape(G.layernorm(x, gm), [1, M, K]), w)
        return _eval(G, y, (M, N))

    on, st_on = run()
    env.set("SAM3_HIP_LN_GEMV_FOLD", 0)
    off, st_off = run()
    assert np.array_equal(on.view(np.uint32), off.view(np.uint32))
    assert st_on.gpu_nodes == st_off.gpu_nodes - 1
    xf = x_h.astype(np.float64)
    ln = (xf - xf.mean(1, keepdims=True)) / np.sqrt(xf.var(1, keepdims=True) + 1e-5)
    if affine == "gamma":
        ln = ln * g_h
    assert_f32_close(on, ref_q8(ln.astype(np.float32), w_h, K, N, nt=True),
                     what=f"LN gemv fold {affine} M={M} K={K}")


def test_one_token_attention_folded_into_the_gemv_keeps_the_bits(env):
    """At one token the attention (one query over one key per head) does
    not run on its own: the proj GEMV forms its output from q, k and v
    with the attention kernel's steps for a one-key row, so two layers
    give the same bits as with the attention kernel run first
    (SAM3_HIP_ATT_GEMV_FOLD=0), with one kernel fewer per layer."""
    n_layers = 2
    G, out = build(1, n_layers, "q8", 1700)
    on, st_on = _eval(G, out, (1, W))
    env.set("SAM3_HIP_ATT_GEMV_FOLD", 0)
    G, out = build(1, n_layers, "q8", 1700)
    off, st_off = _eval(G, out, (1, W))
    assert np.array_equal(on.view(np.uint32), off.view(np.uint32))
    assert st_on.gpu_nodes == st_off.gpu_nodes - n_layers
    assert st_on.fused_nodes == st_off.fused_nodes + n_layers


def _same_bits_or_nan(a, b):
    na, nb = np.isnan(a), np.isnan(b)
    assert np.array_equal(na, nb)
    assert np.array_equal(a[~na].view(np.uint32), b[~nb].view(np.uint32))


@pytest.mark.parametrize("case", ["plain", "nomask", "mask_neg_inf", "mask_big_neg", "score_inf",
                                  "q_nan", "v_neg_zero"])
@pytest.mark.parametrize("H,D", [(16, 64), (8, 32), (4, 128)])
def test_one_key_attention_gemv_fold_cases(case, H, D, env):
    """SDPA of one query over one key per head -> TRANSPOSE (0,2,1,3) ->
    RESHAPE -> Q8_0 linear (+ bias), folded and unfolded: the same bits,
    NaN where the attention kernel gives NaN. The reference's softmax of
    one key (cpu_sdpa.c:49-159): weight 1 for a finite score, so the
    output is v; a -inf score leaves the sum 0 and the output 0; an
    infinite or NaN score gives NaN (checked against the oracle's Q8_0
    product of those rows)."""
    O = oracle()
    K, N = H * D, 512
    rng = np.random.default_rng(1800 + H)
    q_h = rng.standard_normal((1, H, 1, D)).astype(np.float32)
    k_h = rng.standard_normal((1, H, 1, D)).astype(np.float32)
    v_h = rng.standard_normal((1, H, 1, D)).astype(np.float32)
    m_h = np.zeros((1, 1), np.float32)
    if case == "mask_neg_inf":
        m_h[0, 0] = -np.inf
    elif case == "mask_big_neg":
        m_h[0, 0] = np.float32(-1e9)
    elif case == "score_inf":
        q_h[0, 1, 0, :] = np.float32(1e30)
        k_h[0, 1, 0, :] = np.float32(1e30)
    elif case == "q_nan":
        q_h[0, 2, 0, 5] = np.nan
    elif case == "v_neg_zero":
        v_h[0, 0, 0, :8] = np.float32(-0.0)
    w_h = O.q8_quantize(synth.randn(1801, (N, K), 0.03))
    b_h = synth.randn(1802, (N,), 0.1)

    def run():
        G = graph.Graph()
        q, k, v = (G.tensor(abi.F32, (1, H, 1, D), t) for t in (q_h, k_h, v_h))
        m = None if case == "nomask" else G.tensor(abi.F32, (1, 1), m_h)
        a = G.permute(G.sdpa(q, k, v, m, D), (0, 2, 1, 3))
        y = G.linear(G.reshape(a, [1, K]), G.tensor(abi.Q8_0, (N, K), w_h),
                     G.tensor(abi.F32, (N,), b_h))
        return _eval(G, y, (1, N))

    on, st_on = run()
    env.set("SAM3_HIP_ATT_GEMV_FOLD", 0)
    off, st_off = run()
    _same_bits_or_nan(on, off)
    assert st_on.gpu_nodes == st_off.gpu_nodes - 1
    # the attention output the reference forms, per head
    att = v_h.reshape(H, D).copy()
    if case == "mask_neg_inf":
        att[:] = 0.0
    elif case == "score_inf":
        att[1] = np.nan
    elif case == "q_nan":
        att[2] = np.nan
    ref = ref_q8(att.reshape(1, K), w_h, K, N, nt=True, bias=b_h).reshape(1, N)
    if case in ("score_inf", "q_nan"):
        assert np.isnan(on).all()
    else:
        assert_f32_close(on, ref, what=f"one-key attention gemv {case} H={H} D={D}")
