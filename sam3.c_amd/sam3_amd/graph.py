"""Host-side graph building in the shape sam3.c's graph helpers give it.

The reference builds its model graphs with `gh_*` helpers
(src/model/graph_helpers.c) and hands them to a backend's `graph_eval`.
This module restates the helpers a ViT-L image-encoder block uses
(image_encoder.c:755-916) over the ctypes structs of `abi`, so the same
node sequence can be evaluated by the HIP backend and, in the tests, by
the reference's CPU kernels. Tensors own numpy buffers kept alive by the
builder; weights use the checkpoint layout [out, in].
"""
import ctypes as C

import numpy as np

from . import abi

_NP = {abi.F32: np.float32, abi.F16: np.float16, abi.BF16: np.uint16, abi.I32: np.int32,
       abi.I8: np.int8}


class Graph:
    """A `struct sam3_graph` plus the host buffers of its tensors."""

    def __init__(self):
        self.g = abi.Graph()
        self.keep = []

    # ---- tensors ----
    def tensor(self, dtype, dims, arr=None, ephemeral=0):
        """A tensor header over a host buffer (zeros when arr is None)."""
        if arr is None:
            n = int(np.prod(dims))
            arr = (np.zeros(abi.q8_nbytes(n), np.uint8) if dtype == abi.Q8_0
                   else np.zeros(n, _NP[dtype]))
        arr = np.ascontiguousarray(arr)
        self.keep.append(arr)
        t = abi.make_tensor(dtype, list(dims), arr.ctypes.data, arr.nbytes)
        t.ephemeral = ephemeral
        self.keep.append(t)
        return t

    def _out(self, like, dims=None, dtype=None):
        return self.tensor(like.dtype if dtype is None else dtype,
                           list(like.dims)[:like.n_dims] if dims is None else dims)

    def node(self, op, inputs, output, params=(0, 0, 0, 0)):
        """sam3_graph_add_op (src/core/graph.c) with raw int params."""
        i = self.g.n_nodes
        if i >= abi.GRAPH_MAX_NODES:
            raise RuntimeError("graph full")
        n = self.g.nodes[i]
        n.op = op
        for k, t in enumerate(inputs):
            n.inputs[k] = C.pointer(t)
        n.n_inputs = len(inputs)
        n.output = C.pointer(output)
        for k, p in enumerate(params):
            n.params[k] = p
        self.g.n_nodes = i + 1
        return output

    # ---- gh_* restated (graph_helpers.c) ----
    def layernorm(self, x, gamma=None, beta=None):
        """gh_layernorm (:324-349)."""
        ins = [x] + [t for t in (gamma, beta) if t is not None]
        return self.node(abi.OP_LAYERNORM, ins, self._out(x))

    def reshape(self, x, dims):
        """gh_reshape (:351-374): a view node; the output buffer is replaced
        by the input's when the node runs."""
        if int(np.prod(dims)) != int(np.prod(list(x.dims)[:x.n_dims])):
            raise ValueError("reshape: element count mismatch")
        return self.node(abi.OP_RESHAPE, [x], self._out(x, list(dims)))

    def transpose(self, w):
        """gh_transpose (:378-409): swap the last two dims, explicit axes."""
        nd = w.n_dims
        dims = list(w.dims)[:nd]
        dims[-2], dims[-1] = dims[-1], dims[-2]
        axes = list(range(nd))
        axes[-2], axes[-1] = axes[-1], axes[-2]
        return self.node(abi.OP_TRANSPOSE, [w], self._out(w, dims), tuple(axes) + (0,) * (4 - nd))

    def permute(self, x, axes):
        """gh_permute (:410-443)."""
        dims = [x.dims[a] for a in axes]
        return self.node(abi.OP_TRANSPOSE, [x], self._out(x, dims),
                         tuple(axes) + (0,) * (4 - len(axes)))

    def matmul(self, a, b):
        """gh_matmul (:276-293): [M,K] x [K,N]."""
        M, N = a.dims[a.n_dims - 2], b.dims[b.n_dims - 1]
        dt = abi.F32 if b.dtype == abi.Q8_0 else a.dtype
        return self.node(abi.OP_MATMUL, [a, b], self.tensor(dt, [M, N]))

    def add(self, x, y):
        """gh_add (:218-231)."""
        return self.node(abi.OP_ADD, [x, y], self._out(x))

    def unary(self, op, x):
        return self.node(op, [x], self._out(x))

    def linear(self, x, w, b=None):
        """gh_linear (:297-320): TRANSPOSE(W) -> MATMUL -> ADD(bias)."""
        out = self.matmul(x, self.transpose(w))
        return self.add(out, b) if b is not None else out

    def mlp(self, x, w1, b1, w2, b2, act=abi.OP_GELU):
        """gh_mlp (:1258-1276)."""
        return self.linear(self.unary(act, self.linear(x, w1, b1)), w2, b2)

    def slice(self, x, axis, start, end):
        """gh_slice (:587-613)."""
        dims = list(x.dims)[:x.n_dims]
        dims[axis] = end - start
        return self.node(abi.OP_SLICE, [x], self._out(x, dims), (axis, start, end, 0))

    def rope(self, x, cos_t, sin_t, grid_w=0, scale=1.0):
        """gh_rope (:664-684): params head_dim, grid_w, scale (f32 bits)."""
        sbits = int(np.float32(scale).view(np.int32))
        return self.node(abi.OP_ROPE, [x, cos_t, sin_t], self._out(x),
                         (x.dims[3], grid_w, sbits, 0))

    def sdpa(self, q, k, v, mask=None, head_dim=None):
        """gh_sdpa (:688-717)."""
        ins = [q, k, v] + ([mask] if mask is not None else [])
        return self.node(abi.OP_SDPA, ins, self._out(q), (head_dim or q.dims[q.n_dims - 1], 0, 0, 0))

    def window_partition(self, x, ws, grid):
        """gh_window_partition (:447-478): [np, e] -> [n_win, ws*ws, e]."""
        e, nw = x.dims[1], grid // ws
        t = self.permute(self.reshape(x, [nw, ws, nw, ws * e]), (0, 2, 1, 3))
        return self.reshape(t, [nw * nw, ws * ws, e])

    def window_unpartition(self, x, ws, grid):
        """gh_window_unpartition (:480-509): [n_win, ws*ws, e] -> [np, e]."""
        e, nw = x.dims[2], grid // ws
        t = self.permute(self.reshape(x, [nw, nw, ws, ws * e]), (0, 2, 1, 3))
        return self.reshape(t, [grid * grid, e])

    def mha_rope(self, x, qkv_w, qkv_b, out_w, out_b, n_heads, cos_t, sin_t, grid_w, scale,
                 mask=None):
        """gh_multihead_attention_rope (:721-882) with q = k = v = x
        [batch, seq, d_model]; no RoPE when cos_t / sin_t are None
        (:774), an additive [seq, seq] mask when given (:842-843)."""
        batch, seq, d = x.dims[0], x.dims[1], x.dims[2]
        hd = d // n_heads
        flat = [batch * seq, d]
        qkv = self.linear(self.reshape(x, flat), qkv_w, qkv_b)
        sq, sk, sv = (self.slice(qkv, 1, i * d, (i + 1) * d) for i in range(3))
        four = [batch, seq, n_heads, hd]
        if cos_t is not None and sin_t is not None:
            sq = self.reshape(self.rope(self.reshape(sq, four), cos_t, sin_t, grid_w, scale), flat)
            sk = self.reshape(self.rope(self.reshape(sk, four), cos_t, sin_t, grid_w, scale), flat)
        q4, k4, v4 = (self.permute(self.reshape(t, four), (0, 2, 1, 3)) for t in (sq, sk, sv))
        attn = self.permute(self.sdpa(q4, k4, v4, mask, hd), (0, 2, 1, 3))
        return self.linear(self.reshape(attn, flat), out_w, out_b)


def vit_block(G, x, p, n_heads, grid, window, is_global, cos_t, sin_t):
    """One ViT block of image_encoder.c:755-916 on x [np, e]:
    LN -> (window partition) -> MHA with RoPE -> (unpartition) -> + x ->
    LN -> MLP -> + x. p: dict of weight tensors ln1_w, ln1_b, qkv_w, qkv_b,
    proj_w, proj_b, ln2_w, ln2_b, fc1_w, fc1_b, fc2_w, fc2_b."""
    npos, e = x.dims[0], x.dims[1]
    xn = G.layernorm(x, p["ln1_w"], p["ln1_b"])
    if is_global:
        attn = G.mha_rope(G.reshape(xn, [1, npos, e]), p["qkv_w"], p["qkv_b"], p["proj_w"],
                          p["proj_b"], n_heads, cos_t, sin_t, grid, window / grid)
    else:
        xw = G.window_partition(xn, window, grid)
        aw = G.mha_rope(xw, p["qkv_w"], p["qkv_b"], p["proj_w"], p["proj_b"], n_heads,
                        cos_t, sin_t, window, 1.0)
        nw = grid // window
        aw = G.reshape(aw, [nw * nw, window * window, e])
        attn = G.window_unpartition(aw, window, grid)
    x = G.add(x, attn)
    ff = G.mlp(G.layernorm(x, p["ln2_w"], p["ln2_b"]), p["fc1_w"], p["fc1_b"], p["fc2_w"],
               p["fc2_b"])
    return G.add(x, ff)


def text_layer(G, x, p, n_heads, mask):
    """One text-encoder layer as text_encoder.c:588-652 builds it, on x
    [seq, width]: LN -> MHA (fused QKV, causal mask, no RoPE) -> + x ->
    LN -> MLP (GELU) -> + x. p: dict of weight tensors ln1_w, ln1_b,
    qkv_w, qkv_b, proj_w, proj_b, ln2_w, ln2_b, fc1_w, fc1_b, fc2_w, fc2_b."""
    seq, w = x.dims[0], x.dims[1]
    xn = G.reshape(G.layernorm(x, p["ln1_w"], p["ln1_b"]), [1, seq, w])
    attn = G.mha_rope(xn, p["qkv_w"], p["qkv_b"], p["proj_w"], p["proj_b"], n_heads,
                      None, None, 0, 0.0, mask)
    x = G.add(x, attn)
    ff = G.mlp(G.layernorm(x, p["ln2_w"], p["ln2_b"]), p["fc1_w"], p["fc1_b"], p["fc2_w"],
               p["fc2_b"])
    return G.add(x, ff)


def causal_mask(seq):
    """The text encoder's additive causal mask (text_encoder.c:552-557):
    -1e9 above the diagonal, 0 elsewhere."""
    c = np.arange(seq)
    return np.where(c[None, :] > c[:, None], np.float32(-1e9), np.float32(0.0)).astype(np.float32)


# Block parameter -> checkpoint tensor name, as sam3_vit_load looks them up
# (image_encoder.c:344-420); q/k/v are stored separately and fused at load.
VIT_PREFIX = "detector_model.vision_encoder.backbone."
VIT_NAMES = {
    "ln1_w": "layers.{}.layer_norm1.weight", "ln1_b": "layers.{}.layer_norm1.bias",
    "q_w": "layers.{}.attention.q_proj.weight", "k_w": "layers.{}.attention.k_proj.weight",
    "v_w": "layers.{}.attention.v_proj.weight", "q_b": "layers.{}.attention.q_proj.bias",
    "k_b": "layers.{}.attention.k_proj.bias", "v_b": "layers.{}.attention.v_proj.bias",
    "proj_w": "layers.{}.attention.o_proj.weight", "proj_b": "layers.{}.attention.o_proj.bias",
    "ln2_w": "layers.{}.layer_norm2.weight", "ln2_b": "layers.{}.layer_norm2.bias",
    "fc1_w": "layers.{}.mlp.fc1.weight", "fc1_b": "layers.{}.mlp.fc1.bias",
    "fc2_w": "layers.{}.mlp.fc2.weight", "fc2_b": "layers.{}.mlp.fc2.bias",
}
_LINEAR = ("q_w", "k_w", "v_w", "proj_w", "fc1_w", "fc2_w")


def vit_layer_entries(layer, e, mlp, seed, quantize=None):
    """Checkpoint entries (name, dtype, dims, array) of one synthetic ViT
    layer in the file layout: weights [out, in], q/k/v separate. With
    `quantize` (f32 array -> Q8_0 block bytes) the six linear weights are
    Q8_0 and everything else stays F32."""
    from . import synth
    shapes = {"ln1_w": (e,), "ln1_b": (e,), "q_w": (e, e), "k_w": (e, e), "v_w": (e, e),
              "q_b": (e,), "k_b": (e,), "v_b": (e,), "proj_w": (e, e), "proj_b": (e,),
              "ln2_w": (e,), "ln2_b": (e,), "fc1_w": (mlp, e), "fc1_b": (mlp,),
              "fc2_w": (e, mlp), "fc2_b": (e,)}
    std = {"ln1_w": 1.0, "ln2_w": 1.0, "ln1_b": 0.1, "ln2_b": 0.1}
    out = []
    for j, (key, shape) in enumerate(shapes.items()):
        v = synth.randn(seed + j, shape, std.get(key, 0.05 if key in _LINEAR else 0.02))
        name = VIT_PREFIX + VIT_NAMES[key].format(layer)
        if quantize is not None and key in _LINEAR:
            out.append((name, abi.Q8_0, list(shape), np.asarray(quantize(v), np.uint8)))
        else:
            out.append((name, abi.F32, list(shape), v))
    return out


def load_vit_layer(G, wf, layer, be=None):
    """The per-layer part of sam3_vit_load (image_encoder.c:344-420) over
    a `weights.WeightFile`: one tensor per parameter pointing into the
    mapping, with q/k/v (weights and biases) stacked into qkv_w [3e, e]
    and qkv_b [3e]. With a backend the stacking is
    `sam3_hip_backend_fuse_rows` (in HBM, any dtype); without one it is a
    host byte concatenation that keeps the parts' dtype."""
    def get(key):
        i = wf.find(VIT_PREFIX + VIT_NAMES[key].format(layer))
        if i is None:
            raise KeyError(VIT_NAMES[key].format(layer))
        t = wf.to_tensor(i)
        G.keep.append(t)
        return t

    def fuse(keys):
        parts = [get(k) for k in keys]
        out = abi.Tensor()
        if be is not None:
            from . import hip
            hip.check(be.fuse_rows(parts, out), "fuse_rows")
        else:
            raw = np.concatenate([wf.array(wf.find(VIT_PREFIX + VIT_NAMES[k].format(layer)))
                                  for k in keys])
            dims = [sum(p.dims[0] for p in parts)] + ([parts[0].dims[1]]
                                                      if parts[0].n_dims == 2 else [])
            G.keep.append(raw)
            out = abi.make_tensor(parts[0].dtype, dims, raw.ctypes.data, raw.nbytes)
        G.keep.append(out)
        return out

    p = {k: get(k) for k in ("ln1_w", "ln1_b", "proj_w", "proj_b", "ln2_w", "ln2_b", "fc1_w",
                             "fc1_b", "fc2_w", "fc2_b")}
    p["qkv_w"] = fuse(("q_w", "k_w", "v_w"))
    p["qkv_b"] = fuse(("q_b", "k_b", "v_b"))
    return p


def rope_tables(seq_side, hd, theta=10000.0):
    """2-D axial RoPE tables [seq_side^2, hd/2] (x then y frequencies),
    f32: synthetic stand-ins of the checkpoint's precomputed tables."""
    quarter = hd // 4
    freqs = 1.0 / (theta ** (np.arange(quarter) / quarter))
    ys, xs = np.meshgrid(np.arange(seq_side), np.arange(seq_side), indexing="ij")
    ang = np.concatenate([np.outer(xs.ravel(), freqs), np.outer(ys.ravel(), freqs)], axis=1)
    return np.cos(ang).astype(np.float32), np.sin(ang).astype(np.float32)

