#!/usr/bin/env python3
"""Benchmark of the MI355X matmul backend for sam3.c (one GPU).

Headline (the JSON line's `value`): BASELINE.json configs[1], the bf16
ViT-L MLP fc1 GEMM C[5184,4096] = A[5184,1024] * W[4096,1024]^T with f32
accumulation, in TFLOP/s (2*M*N*K per step), inputs resident in HBM. One
step = one GEMM launch. The other BASELINE configs are measured too and
reported under "extra":
  config 1  Q8 matmul, f32 activations, 5184x1024x1024
  config 2  bf16/f16 fc1 and fc2, plain and with fused bias+GELU
  config 3  32 ViT-L layers x {qkv, proj, fc1, fc2}, Q8 weights (distinct
            per layer, 453 MB streamed from HBM), bf16 activations
  config 4  skinny Q8 GEMVs (M in {1,8,32,77}) over a pool of >256 MB of
            distinct weight copies, reported in HBM GB/s per launch (HIP graph
            of one launch per copy) and for one batched launch
  config 5  batched attention QK^T / PV, windowed (1296 x 576 x 64), and
            the fused SDPA kernel (windowed 1296 x 576, global 16 x 5184;
            bf16, f16, f32)
`roofline` is for the headline kernel; `cpu_baseline` times the reference
CPU bf16 kernel (oracle/_ref, compiled from the reference's own sources)
on the GPU box's host cores over a bounded row sample of the same GEMM.
"q8" is the same kind of record for the Q8_0 path on config 3's fc1
layer (bf16 activations x Q8_0 W[4096,1024], f32 out): its own value,
roofline (f16 MFMA peak, with the f16 GEMM timed on its own as the
dominant kernel) and the reference's Q8_0 CPU kernel as cpu_baseline.

  python bench.py [--gpus 1] [--steps K] [--warmup W] [--quick]
"""
import argparse
import json
import os
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT / "sam3.c_amd"))
sys.path.insert(0, str(ROOT / "tests"))

from sam3_amd import abi, hip, synth  # noqa: E402

PEAK_BF16_TFLOPS = 2500.0   # MI355X dense bf16/f16 MFMA
PEAK_HBM_GBS = 8000.0       # MI355X HBM3E
PEAK_PCIE_GBS = 64.0        # host link, PCIe 5.0 x16, one direction


def log(*a):
    print("[bench]", *a, file=sys.stderr, flush=True)


def bf16_bits(x):
    u = np.ascontiguousarray(x, np.float32).view(np.uint32).astype(np.uint64)
    r = (u + 0x7FFF + ((u >> 16) & 1)) >> 16
    return r.astype(np.uint16)


def f16_bits(x):
    return np.ascontiguousarray(x, np.float32).astype(np.float16).view(np.uint16)


class Timer:
    """HIP events on the stream the kernels are launched on."""

    def __init__(self, stream):
        self.stream = stream
        self.e0, self.e1 = hip.Event(), hip.Event()

    def run(self, fn, steps, warmup, settle_s=0.0):
        """Mean ms per call of fn over `steps` timed calls, after `warmup`
        untimed ones. settle_s > 0 first runs fn untimed for that many
        seconds, so that a GPU coming out of idle reaches its working
        clock before the warmup steps."""
        if settle_s > 0:
            t_end = time.perf_counter() + settle_s
            while time.perf_counter() < t_end:
                for _ in range(20):
                    fn()
                hip.check(hip.load().sam3_hip_stream_synchronize(self.stream), "sync")
        for _ in range(warmup):
            fn()
        hip.check(hip.load().sam3_hip_stream_synchronize(self.stream), "sync")
        self.e0.record(self.stream)
        for _ in range(steps):
            fn()
        self.e1.record(self.stream)
        hip.check(hip.load().sam3_hip_stream_synchronize(self.stream), "sync")
        return self.e0.elapsed_ms(self.e1) / steps


def gemm_case(stream, timer, a_dt, a, b_dt, b, c_dt, M, N, K, flags, steps, warmup, bias=None,
              settle_s=0.0):
    da, db = hip.DeviceBuffer.of(a), hip.DeviceBuffer.of(b)
    dc = hip.DeviceBuffer(M * N * (4 if c_dt == abi.F32 else 2))
    dbias = hip.DeviceBuffer.of(bias) if bias is not None else None
    bp = dbias.ptr if dbias else None

    def step():
        hip.matmul_dev(a_dt, da.ptr, b_dt, db.ptr, c_dt, dc.ptr, M, N, K, bp, flags, stream)

    ms = timer.run(step, steps, warmup, settle_s)
    for buf in (da, db, dc, dbias):
        if buf:
            buf.free()
    return ms


def tflops(M, N, K, ms):
    return 2.0 * M * N * K / (ms * 1e-3) / 1e12


def cpu_baseline(a_bits, w_bits, M, N, K, target_s=10.0):
    """Reference CPU bf16 kernel (cpu_kernel_matmul_bf16 via oracle/_ref, B
    as [K,N] per its contract) on all allowed host cores, on a row sample
    of the headline GEMM sized to ~target_s seconds."""
    from oracle_bind import Oracle, Ref, have_ref
    threads = int(os.environ.get("OMP_NUM_THREADS") or os.cpu_count() or 1)
    threads = max(1, min(threads, os.cpu_count() or 1))
    b_kn = np.ascontiguousarray(w_bits.T)
    if have_ref():
        R, kind = Ref(), "reference"
        fn = lambda a: R.matmul_bf16(a, b_kn, threads)  # noqa: E731
    else:
        R, kind = Oracle(), "port"
        fn = lambda a: R.matmul_bf16(a, b_kn, threads)  # noqa: E731
    probe = max(threads, 32)
    t0 = time.perf_counter()
    fn(a_bits[:probe])
    per_row = (time.perf_counter() - t0) / probe
    rows = int(min(M, max(probe, target_s / max(per_row, 1e-9))))
    rows -= rows % threads if rows > threads else 0
    t0 = time.perf_counter()
    fn(a_bits[:rows])
    dt = time.perf_counter() - t0
    if kind == "reference":
        R.close()
    model = ""
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    return {"value": round(tflops(rows, N, K, dt * 1e3), 6), "unit": "TFLOP/s", "cores": threads,
            "kind": kind,
            "sample": f"bf16 GEMM rows 0..{rows - 1} of {M} (x {N}x{K}), one call, "
                      f"{dt:.2f} s, cpu_kernel_matmul_bf16 with a {threads}-thread pool"
                      + (f", {model}" if model else "")}


def cpu_sdpa(BH, S, D, target_s=4.0):
    """The reference's f32 SDPA (cpu_kernel_sdpa via oracle/_ref, or the
    restatement) on the host cores, over a sample of the heads (and, for
    long sequences, of the queries) of a BH x S x S problem, sized to about
    target_s seconds; returned as TFLOP/s of 4*S*D flops per (query, key)."""
    from oracle_bind import Oracle, Ref, have_ref
    threads = int(os.environ.get("OMP_NUM_THREADS") or os.cpu_count() or 1)
    threads = max(1, min(threads, os.cpu_count() or 1))
    R, kind = (Ref(), "reference") if have_ref() else (Oracle(), "port")
    k = synth.randn(synth.tensor_seed(7, 1), (1, S, D)) / 4
    v = synth.randn(synth.tensor_seed(7, 2), (1, S, D))
    q = synth.randn(synth.tensor_seed(7, 0), (1, S, D)) / 4
    probe = min(S, 64)
    t0 = time.perf_counter()
    R.sdpa(q[:, :probe], k, v, None, threads)
    per_q = (time.perf_counter() - t0) / probe
    nq = int(max(probe, min(BH * S, target_s / max(per_q, 1e-9))))
    heads, rows = (max(1, nq // S), S) if nq >= S else (1, nq)
    qs = np.ascontiguousarray(np.broadcast_to(q[:, :rows], (heads, rows, D)))
    ks = np.ascontiguousarray(np.broadcast_to(k, (heads, S, D)))
    vs = np.ascontiguousarray(np.broadcast_to(v, (heads, S, D)))
    t0 = time.perf_counter()
    R.sdpa(qs, ks, vs, None, threads)
    dt = time.perf_counter() - t0
    if kind == "reference":
        R.close()
    return {"value": round(4.0 * heads * rows * S * D / dt / 1e12, 6), "unit": "TFLOP/s",
            "cores": threads, "kind": kind,
            "sample": f"f32 SDPA, {heads} head(s) x {rows} queries x {S} keys, D={D}, "
                      f"{dt:.2f} s, cpu_kernel_sdpa with a {threads}-thread pool"}


def vit_block_flops(npos, e, heads, mlp, seq):
    """GEMM flops of a ViT-L block (qkv, proj, fc1, fc2) plus attention's
    4*S^2*D per head over npos/seq windows."""
    gemm = 2.0 * npos * e * (3 * e + e + 2 * mlp)
    return gemm + 4.0 * (npos // seq) * heads * seq * seq * (e // heads)


def vit_block_graph(grid, window, e, heads, mlp, is_global, wkind, x_dev=None, seed=500):
    """One ViT-L block as image_encoder.c:755-916 builds it (sam3_amd.graph),
    f32 activations, weights f32 or Q8_0 (quantized on the device) in the
    checkpoint layout [out, in]; x on the device when x_dev is given."""
    from sam3_amd import graph
    G = graph.Graph()
    npos = grid * grid
    if x_dev is not None:
        x = abi.make_tensor(abi.F32, [npos, e], x_dev, npos * e * 4)
        G.keep.append(x)
    else:
        x = G.tensor(abi.F32, (npos, e), synth.randn(seed, (npos, e)), ephemeral=1)

    def w(i, shape, std, quant=False):
        v = synth.randn(seed + i, shape, std)
        if quant and wkind == "q8":
            return G.tensor(abi.Q8_0, shape, hip.q8_quantize(v))
        return G.tensor(abi.F32, shape, v)
    p = {"ln1_w": w(1, (e,), 1.0), "ln1_b": w(2, (e,), 0.1),
         "qkv_w": w(3, (3 * e, e), 0.03, True), "qkv_b": w(4, (3 * e,), 0.02),
         "proj_w": w(5, (e, e), 0.03, True), "proj_b": w(6, (e,), 0.02),
         "ln2_w": w(7, (e,), 1.0), "ln2_b": w(8, (e,), 0.1),
         "fc1_w": w(9, (mlp, e), 0.03, True), "fc1_b": w(10, (mlp,), 0.02),
         "fc2_w": w(11, (e, mlp), 0.03, True), "fc2_b": w(12, (e,), 0.02)}
    c, s_ = graph.rope_tables(grid if is_global else window, e // heads)
    tc, ts = G.tensor(abi.F32, c.shape, c), G.tensor(abi.F32, s_.shape, s_)
    out = graph.vit_block(G, x, p, heads, grid, window, is_global, tc, ts)
    return G, out


def vit_block_bench(is_global, wkind, steps=5, warmup=2):
    """A full ViT-L block (72x72 tokens, e 1024, 16 heads, MLP 4096, window
    24) through the backend's graph_eval with the block input in HBM and
    no readback: the latency a sam3.c caller of the vtable sees, weights
    resident after the first eval."""
    grid, window, e, heads, mlp = 72, 24, 1024, 16, 4096
    npos = grid * grid
    xd = hip.DeviceBuffer.of(synth.randn(500, (npos, e)))
    G, _ = vit_block_graph(grid, window, e, heads, mlp, is_global, wkind, xd.ptr)
    G.g.no_readback = True
    be = hip.Backend(0)
    try:
        for _ in range(warmup):
            hip.check(be.graph_eval(G.g), "graph_eval")
        t0 = time.perf_counter()
        for _ in range(steps):
            hip.check(be.graph_eval(G.g), "graph_eval")
        ms = (time.perf_counter() - t0) * 1e3 / steps
        st = be.stats()
    finally:
        be.close()
        xd.free()
    fl = vit_block_flops(npos, e, heads, mlp, npos if is_global else window * window)
    return {"ms": round(ms, 3), "tokens_per_s": round(npos / (ms * 1e-3), 1),
            "tflops": round(fl / (ms * 1e-3) / 1e12, 1), "nodes": G.g.n_nodes,
            "gpu_nodes": st.gpu_nodes, "fused_nodes": st.fused_nodes, "host_nodes": st.host_nodes,
            "range_reruns": st.range_reruns}


def vit_trunk_bench(wkind, depth=32, per_graph=4, steps=3, warmup=1):
    """The ViT-L trunk (image_encoder.c:736-915): `depth` blocks, global
    attention at blocks 7, 15, 23, 31 (image_encoder.c:35), evaluated
    `per_graph` blocks per graph_eval as the reference's block loop does,
    each graph's output forwarded on the device to the next graph
    (no_readback on all but the last). One layer's weights are shared by
    every block (the time does not depend on their values). Wall time of
    the whole trunk, block input in HBM."""
    from sam3_amd import graph
    grid, window, e, heads, mlp = 72, 24, 1024, 16, 4096
    npos = grid * grid
    xd = hip.DeviceBuffer.of(synth.randn(500, (npos, e)))
    W = graph.Graph()

    def w(i, shape, std, quant=False):
        v = synth.randn(520 + i, shape, std)
        if quant and wkind == "q8":
            return W.tensor(abi.Q8_0, shape, hip.q8_quantize(v))
        return W.tensor(abi.F32, shape, v)
    p = {"ln1_w": w(1, (e,), 1.0), "ln1_b": w(2, (e,), 0.1),
         "qkv_w": w(3, (3 * e, e), 0.03, True), "qkv_b": w(4, (3 * e,), 0.02),
         "proj_w": w(5, (e, e), 0.03, True), "proj_b": w(6, (e,), 0.02),
         "ln2_w": w(7, (e,), 1.0), "ln2_b": w(8, (e,), 0.1),
         "fc1_w": w(9, (mlp, e), 0.03, True), "fc1_b": w(10, (mlp,), 0.02),
         "fc2_w": w(11, (e, mlp), 0.03, True), "fc2_b": w(12, (e,), 0.02)}
    tabs = {}
    for side in (window, grid):
        c, s_ = graph.rope_tables(side, e // heads)
        tabs[side] = (W.tensor(abi.F32, c.shape, c), W.tensor(abi.F32, s_.shape, s_))
    graphs, x = [], abi.make_tensor(abi.F32, [npos, e], xd.ptr, npos * e * 4)
    W.keep.append(x)
    for base in range(0, depth, per_graph):
        G = graph.Graph()
        G.keep.append(W)
        for i in range(base, min(depth, base + per_graph)):
            glob = i in (7, 15, 23, 31)
            tc, ts = tabs[grid if glob else window]
            x = graph.vit_block(G, x, p, heads, grid, window, glob, tc, ts)
        G.g.no_readback = True
        graphs.append(G)
    be = hip.Backend(0)
    try:
        def run():
            for G in graphs:
                hip.check(be.graph_eval(G.g), "graph_eval")
        for _ in range(warmup):
            run()
        t0 = time.perf_counter()
        for _ in range(steps):
            run()
        ms = (time.perf_counter() - t0) * 1e3 / steps
        st = be.stats()
    finally:
        be.close()
        xd.free()
    fl = 28 * vit_block_flops(npos, e, heads, mlp, window * window) + \
        4 * vit_block_flops(npos, e, heads, mlp, npos)
    return {"ms": round(ms, 2), "images_per_s": round(1e3 / ms, 2), "blocks": depth,
            "graph_evals": len(graphs), "tflops": round(fl / (ms * 1e-3) / 1e12, 1),
            "last_eval_host_nodes": st.host_nodes}


def text_encoder_bench(seqs=(1, 8, 32, 77), layers=24, per_graph=4, steps=3, warmup=1):
    """BASELINE config 4's shapes as a dependent chain: the text encoder's
    24 layers (text_encoder.c:559-660: width 1024, 16 heads, MLP 4096,
    causal mask) with distinct Q8_0 linear weights per layer (254 MB, as
    much as the MALL holds), evaluated 4 layers per graph_eval as the
    reference's block loop does, x forwarded on the device between evals,
    for seq in `seqs`. Reports the wall time of all 24 layers and the
    weight bytes streamed per second."""
    from sam3_amd import graph
    w_, heads, mlp = 1024, 16, 4096
    shapes = {"qkv_w": (3 * w_, w_), "proj_w": (w_, w_), "fc1_w": (mlp, w_), "fc2_w": (w_, mlp)}
    base = {k: hip.q8_quantize(synth.randn(900 + i, sh, 0.02)) for i, (k, sh) in enumerate(shapes.items())}
    W = graph.Graph()
    params = []
    wbytes = 0
    for li in range(layers):
        p = {}
        for k, sh in shapes.items():
            blk = base[k].copy()
            blk[4::36] ^= np.uint8(li)  # distinct bytes per layer (a q value of each block)
            p[k] = W.tensor(abi.Q8_0, sh, blk)
            wbytes += blk.nbytes
        for k, n in (("qkv_b", 3 * w_), ("proj_b", w_), ("fc1_b", mlp), ("fc2_b", w_)):
            p[k] = W.tensor(abi.F32, (n,), synth.randn(950 + li, (n,), 0.02))
        for k in ("ln1", "ln2"):
            p[k + "_w"] = W.tensor(abi.F32, (w_,), synth.randn(960 + li, (w_,), 1.0))
            p[k + "_b"] = W.tensor(abi.F32, (w_,), synth.randn(970 + li, (w_,), 0.1))
        params.append(p)
    out = {}
    for seq in seqs:
        xd = hip.DeviceBuffer.of(synth.randn(980 + seq, (seq, w_)))
        mask = W.tensor(abi.F32, (seq, seq), graph.causal_mask(seq))
        graphs, x = [], abi.make_tensor(abi.F32, [seq, w_], xd.ptr, seq * w_ * 4)
        W.keep.append(x)
        for b0 in range(0, layers, per_graph):
            G = graph.Graph()
            G.keep.append(W)
            for li in range(b0, min(layers, b0 + per_graph)):
                x = graph.text_layer(G, x, params[li], heads, mask)
            G.g.no_readback = True
            graphs.append(G)
        be = hip.Backend(0)
        try:
            def run():
                for G in graphs:
                    hip.check(be.graph_eval(G.g), "graph_eval")
            for _ in range(warmup):
                run()
            t0 = time.perf_counter()
            for _ in range(steps):
                run()
            ms = (time.perf_counter() - t0) * 1e3 / steps
            st = be.stats()
        finally:
            be.close()
            xd.free()
        gbs = wbytes / (ms * 1e-3) / 1e9
        out[f"seq{seq}"] = {"ms": round(ms, 3), "us_per_layer": round(ms * 1e3 / layers, 1),
                            "weights_gbs": round(gbs, 1), "frac_hbm": round(gbs / PEAK_HBM_GBS, 4),
                            "gpu_nodes_per_eval": st.gpu_nodes, "fused_nodes_per_eval": st.fused_nodes,
                            "range_reruns": st.range_reruns,
                            "nodes_per_eval": graphs[0].g.n_nodes}
        log(f"  seq {seq}: {out[f'seq{seq}']}")
    out["note"] = (f"{layers} layers, {per_graph} per graph_eval, Q8_0 weights "
                   f"{wbytes / 1e6:.0f} MB in all (distinct per layer), f32 activations; weights_gbs = "
                   "weight bytes / wall time of all layers")
    return out


def vit_block_cpu(threads=None):
    """The reference's CPU kernels (cpu_dispatch_node over the same node
    sequence, oracle/_ref) on one 24x24 window of the block (576 tokens,
    full width): a bounded sample, reported in tokens/s."""
    sys.path.insert(0, str(ROOT / "tests"))
    from oracle_bind import Ref, have_ref
    from test_gpu_blockops import reference_eval
    if not have_ref():
        return None
    threads = threads or max(1, min(int(os.environ.get("OMP_NUM_THREADS") or os.cpu_count() or 1),
                                    os.cpu_count() or 1))
    G, _ = vit_block_graph(24, 24, 1024, 16, 4096, False, "f32")
    R = Ref()
    t0 = time.perf_counter()
    rc = reference_eval(R, G.g, R.pool(threads))
    dt = time.perf_counter() - t0
    R.close()
    if rc != 0:
        return None
    return {"value": round(576 / dt, 1), "unit": "tokens/s", "cores": threads, "kind": "reference",
            "sample": f"one 24x24 window (576 tokens) of a windowed ViT-L block, f32 weights, "
                      f"{dt:.2f} s, cpu_dispatch_node over the same node sequence with a "
                      f"{threads}-thread pool"}


def weights_upload_bench(layers=32, e=1024, mlp=4096):
    """A .sam3 checkpoint of `layers` ViT-L layers (Q8_0 linear weights as
    in config 3, f32 norms and biases; q/k/v stored separately) written to
    a temporary file, mmap'd, and its data blob copied to HBM by
    sam3_hip_backend_map_weights. Beside it: the per-tensor pageable
    copies graph_eval makes for weights that are not mapped (one hipMemcpy
    per tensor into a preallocated buffer, so no allocation is timed), and
    the QKV stacking of every layer (fuse_rows, in HBM)."""
    import tempfile
    from sam3_amd import graph
    from sam3_amd import weights as W
    one = graph.vit_layer_entries(0, e, mlp, 700, hip.q8_quantize)
    ents = []
    for i in range(layers):
        for name, dt, dims, arr in one:
            ents.append((name.replace("layers.0.", f"layers.{i}."), dt, dims, arr))
    fd, path = tempfile.mkstemp(suffix=".sam3")
    os.close(fd)
    lib = hip.load()
    try:
        W.write(path, ents)
        wf = W.WeightFile(path)
        nbytes = wf.data_size
        be = hip.Backend(0)
        t0 = time.perf_counter()
        hip.check(be.map_weights(wf.data_base, nbytes), "map_weights")
        t_first = time.perf_counter() - t0
        be.cache_invalidate(wf.data_base, nbytes)
        ts = []
        for _ in range(3):
            t0 = time.perf_counter()
            hip.check(be.map_weights(wf.data_base, nbytes), "map_weights")
            ts.append(time.perf_counter() - t0)
            if len(ts) < 3:
                be.cache_invalidate(wf.data_base, nbytes)
        t_map = min(ts)
        t0 = time.perf_counter()
        fused = 0
        for i in range(layers):
            G = graph.Graph()
            graph.load_vit_layer(G, wf, i, be)
            fused += 2
        t_fuse = time.perf_counter() - t0
        be.close()
        dev = hip.DeviceBuffer(nbytes)
        hip.synchronize()
        t0 = time.perf_counter()
        for i in range(wf.n_tensors):
            d = wf.descs[i]
            off = int(d["data_offset"])
            hip.check(lib.sam3_hip_memcpy_h2d(dev.ptr + off, wf.data_base + off,
                                              int(d["data_size"])), "memcpy_h2d")
        hip.synchronize()
        t_tensor = time.perf_counter() - t0
        dev.free()
        n_t = wf.n_tensors
        wf.close()
    finally:
        os.remove(path)
    gbs = nbytes / t_map / 1e9
    return {"bytes": nbytes, "tensors": n_t, "layers": layers,
            "map_weights_ms": round(t_map * 1e3, 2), "map_weights_gbs": round(gbs, 2),
            "first_map_ms": round(t_first * 1e3, 2),
            "per_tensor_pageable_ms": round(t_tensor * 1e3, 2),
            "per_tensor_pageable_gbs": round(nbytes / t_tensor / 1e9, 2),
            "fuse_qkv_ms_per_layer": round(t_fuse * 1e3 / layers, 3),
            "roofline": {"bound": "pcie", "achieved": round(gbs, 2), "peak": PEAK_PCIE_GBS,
                         "unit": "GB/s", "frac": round(gbs / PEAK_PCIE_GBS, 4)},
            "note": "file in the page cache; first_map includes the pinned staging "
                    "allocation and the first touch of the mapping"}


# name: (x [N,H,W,C], w [OC,KH,KW,C], stride, pad) -- the patch embedding
# (image_encoder.c:577) and the neck's convs at the 1x and 4x scales
# (necks.c:345-365)
CONV_SHAPES = {
    "patch_embed": ((1, 1008, 1008, 3), (1024, 14, 14, 3), 14, 0),
    "neck_1x1_72": ((1, 72, 72, 1024), (256, 1, 1, 1024), 1, 0),
    "neck_3x3_72": ((1, 72, 72, 256), (256, 3, 3, 256), 1, 1),
    "neck_3x3_288": ((1, 288, 288, 256), (256, 3, 3, 256), 1, 1),
}


def conv_case(lib, stream, timer, kind, xs, ws, stride, pad, steps, warmup):
    """One CONV2D node (sam3_hip_kernel_conv2d) on device buffers, timed."""
    dt, npt = {"f32": (abi.F32, np.float32), "bf16": (abi.BF16, np.uint16)}[kind]
    x = synth.randn(600, xs)
    w = synth.randn(601, ws, 0.02)
    if kind == "bf16":
        x, w = bf16_bits(x), bf16_bits(w)
    N, H, W, C = xs
    OC, KH, KW, _ = ws
    OH, OW = (H + 2 * pad - KH) // stride + 1, (W + 2 * pad - KW) // stride + 1
    bx, bw = hip.DeviceBuffer.of(x), hip.DeviceBuffer.of(w)
    by = hip.DeviceBuffer(N * OH * OW * OC * np.dtype(npt).itemsize)
    tx = abi.make_tensor(dt, list(xs), bx.ptr, x.nbytes)
    tw = abi.make_tensor(dt, list(ws), bw.ptr, w.nbytes)
    ty = abi.make_tensor(dt, [N, OH, OW, OC], by.ptr, by.nbytes)
    node = abi.make_node(abi.OP_CONV2D, [tx, tw], ty, (stride, pad, 1, 0))
    path = lib.sam3_hip_conv2d_path(hip.C.byref(node))

    def step():
        hip.check(lib.sam3_hip_kernel_conv2d(hip.C.byref(node), stream), "conv2d")

    ms = timer.run(step, steps, warmup)
    for b in (bx, bw, by):
        b.free()
    M, K = N * OH * OW, KH * KW * C
    return {"us": round(ms * 1e3, 1), "tflops": round(tflops(M, OC, K, ms), 1),
            "path": {1: "implicit_gemm", 2: "im2col_gemm", 3: "direct"}.get(path, path)}


def cpu_conv(name, threads=None, target_s=3.0):
    """The reference's f32 conv (cpu_kernel_conv2d via oracle/_ref, or the
    restatement) on the host cores, on a crop of the input rows sized to a
    few seconds; TFLOP/s of 2*M*OC*K."""
    from oracle_bind import Oracle, Ref, have_ref
    threads = threads or max(1, min(int(os.environ.get("OMP_NUM_THREADS") or os.cpu_count() or 1),
                                    os.cpu_count() or 1))
    xs, ws, stride, pad = CONV_SHAPES[name]
    N, H, W, C = xs
    OC, KH, KW, _ = ws
    # probe on a few rows, then as many rows as fit in about target_s
    rows = min(H, max(KH, 4 * stride))
    R0 = Ref() if have_ref() else Oracle()
    t0 = time.perf_counter()
    if have_ref():
        R0.conv2d(synth.randn(602, (N, rows, W, C)), synth.randn(603, ws, 0.02), stride, pad, None,
                  1, "f32", None, threads)
        R0.close()
    else:
        R0.conv2d(synth.randn(602, (N, rows, W, C)), synth.randn(603, ws, 0.02), stride, pad,
                  threads=threads)
    per_row = (time.perf_counter() - t0) / rows
    rows = int(min(H, max(rows, target_s / max(per_row, 1e-9))))
    rows -= rows % stride
    x = synth.randn(602, (N, rows, W, C))
    w = synth.randn(603, ws, 0.02)
    R, kind = (Ref(), "reference") if have_ref() else (Oracle(), "port")
    t0 = time.perf_counter()
    if kind == "reference":
        rc, y = R.conv2d(x, w, stride, pad, None, 1, "f32", None, threads)
        R.close()
    else:
        y = R.conv2d(x, w, stride, pad, threads=threads)
    dt = time.perf_counter() - t0
    M = y.shape[0] * y.shape[1] * y.shape[2]
    return {"value": round(2.0 * M * OC * KH * KW * C / dt / 1e12, 6), "unit": "TFLOP/s",
            "cores": threads, "kind": kind,
            "sample": f"f32 {name}, {rows} of {H} input rows -> {M} output pixels, {dt:.2f} s"}


def neck_graph(x_dev, dim=1024, d=256, grid=72, seed=640):
    """The FPN neck of necks.c:30-140 on the trunk's [1, grid, grid, dim]
    map, all four scales in one graph (f32, synthetic weights, biases on
    every conv): 4x ConvT(dim->dim/2)+GELU, ConvT(dim/2->dim/4), 1x1, 3x3;
    2x ConvT(dim->dim/2), 1x1, 3x3; 1x 1x1, 3x3; 0.5x MaxPool 2/2, 1x1, 3x3.
    Returns the graph, its outputs and its flop count."""
    from sam3_amd import graph
    G = graph.Graph()
    F = abi.F32
    x = abi.make_tensor(F, [1, grid, grid, dim], x_dev, grid * grid * dim * 4)
    G.keep.append(x)
    k = [seed]
    flops = [0.0]

    def conv(t, oc, ksz, transpose=False, gelu=False):
        _, h, w, c = (t.dims[i] for i in range(4))
        k[0] += 2
        wt = G.tensor(F, (oc, ksz, ksz, c), synth.randn(k[0], (oc, ksz, ksz, c), 0.02))
        b = G.tensor(F, (oc,), synth.randn(k[0] + 1, (oc,), 0.02))
        if transpose:
            oh, ow = h * 2, w * 2
            t = G.node(abi.OP_CONV_TRANSPOSE2D, [t, wt], G.tensor(F, (1, oh, ow, oc)), (2, 0, 0, 0))
            flops[0] += 2.0 * h * w * c * oc * ksz * ksz
        else:
            oh, ow = h, w
            t = G.node(abi.OP_CONV2D, [t, wt], G.tensor(F, (1, oh, ow, oc)), (1, ksz // 2, 1, 0))
            flops[0] += 2.0 * oh * ow * oc * c * ksz * ksz
        t = G.node(abi.OP_BIAS_ADD, [t, b], G.tensor(F, (1, oh, ow, oc)))
        if gelu:
            t = G.node(abi.OP_GELU, [t], G.tensor(F, (1, oh, ow, oc)))
        return t

    outs = []
    t = conv(conv(x, dim // 2, 2, True, True), dim // 4, 2, True)
    outs.append(conv(conv(t, d, 1), d, 3))
    t = conv(x, dim // 2, 2, True)
    outs.append(conv(conv(t, d, 1), d, 3))
    outs.append(conv(conv(x, d, 1), d, 3))
    t = G.node(abi.OP_MAXPOOL2D, [x], G.tensor(F, (1, grid // 2, grid // 2, dim)), (2, 2, 0, 0))
    outs.append(conv(conv(t, d, 1), d, 3))
    return G, outs, flops[0]


def neck_bench(steps=10, warmup=2):
    """The four-scale neck through graph_eval: input map in HBM, outputs
    kept in HBM (no_readback), f32 weights prepared once."""
    xd = hip.DeviceBuffer.of(synth.randn(630, (1, 72, 72, 1024)))
    G, outs, fl = neck_graph(xd.ptr)
    G.g.no_readback = True
    be = hip.Backend(0)
    try:
        for _ in range(warmup):
            hip.check(be.graph_eval(G.g), "graph_eval")
        t0 = time.perf_counter()
        for _ in range(steps):
            hip.check(be.graph_eval(G.g), "graph_eval")
        ms = (time.perf_counter() - t0) * 1e3 / steps
        st = be.stats()
    finally:
        be.close()
        xd.free()
    return {"ms": round(ms, 3), "tflops": round(fl / (ms * 1e-3) / 1e12, 1),
            "gflop": round(fl / 1e9, 1), "nodes": G.g.n_nodes, "gpu_nodes": st.gpu_nodes,
            "fused_nodes": st.fused_nodes, "host_nodes": st.host_nodes,
            "range_reruns": st.range_reruns}


def measured_traffic(key):
    """HBM bytes per launch of the headline kernel, from the rocprofv3
    FETCH_SIZE / WRITE_SIZE runs recorded in profiles/traffic.json (scaled
    by a copy kernel of known size); None when not recorded."""
    try:
        rec = json.loads((ROOT / "profiles" / "traffic.json").read_text())[key]
        return int(rec["traffic_bytes"])
    except (OSError, KeyError, ValueError):
        return None


def q8_host_f16(wq, N, K):
    """f16 bits of q * scale (f32 product, rounded once) for Q8_0 blocks
    [N, K/32] x 36 bytes: the weight the per-call expansion hands the f16
    GEMM (bench plumbing, to time that GEMM on its own)."""
    blk = wq.reshape(N * K // 32, 36)
    scale = blk[:, :4].copy().view(np.float32)
    q = blk[:, 4:].view(np.int8).astype(np.float32)
    return (q * scale).reshape(N, K).astype(np.float16).view(np.uint16)


def q8_cpu_baseline(a32, N, K, target_s=10.0):
    """The reference's Q8_0 kernel (cpu_kernel_matmul_q8 via oracle/_ref: f32
    activations, Q8_0 weight [K,N] per its contract, f32 out) on all allowed
    host cores, on a row sample of the Q8 fc1 GEMM sized to ~target_s s."""
    from oracle_bind import Oracle, Ref, have_ref
    threads = int(os.environ.get("OMP_NUM_THREADS") or os.cpu_count() or 1)
    threads = max(1, min(threads, os.cpu_count() or 1))
    wkn = hip.q8_quantize(synth.randn(synth.tensor_seed(7, 1), (K, N), 0.02))
    if have_ref():
        R, kind = Ref(), "reference"
    else:
        R, kind = Oracle(), "port"
    fn = lambda a: R.matmul_q8(a, wkn, K, N, threads)  # noqa: E731
    M = a32.shape[0]
    probe = max(threads, 32)
    t0 = time.perf_counter()
    fn(a32[:probe])
    per_row = (time.perf_counter() - t0) / probe
    rows = int(min(M, max(probe, target_s / max(per_row, 1e-9))))
    rows -= rows % threads if rows > threads else 0
    t0 = time.perf_counter()
    fn(a32[:rows])
    dt = time.perf_counter() - t0
    if kind == "reference":
        R.close()
    return {"value": round(tflops(rows, N, K, dt * 1e3), 6), "unit": "TFLOP/s", "cores": threads,
            "kind": kind,
            "sample": f"Q8_0 matmul rows 0..{rows - 1} of {M} (x {N}x{K}), one call, {dt:.2f} s, "
                      f"cpu_kernel_matmul_q8 (f32 activations, W [K,N]) with a "
                      f"{threads}-thread pool"}


def q8_record(stream, timer, a_bf, w32, steps, warmup, with_cpu):
    """The Q8 line: BASELINE configs[2]'s fc1 layer GEMM, C[5184,4096] f32 =
    A[5184,1024] bf16 x W[4096,1024] Q8_0, one sam3_hip_matmul per step
    (row-scaled f16 copy of A, per-call f16 expansion of W, f16 MFMA GEMM).
    The dominant kernel, the f16 GEMM, is also timed on its own: the same
    kernel over f16 copies made beforehand."""
    M, K = a_bf.shape
    N = w32.shape[0]
    wq = hip.q8_quantize(w32)
    ms = gemm_case(stream, timer, abi.BF16, a_bf, abi.Q8_0, wq, abi.F32, M, N, K, hip.B_NT,
                   steps, warmup)
    value = tflops(M, N, K, ms)
    a16 = f16_bits((a_bf.astype(np.uint32) << 16).view(np.float32))
    w16 = q8_host_f16(wq, N, K)
    ms_g = gemm_case(stream, timer, abi.F16, a16, abi.F16, w16, abi.F32, M, N, K, hip.B_NT,
                     steps, warmup)
    g = tflops(M, N, K, ms_g)
    rec = {
        "metric": "TFLOP/s, bf16 activations x Q8_0 weights 5184x1024x4096 (ViT-L fc1), "
                  "f32 out",
        "value": round(value, 2), "unit": "TFLOP/s", "ms_per_step": round(ms, 5),
        "steps": steps, "warmup": warmup, "dtype": "f16 MFMA (bf16 A and Q8_0 W rounded to f16 "
                                                     "once), f32 accumulate",
        "config": {"workload": "BASELINE configs[2] fc1: C[5184,4096] f32 = A[5184,1024] bf16 x "
                               "W[4096,1024]^T Q8_0 (36-byte blocks along K), one "
                               "sam3_hip_matmul per step", "M": M, "N": N, "K": K},
        "roofline": {"bound": "mfma", "achieved": round(value, 2), "peak": PEAK_BF16_TFLOPS,
                     "unit": "TFLOP/s", "frac": round(value / PEAK_BF16_TFLOPS, 4),
                     "traffic": measured_traffic("q8_fc1_f16_gemm_5184x4096x1024"),
                     "dominant_kernel": {
                         "kernel": "f16 GEMM on the expanded weight (f32 out)",
                         "us": round(ms_g * 1e3, 2), "tflops": round(g, 2),
                         "frac": round(g / PEAK_BF16_TFLOPS, 4)},
                     "other_kernels_us": round((ms - ms_g) * 1e3, 2)},
    }
    if with_cpu:
        log("cpu baseline (reference Q8_0 kernel, row sample)")
        rec["cpu_baseline"] = q8_cpu_baseline(synth.randn(synth.tensor_seed(7, 0), (M, K)), N, K)
    return rec


def traffic_calibration(stream, n=64 << 20, reps=5):
    """Known-traffic launches for the FETCH_SIZE / WRITE_SIZE scale: the
    CAST node kernel f32 -> bf16 (cast_k) over n elements reads 4n bytes
    and writes 2n bytes once each, no reuse (256 MiB and 128 MiB here)."""
    import ctypes as C
    lib = hip.load()
    src, dst = hip.DeviceBuffer(4 * n), hip.DeviceBuffer(2 * n)
    ti = abi.make_tensor(abi.F32, [n], src.ptr, 4 * n)
    to = abi.make_tensor(abi.BF16, [n], dst.ptr, 2 * n)
    nd = abi.Node()
    nd.op, nd.n_inputs = abi.OP_CAST, 1
    nd.inputs[0] = C.pointer(ti)
    nd.output = C.pointer(to)
    nd.params[0] = abi.BF16
    for _ in range(reps):
        hip.check(lib.sam3_hip_cast_on_path(2, C.byref(nd), stream), "calibration cast")
    hip.check(lib.sam3_hip_stream_synchronize(stream), "sync")
    src.free(); dst.free()  # noqa: E702
    return {"kernel": "cast_k<f32,bf16,hw>", "read_bytes": 4 * n, "write_bytes": 2 * n}


class HipGraph:
    """Stream capture into a HIP graph, through the HIP runtime our library
    already loaded (bench plumbing: replaying a captured sequence of
    launches removes the per-call host cost from the measurement)."""

    def __init__(self, stream, record):
        import ctypes as C
        self.rt = rt = C.CDLL("libamdhip64.so.7")
        vp = C.c_void_p
        rt.hipStreamBeginCapture.argtypes = [vp, C.c_int]
        rt.hipStreamEndCapture.argtypes = [vp, C.POINTER(vp)]
        rt.hipGraphInstantiate.argtypes = [C.POINTER(vp), vp, vp, vp, C.c_size_t]
        rt.hipGraphLaunch.argtypes = [vp, vp]
        rt.hipGraphExecDestroy.argtypes = [vp]
        rt.hipGraphDestroy.argtypes = [vp]
        self.stream = stream
        self.graph, self.exec = C.c_void_p(), C.c_void_p()
        self._ok(rt.hipStreamBeginCapture(stream, 2), "begin capture")
        try:
            record()
        finally:
            self._ok(rt.hipStreamEndCapture(stream, C.byref(self.graph)), "end capture")
        self._ok(rt.hipGraphInstantiate(C.byref(self.exec), self.graph, None, None, 0),
                 "instantiate")

    @staticmethod
    def _ok(rc, what):
        if rc != 0:
            raise RuntimeError(f"HIP graph {what}: error {rc}")

    def launch(self):
        self._ok(self.rt.hipGraphLaunch(self.exec, self.stream), "launch")

    def close(self):
        self.rt.hipGraphExecDestroy(self.exec)
        self.rt.hipGraphDestroy(self.graph)


def skinny_stream(lib, stream, O, use_graph=True):
    """Q8 weights [N,K] (36-byte blocks), f32
    activations [M,K], M in {1,8,32,77}. Each shape streams `copies`
    distinct weight copies (> 256 MB in total, so the MALL cannot hold
    them) and reports bytes / time with bytes = W + 4MK + 4MN per call:
      graph_*    one launch per weight copy, the launches captured in a HIP
                 graph and replayed (what a decoder layer loop sees); with
                 use_graph False the launches are issued one by one instead
                 ("eager_*", host launch cost included);
      batched_*  all copies in one sam3_hip_matmul_q8_batched launch (the
                 kernel's streaming rate without per-launch cost);
      launch_us  the difference per call: the per-launch cost."""
    timer = Timer(stream)
    out = {}
    for (kk, nn) in [(4096, 1024), (1024, 4096), (1024, 1024), (256, 2048), (256, 256)]:
        wq = O.q8_quantize(synth.randn(synth.tensor_seed(4, kk + nn), (nn, kk), 0.02))
        wb = wq.nbytes
        copies = min(4096, max(16, int(300e6 // wb) + 1))
        pool = hip.DeviceBuffer(wb * copies)
        for i in range(copies):
            hip.check(lib.sam3_hip_memcpy_h2d(pool.ptr + i * wb, wq.ctypes.data, wb), "h2d")
        for m in (1, 8, 32, 77):
            xa = hip.DeviceBuffer.of(synth.randn(synth.tensor_seed(4, m), (m, kk)))
            yc = hip.DeviceBuffer(m * nn * 4 * copies)

            def calls():
                for i in range(copies):
                    hip.matmul_dev(abi.F32, xa.ptr, abi.Q8_0, pool.ptr + i * wb, abi.F32,
                                   yc.ptr + i * m * nn * 4, m, nn, kk, None, hip.B_NT, stream)

            if use_graph:
                g = HipGraph(stream, calls)
                ms_g = timer.run(g.launch, 3, 1) / copies
                g.close()
            else:
                ms_g = timer.run(calls, 3, 1) / copies
            mode = "graph" if use_graph else "eager"

            def batched():
                hip.q8_batched_dev(abi.F32, xa.ptr, pool.ptr, yc.ptr, copies, m, nn, kk,
                                   0, wb, m * nn, None, 0, stream)

            ms_b = timer.run(batched, 3, 1) / copies
            byts = wb + 4 * m * kk + 4 * m * nn
            out[f"M{m}_K{kk}_N{nn}"] = {
                f"{mode}_us": round(ms_g * 1e3, 3),
                f"{mode}_gbs": round(byts / (ms_g * 1e-3) / 1e9, 1),
                "batched_us": round(ms_b * 1e3, 3),
                "batched_gbs": round(byts / (ms_b * 1e-3) / 1e9, 1),
                "launch_us": round((ms_g - ms_b) * 1e3, 3)}
            log(f"  M{m} K{kk} N{nn}: {out[f'M{m}_K{kk}_N{nn}']}")
            xa.free(); yc.free()  # noqa: E702
        pool.free()
    return out


def main():
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--quick", action="store_true", help="headline only, no extra configs")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-q8", action="store_true", help="leave out the Q8 line (\"q8\" key)")
    ap.add_argument("--calibrate-traffic", action="store_true",
                    help="also run the known-traffic cast launches that scale rocprofv3's "
                         "FETCH_SIZE / WRITE_SIZE")
    ap.add_argument("--no-graph", action="store_true",
                    help="config 4: issue the per-copy launches directly, not from a HIP graph")
    ap.add_argument("--only", default="cfg1,cfg2,cfg3,cfg4,cfg5,textenc,block,conv,neck,weights",
                    help="comma list of extra sections to run (cfg1..cfg5, textenc, block, conv, "
                         "neck, weights)")
    ap.add_argument("--block",
                    default="windowed_f32,windowed_q8,global_f32,global_q8,trunk_q8,trunk_f32",
                    help="block section: comma list of {windowed,global}_{f32,q8} and "
                         "trunk_{q8,f32} (32 blocks)")
    args = ap.parse_args()
    only = set(args.only.split(","))
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print("bench.py: this backend is measured on one GPU only; multi-GPU sharding is a "
              "design note (row/column/split-K split, see the design document), not a run.",
              file=sys.stderr)
        sys.exit(2)

    lib = hip.load()
    if lib.sam3_hip_device_count() < 1:
        print("bench.py: no HIP device", file=sys.stderr)
        sys.exit(1)
    arch = lib.sam3_hip_device_arch(0).decode()
    log("device", arch)
    sp = hip.C.c_void_p()
    hip.check(lib.sam3_hip_stream_create(hip.C.byref(sp)), "stream_create")
    stream = sp.value
    timer = Timer(stream)
    K_, W_ = args.steps, args.warmup

    # ---------------- headline: config 2 fc1, bf16, C = A W^T
    M, N, K = 5184, 4096, 1024
    a32 = synth.randn(synth.tensor_seed(2, 0), (M, K))
    w32 = synth.randn(synth.tensor_seed(2, 1), (N, K), 0.02)
    a_bf, w_bf = bf16_bits(a32), bf16_bits(w32)
    log("headline bf16 fc1", M, N, K)
    # the first GPU work of the process: 0.2 s untimed, then the W warmup steps
    ms = gemm_case(stream, timer, abi.BF16, a_bf, abi.BF16, w_bf, abi.BF16, M, N, K, hip.B_NT, K_, W_,
                   settle_s=0.2)
    value = tflops(M, N, K, ms)
    log(f"  {ms * 1e3:.1f} us/step  {value:.1f} TFLOP/s")

    q8 = None
    if not args.no_q8:
        log("Q8 line: bf16 x Q8_0 fc1", M, N, K)
        q8 = q8_record(stream, timer, a_bf, w32, K_, W_, not args.no_cpu_baseline)
        log(f"  {q8['ms_per_step'] * 1e3:.1f} us/step  {q8['value']:.1f} TFLOP/s; f16 GEMM "
            f"{q8['roofline']['dominant_kernel']['us']:.1f} us")

    extra = {}
    if args.calibrate_traffic:
        extra["traffic_calibration"] = traffic_calibration(stream)
    steps2, warm2 = max(10, K_ // 4), max(3, W_ // 2)
    if not args.quick and "cfg2" in only:
        bias = bf16_bits(synth.randn(synth.tensor_seed(2, 2), N, 0.01))
        log("config 2 variants")
        ms_e = gemm_case(stream, timer, abi.BF16, a_bf, abi.BF16, w_bf, abi.BF16, M, N, K,
                         hip.B_NT | hip.BIAS | hip.GELU, steps2, warm2, bias=bias)
        extra["cfg2_bf16_fc1_bias_gelu_tflops"] = round(tflops(M, N, K, ms_e), 2)
        ms_nn = gemm_case(stream, timer, abi.BF16, a_bf, abi.BF16, np.ascontiguousarray(w_bf.T),
                          abi.BF16, M, N, K, 0, steps2, warm2)
        extra["cfg2_bf16_fc1_kn_layout_tflops"] = round(tflops(M, N, K, ms_nn), 2)
        a2 = bf16_bits(synth.randn(synth.tensor_seed(2, 3), (M, 4096)))
        w2 = bf16_bits(synth.randn(synth.tensor_seed(2, 4), (1024, 4096), 0.02))
        ms2 = gemm_case(stream, timer, abi.BF16, a2, abi.BF16, w2, abi.BF16, M, 1024, 4096,
                        hip.B_NT, steps2, warm2)
        extra["cfg2_bf16_fc2_tflops"] = round(tflops(M, 1024, 4096, ms2), 2)
        ms_h = gemm_case(stream, timer, abi.F16, f16_bits(a32), abi.F16, f16_bits(w32), abi.F16,
                         M, N, K, hip.B_NT, steps2, warm2)
        extra["cfg2_f16_fc1_tflops"] = round(tflops(M, N, K, ms_h), 2)
        del a2, w2

    O = hip  # Q8 weights are quantized on the device (sam3_hip_q8_quantize)
    if not args.quick and "cfg1" in only:
        log("config 1 / Q8")
        a1 = synth.randn(0, (5184, 1024))
        wq1 = O.q8_quantize(synth.randn(1, (1024, 1024), 0.02))
        ms1 = gemm_case(stream, timer, abi.F32, a1, abi.Q8_0, wq1, abi.F32, 5184, 1024, 1024,
                        hip.B_NT, steps2, warm2)
        bytes1 = 5184 * 1024 * 4 * 2 + wq1.nbytes
        extra["cfg1_q8_f32act_5184x1024x1024"] = {
            "us": round(ms1 * 1e3, 2), "tflops": round(tflops(5184, 1024, 1024, ms1), 2),
            "gbs": round(bytes1 / (ms1 * 1e-3) / 1e9, 1)}

    if not args.quick and "cfg3" in only:
        log("config 3: 32 layers, distinct Q8 weights")
        shapes = [(3072, 1024), (1024, 1024), (4096, 1024), (1024, 4096)]
        # distinct seeded weights for every layer, quantized on the device
        layers, wbytes, wlast = [], 0, None
        for L in range(32):
            bufs = []
            for i, s in enumerate(shapes):
                wq = O.q8_quantize(synth.randn(synth.tensor_seed(3, 100 + 4 * L + i), s, 0.02))
                bufs.append(hip.DeviceBuffer.of(wq))
                wbytes += wq.nbytes
                wlast = wq
            layers.append(bufs)
        a4_bits = bf16_bits(synth.randn(synth.tensor_seed(3, 10), (M, 4096)))
        act1 = hip.DeviceBuffer.of(bf16_bits(synth.randn(synth.tensor_seed(3, 9), (M, 1024))))
        act4 = hip.DeviceBuffer.of(a4_bits)
        out = hip.DeviceBuffer(M * 4096 * 4)

        def encoder():
            for L in layers:
                for (n_, k_), wb in zip(shapes, L):
                    hip.matmul_dev(abi.BF16, (act4 if k_ == 4096 else act1).ptr, abi.Q8_0, wb.ptr,
                                   abi.F32, out.ptr, M, n_, k_, None, hip.B_NT, stream)

        ms3 = timer.run(encoder, 3, 1)
        flops3 = 32 * sum(2.0 * M * n_ * k_ for n_, k_ in shapes)
        # the stream's last GEMM (layer 31's fc2) left its whole output:
        # against float64 on the dequantized weight (outside the timing)
        hip.check(lib.sam3_hip_stream_synchronize(stream), "sync")
        n_, k_ = shapes[-1]
        got = out.download(np.float32, (M, n_)).astype(np.float64)
        wd = hip.q8_dequantize(wlast, n_ * k_).reshape(n_, k_).astype(np.float64)
        a4 = (a4_bits.astype(np.uint32) << 16).view(np.float32).astype(np.float64)
        ref = a4 @ wd.T
        err3 = float(np.abs(got - ref).max() / np.abs(ref).max())
        extra["cfg3_q8_32layers"] = {"ms": round(ms3, 3),
                                     "tflops": round(flops3 / (ms3 * 1e-3) / 1e12, 2),
                                     "weights_mb": round(wbytes / 1e6, 1),
                                     "last_output_normwise_err_vs_f64": float(f"{err3:.3g}")}
        del got, ref, a4, wd
        for L in layers:
            for b in L:
                b.free()
        act1.free(); act4.free(); out.free()  # noqa: E702

    if not args.quick and "cfg4" in only:
        log("config 4: skinny Q8 (stream of distinct weight copies)")
        extra["cfg4_skinny_q8"] = skinny_stream(lib, stream, O, not args.no_graph)

    if not args.quick and "cfg5" in only:
        log("config 5: attention matmuls (windowed)")
        BH, S, D = 1296, 576, 64
        qk = bf16_bits(synth.randn(synth.tensor_seed(5, 0), (BH, S, D)) / 8)
        dq, dk = hip.DeviceBuffer.of(qk), hip.DeviceBuffer.of(qk)
        ds = hip.DeviceBuffer(BH * S * S * 2)
        do = hip.DeviceBuffer(BH * S * D * 2)

        def qkt():
            hip.check(lib.sam3_hip_matmul_batched(abi.BF16, dq.ptr, dk.ptr, ds.ptr, BH, S, S, D,
                                                  S * D, S * D, S * S, hip.B_NT, stream), "qkt")

        def pv():
            hip.check(lib.sam3_hip_matmul_batched(abi.BF16, ds.ptr, dq.ptr, do.ptr, BH, S, D, S,
                                                  S * S, S * D, S * D, 0, stream), "pv")

        ms_qk = timer.run(qkt, 5, 2)
        ms_pv = timer.run(pv, 5, 2)
        bytes_qk = BH * (2 * S * D * 2 + S * S * 2)
        extra["cfg5_attn_windowed"] = {
            "qkt_us": round(ms_qk * 1e3, 1), "qkt_tflops": round(tflops(BH * S, S, D, ms_qk), 1),
            "qkt_gbs": round(bytes_qk / (ms_qk * 1e-3) / 1e9, 1),
            "pv_us": round(ms_pv * 1e3, 1), "pv_tflops": round(tflops(BH * S, D, S, ms_pv), 1),
            "pv_gbs": round(bytes_qk / (ms_pv * 1e-3) / 1e9, 1)}
        for b in (dq, dk, ds, do):
            b.free()

        log("config 5: fused attention (SDPA), windowed and global")
        fused = {}
        for name, BH, S in (("windowed", 1296, 576), ("global", 16, 5184)):
            for dname, dt, es in (("bf16", abi.BF16, 2), ("f16", abi.F16, 2), ("f32", abi.F32, 4)):
                n = BH * S * D
                x = synth.randn(synth.tensor_seed(6, 0), (n,))
                host = (bf16_bits(x) if dt == abi.BF16 else f16_bits(x) if dt == abi.F16
                        else x)
                bq = hip.DeviceBuffer.of(host)
                bk = hip.DeviceBuffer.of(host[::-1].copy())
                bv = hip.DeviceBuffer.of(host)
                bo = hip.DeviceBuffer(n * es)

                def sdpa():
                    hip.check(lib.sam3_hip_sdpa(dt, bq.ptr, bk.ptr, bv.ptr, None, bo.ptr,
                                                BH, S, S, D, stream), "sdpa")

                ms_f = timer.run(sdpa, 5, 2)
                tf = 4.0 * BH * S * S * D / (ms_f * 1e-3) / 1e12
                fused[f"{name}_{dname}"] = {"us": round(ms_f * 1e3, 1), "tflops": round(tf, 1),
                                            "frac_bf16_peak": round(tf / PEAK_BF16_TFLOPS, 4)}
                for b in (bq, bk, bv, bo):
                    b.free()
        extra["cfg5_sdpa_fused"] = dict(
            fused, note="one sam3_hip_sdpa launch over BH heads, D=64, no mask; "
                        "4*S^2*D flops per head (Q K^T and P V)")
        if not args.no_cpu_baseline:
            log("config 5: reference CPU SDPA (head sample)")
            extra["cfg5_sdpa_fused"]["cpu_reference"] = {
                "windowed": cpu_sdpa(1296, 576, D), "global": cpu_sdpa(16, 5184, D)}
        log("  ", extra["cfg5_sdpa_fused"])

    if not args.quick and "block" in only:
        log("ViT-L block through graph_eval (windowed / global; f32 / Q8_0 weights)")
        blk = {}
        want = set(args.block.split(","))
        for name, glob in (("windowed", False), ("global", True)):
            for wk in ("f32", "q8"):
                if f"{name}_{wk}" not in want:
                    continue
                blk[f"{name}_{wk}"] = vit_block_bench(glob, wk)
                log("  ", name, wk, blk[f"{name}_{wk}"])
        for wk in ("q8", "f32"):
            if f"trunk_{wk}" not in want:
                continue
            blk[f"trunk_32_blocks_{wk}"] = vit_trunk_bench(wk)
            log("   trunk", wk, blk[f"trunk_32_blocks_{wk}"])
        if not args.no_cpu_baseline:
            blk["cpu_reference"] = vit_block_cpu()
        blk["note"] = ("5184 tokens, e 1024, 16 heads, MLP 4096, f32 activations; every node "
                       "on the GPU; block input in HBM, no readback; wall time of graph_eval")
        extra["vit_block"] = blk

    if not args.quick and "textenc" in only:
        log("text encoder: 24 dependent layers, Q8_0 weights, seq 1/8/32/77")
        extra["text_encoder_chain"] = text_encoder_bench()

    if not args.quick and "conv" in only:
        log("conv2d: patch embedding and neck convs (NHWC x OHWI)")
        cv = {}
        for name, (xs, ws, st, pd) in CONV_SHAPES.items():
            for kind in ("f32", "bf16"):
                cv[f"{name}_{kind}"] = conv_case(lib, stream, timer, kind, xs, ws, st, pd,
                                                 min(K_, 20), min(W_, 3))
                log("  ", name, kind, cv[f"{name}_{kind}"])
        if not args.no_cpu_baseline:
            cv["cpu_reference"] = {n: cpu_conv(n) for n in ("patch_embed", "neck_3x3_72")}
        cv["note"] = ("one sam3_hip_kernel_conv2d per step, inputs in HBM; 2*M*OC*K flops with "
                      "M = N*OH*OW, K = KH*KW*C; f32 runs on bf16 hi/lo planes")
        extra["conv2d"] = cv

    if not args.quick and "neck" in only:
        log("FPN neck, four scales, f32 (necks.c)")
        extra["neck_f32"] = neck_bench()
        log("  ", extra["neck_f32"])

    if not args.quick and "weights" in only:
        log("weights: .sam3 blob (32 ViT-L layers, Q8_0 linear weights) to HBM")
        extra["weights_upload"] = weights_upload_bench()
        log("  ", extra["weights_upload"])

    cpu = None
    if not args.no_cpu_baseline:
        log("cpu baseline (reference bf16 kernel, row sample)")
        cpu = cpu_baseline(a_bf, w_bf, M, N, K)
        log("  ", cpu)

    line = {
        "metric": "TFLOP/s, bf16 GEMM 5184x1024x4096 (ViT-L fc1, f32 accumulate)",
        "value": round(value, 2),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": K_,
        "warmup": W_,
        "ms_per_step": round(ms, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic: seeded SplitMix64/Box-Muller, A N(0,1), W N(0,0.02)",
        "config": {"workload": "BASELINE configs[1] fc1: C[5184,4096] = A[5184,1024] W[4096,1024]^T, "
                               "bf16 in/out, f32 accumulate, one GEMM launch per step",
                   "M": M, "N": N, "K": K, "arch": arch},
        "roofline": {"bound": "mfma", "achieved": round(value, 2), "peak": PEAK_BF16_TFLOPS,
                     "unit": "TFLOP/s", "frac": round(value / PEAK_BF16_TFLOPS, 4),
                     "traffic": measured_traffic("bf16_fc1_5184x4096x1024")},
        "cpu_baseline": cpu,
        "q8": q8,
        "extra": extra,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
