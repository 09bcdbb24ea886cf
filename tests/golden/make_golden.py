"""Write the golden vectors for the matmul path from the REAL reference.

Run in the build container (where /root/reference exists):

    make -C oracle ref && python tests/golden/make_golden.py

It loads oracle/_ref/libsam3ref.so -- the reference's own CPU sources
compiled in place by oracle/Makefile -- and drives its kernels the way the
reference tests do (hand-built sam3_node, cpu_kernel_*(node, pool)). Inputs
come from sam3_amd.synth (seeded SplitMix64/Box-Muller) or from the
reference tests' own formulas (tests/test_matmul_q8.c:73-76). Inputs and
outputs are stored together in matmul_golden.npz, so the GPU box (which has
no /root/reference) can check the oracle and the HIP path against them.
"""
import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parent))

from oracle_bind import Ref  # noqa: E402
from sam3_amd import abi, synth  # noqa: E402


def bf16_bits(ref, x):
    return ref.cast(np.asarray(x, np.float32), abi.F32, abi.BF16, np.uint16).reshape(np.shape(x))


def fp16_bits(ref, x):
    return ref.cast(np.asarray(x, np.float32), abi.F32, abi.F16, np.uint16).reshape(np.shape(x))


WEIGHTS_CONFIG = dict(image_size=1008, encoder_dim=1024, decoder_dim=256, n_encoder_layers=32,
                      n_decoder_layers=2, backbone_type=1, n_fpn_scales=3, variant=2,
                      text_backbone=1)


def weight_fixture_tensors(q8_quantize):
    """Tensors of weights_golden.sam3: every dtype, ragged sizes (padding
    between tensors), a 127-byte name, a 140-byte name (the writer keeps
    127 bytes, weight.c:111-117) and 48 small tensors so lookups probe."""
    t = [("enc.w", abi.F32, [3, 5], synth.randn(synth.tensor_seed(80, 0), (3, 5))),
         ("enc.q8", abi.Q8_0, [4, 32], q8_quantize(synth.randn(synth.tensor_seed(80, 1), 128))),
         ("enc.bf16", abi.BF16, [7], np.arange(7, dtype=np.uint16) * 4099),
         ("enc.i32", abi.I32, [2, 2, 2], np.arange(8, dtype=np.int32) - 3),
         ("enc.f16", abi.F16, [1], np.array([0x3C00], np.uint16)),
         ("enc.i8", abi.I8, [65], (np.arange(65) - 32).astype(np.int8)),
         ("n" * 127, abi.F32, [2], np.array([1.5, -2.5], np.float32)),
         ("m" * 140, abi.F32, [1], np.array([7.0], np.float32))]
    for i in range(48):
        t.append((f"blk.{i}.w", abi.F32, [i % 5 + 1], np.full(i % 5 + 1, i, np.float32)))
    return t


def main():
    R = Ref()
    g = {}

    # -- .sam3 container written by the reference's sam3_weight_write
    from oracle_bind import ref_weight_write
    rc = ref_weight_write(R, HERE / "weights_golden.sam3", weight_fixture_tensors(R.q8_quantize),
                          WEIGHTS_CONFIG)
    assert rc == 0, rc

    # -- Q8 quantize: random, a zero block, a ragged tail and exact .5 ties
    # (scale 1.0 makes x*inv == x; x86 roundf rounds ties away from zero,
    # src/core/quant.c:118-124).
    x = synth.randn(11, 200, 0.02)
    x[32:64] = 0.0
    ties = np.array([127.0, 2.5, -2.5, 0.5, -0.5, 1.5, -1.5, 126.5] + [0.25] * 24, np.float32)
    qx = np.concatenate([x, ties, synth.randn(12, 45, 3.0)]).astype(np.float32)
    g["quant_x"] = qx
    g["quant_blocks"] = R.q8_quantize(qx)
    g["quant_deq"] = R.q8_dequantize(g["quant_blocks"], qx.size)

    # -- Q8 matmul, kernel contract B[K,N] with blocks over the flat index.
    cases_q8 = [
        ("q8_a", 64, 256, 96, 21),   # N % 32 != 0: blocks straddle k-rows
        ("q8_b", 5, 33, 7, 22),      # K*N % 32 != 0: zero-padded tail block
        ("q8_c", 1, 128, 64, 23),    # M == 1 (serial path, cpu_matmul_q8.c:226)
    ]
    for name, M, K, N, seed in cases_q8:
        a = synth.randn(synth.tensor_seed(seed, 0), (M, K))
        w = synth.randn(synth.tensor_seed(seed, 1), (K, N), 0.02)
        b = R.q8_quantize(w)
        g[f"{name}_a"], g[f"{name}_b"] = a, b
        g[f"{name}_shape"] = np.array([M, K, N])
        g[f"{name}_c"] = R.matmul_q8(a, b, K, N, threads=4)

    # the reference test's own small case (tests/test_matmul_q8.c:66-116)
    M, K, N = 4, 64, 4
    a = (np.sin(np.arange(M * K, dtype=np.float32) * np.float32(0.1)) * np.float32(0.5)).reshape(M, K)
    w = (np.cos(np.arange(K * N, dtype=np.float32) * np.float32(0.1)) * np.float32(0.5)).reshape(K, N)
    b = R.q8_quantize(w.astype(np.float32))
    g["q8_t_a"], g["q8_t_b"], g["q8_t_shape"] = a.astype(np.float32), b, np.array([M, K, N])
    g["q8_t_c"] = R.matmul_q8(a.astype(np.float32), b, K, N)

    # -- Q8 with W stored [N,K] (blocks along K): column n is the reference
    # kernel with B = W[n,:] viewed as [K,1].
    M, K, N = 16, 256, 40
    a = synth.randn(synth.tensor_seed(31, 0), (M, K))
    w = synth.randn(synth.tensor_seed(31, 1), (N, K), 0.02)
    wb = R.q8_quantize(w)
    row = K // 32 * 36
    cols = [R.matmul_q8(a, wb[n * row:(n + 1) * row], K, 1) for n in range(N)]
    g["q8nt_a"], g["q8nt_w"], g["q8nt_shape"] = a, wb, np.array([M, K, N])
    g["q8nt_c"] = np.concatenate(cols, axis=1)

    # -- bf16 / f16 / f32 dense GEMMs
    M, K, N = 37, 96, 80
    a32 = synth.randn(synth.tensor_seed(41, 0), (M, K))
    b32 = synth.randn(synth.tensor_seed(41, 1), (K, N))
    ab, bb = bf16_bits(R, a32), bf16_bits(R, b32)
    g["bf16_a"], g["bf16_b"] = ab, bb
    g["bf16_c"] = R.matmul_bf16(ab, bb, threads=3)
    M2, K2, N2 = 19, 70, 23
    ah = fp16_bits(R, synth.randn(synth.tensor_seed(42, 0), (M2, K2)))
    bh = fp16_bits(R, synth.randn(synth.tensor_seed(42, 1), (K2, N2)))
    g["f16_a"], g["f16_b"] = ah, bh
    g["f16_c"] = R.matmul_f16(ah, bh, threads=3)
    af = synth.randn(synth.tensor_seed(43, 0), (7, 13))
    bf = synth.randn(synth.tensor_seed(43, 1), (13, 5))
    g["f32_a"], g["f32_b"] = af, bf
    g["f32_c"] = R.matmul_f32(af, bf)
    af2 = synth.randn(synth.tensor_seed(44, 0), (33, 200))
    bf2 = synth.randn(synth.tensor_seed(44, 1), (200, 65))
    g["f32b_a"], g["f32b_b"] = af2, bf2
    g["f32b_c"] = R.matmul_f32(af2, bf2, threads=4)

    # -- epilogues. The x86 scalar broadcast add only covers the first
    # `rows` elements (split in rows, loop in elements:
    # cpu_elementwise.c:70-78 vs :357-371, cpu_add_bf16.c:86-98 vs
    # :120-135), so the bias is tiled to full shape and the same-shape path
    # (which applies the identical per-element formula) is recorded.
    rows, N = 24, 96
    x = synth.randn(51, (rows, N), 2.0)
    bias = synth.randn(52, N, 0.5)
    tiled = np.tile(bias, rows).reshape(rows, N)

    def add_same(xx, bbias, dt, npt, fn):
        rc, out = R.run(fn, abi.OP_ADD, [(dt, [rows, N], np.ascontiguousarray(xx, npt)),
                                         (dt, [rows, N], np.ascontiguousarray(bbias, npt))],
                        dt, (rows, N), npt)
        assert rc == 0
        return out

    g["ep_x"], g["ep_bias"] = x, bias
    g["ep_add_f32"] = add_same(x, tiled, abi.F32, np.float32, "cpu_kernel_add")
    xb, bb_ = bf16_bits(R, x), bf16_bits(R, bias)
    g["ep_add_bf16"] = add_same(xb, np.tile(bb_, rows).reshape(rows, N), abi.BF16, np.uint16,
                                "cpu_kernel_add_bf16")
    xh, bh_ = fp16_bits(R, x), fp16_bits(R, bias)
    g["ep_add_f16"] = R.add(xh, bh_, "f16")   # f16 broadcast path is row-wise (correct)
    gx = np.linspace(-8.0, 8.0, 4097, dtype=np.float32)
    g["gelu_x"] = gx
    g["gelu_f32"] = R.gelu(gx, "f32")
    g["gelu_bf16"] = R.gelu(bf16_bits(R, gx), "bf16")
    g["gelu_f16"] = R.gelu(fp16_bits(R, gx), "f16")

    # -- conversions: a sample of f32 bit patterns incl. specials
    rng = np.random.default_rng(61)
    pats = rng.integers(0, 2 ** 32, 4096, dtype=np.uint64).astype(np.uint32)
    specials = np.array([0, 0x80000000, 0x7F800000, 0xFF800000, 0x7FC00000, 0x7F800001,
                         0x33000000, 0x387FC000, 0x477FE000, 0x477FF000, 0x3F808000,
                         0x3F818000, 0x00000001, 0x007FFFFF], np.uint32)
    pats = np.concatenate([specials, pats]).view(np.float32)
    g["cvt_f32"] = pats
    g["cvt_bf16"] = R.cast(pats, abi.F32, abi.BF16, np.uint16)
    g["cvt_fp16"] = R.cast(pats, abi.F32, abi.F16, np.uint16)

    # -- SDPA (cpu_kernel_sdpa, cpu_sdpa.c:216-288): 4-D path, with and
    # without the additive mask, ragged key count (not a multiple of the
    # reference's 64-key tile), head_dim 64.
    BH, Sq, Sk, D = 3, 37, 70, 64
    g["sdpa_q"] = synth.randn(synth.tensor_seed(71, 0), (BH, Sq, D)) / 4
    g["sdpa_k"] = synth.randn(synth.tensor_seed(71, 1), (BH, Sk, D)) / 4
    g["sdpa_v"] = synth.randn(synth.tensor_seed(71, 2), (BH, Sk, D))
    g["sdpa_mask"] = synth.randn(synth.tensor_seed(71, 3), (Sq, Sk), 2.0)
    g["sdpa_out"] = R.sdpa(g["sdpa_q"], g["sdpa_k"], g["sdpa_v"], None, threads=3)
    g["sdpa_out_mask"] = R.sdpa(g["sdpa_q"], g["sdpa_k"], g["sdpa_v"], g["sdpa_mask"], threads=3)

    # -- LayerNorm (cpu_layernorm.c, f32, eps 1e-5) over a 96-wide last dim
    # with gamma and beta, and RoPE (cpu_rope.c, f32) on [2, 9, 3, 16].
    g["ln_x"] = synth.randn(synth.tensor_seed(72, 0), (37, 96), 3.0, 0.5)
    g["ln_gamma"] = synth.randn(synth.tensor_seed(72, 1), (96,))
    g["ln_beta"] = synth.randn(synth.tensor_seed(72, 2), (96,))
    g["ln_out"] = R.layernorm(g["ln_x"], g["ln_gamma"], g["ln_beta"], "f32")
    g["rope_x"] = synth.randn(synth.tensor_seed(73, 0), (2, 9, 3, 16))
    ang = np.outer(np.arange(9), 1.0 / (10000.0 ** (np.arange(8) / 8.0)))
    g["rope_cos"] = np.cos(ang).astype(np.float32)
    g["rope_sin"] = np.sin(ang).astype(np.float32)
    g["rope_out"] = R.rope(g["rope_x"], g["rope_cos"], g["rope_sin"], "f32")

    # -- Conv2D NHWC x OHWI (cpu_conv2d.c): 3x3 pad 1; stride 2 with 2
    # groups; the patch embedding's non-overlapping 4x4 stride 4 on C = 3;
    # asymmetric padding; bf16 and f16 twins of the first case
    conv_cases = {"p1": ((1, 9, 7, 8), (6, 3, 3, 8), 1, 1, 0, 1),
                  "s2g2": ((2, 10, 10, 6), (4, 3, 3, 3), 2, 1, 0, 2),
                  "patch": ((1, 12, 12, 3), (16, 4, 4, 3), 4, 0, 0, 1),
                  "asym": ((1, 9, 9, 8), (4, 3, 3, 8), 1, 2, 1, 1)}
    for i, (key, (xs, ws, st, ph, pw, gr)) in enumerate(conv_cases.items()):
        x = synth.randn(synth.tensor_seed(90 + i, 0), xs)
        w = synth.randn(synth.tensor_seed(90 + i, 1), ws, 0.2)
        rc, y = R.conv2d(x, w, st, ph, pw if pw else None, gr)
        assert rc == 0
        g[f"conv_{key}_x"], g[f"conv_{key}_w"], g[f"conv_{key}_y"] = x, w, y
        g[f"conv_{key}_p"] = np.array([st, ph, gr, pw], np.int32)
    x, w = g["conv_p1_x"], g["conv_p1_w"]
    for kind, cv in (("bf16", bf16_bits), ("f16", fp16_bits)):
        xb, wb = cv(R, x), cv(R, w)
        rc, y = R.conv2d(xb, wb, 1, 1, None, 1, kind)
        assert rc == 0
        g[f"conv_p1_{kind}_x"], g[f"conv_p1_{kind}_w"], g[f"conv_p1_{kind}_y"] = xb, wb, y

    # -- ConvTranspose2D (the neck's 2x2 stride 2, and an overlapping 3x3
    # stride 2 pad 1) and MaxPool2D with NaNs in and out of first taps
    for i, (key, xs, ws, st, pd) in enumerate([("k2", (1, 5, 6, 8), (4, 2, 2, 8), 2, 0),
                                               ("k3", (2, 4, 4, 3), (5, 3, 3, 3), 2, 1)]):
        x = synth.randn(synth.tensor_seed(95 + i, 0), xs)
        w = synth.randn(synth.tensor_seed(95 + i, 1), ws, 0.2)
        rc, y = R.conv_transpose2d(x, w, st, pd)
        assert rc == 0
        g[f"convt_{key}_x"], g[f"convt_{key}_w"], g[f"convt_{key}_y"] = x, w, y
        g[f"convt_{key}_p"] = np.array([st, pd], np.int32)
    x = synth.randn(synth.tensor_seed(97, 0), (2, 9, 7, 5))
    x[0, 0, 0, 0] = np.nan
    x[1, 2, 3, 1] = np.nan
    g["maxpool_x"] = x
    for k, st in ((2, 2), (3, 2)):
        rc, y = R.maxpool2d(x, k, st)
        assert rc == 0
        g[f"maxpool_{k}{st}_y"] = y

    R.close()
    out = HERE / "matmul_golden.npz"
    np.savez_compressed(out, **g)
    print(f"wrote {out} ({out.stat().st_size} bytes, {len(g)} arrays)")


if __name__ == "__main__":
    main()
