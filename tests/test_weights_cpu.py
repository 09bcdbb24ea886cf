"""The `.sam3` container mirror (sam3_amd.weights) against the reference's
own loader and writer (src/core/weight.c), on the CPU.

Pins: weights_golden.sam3 was written by the reference's
sam3_weight_write (tests/golden/make_golden.py); the mirror must read it
and re-write it byte for byte. Where oracle/_ref is built, files written
by the mirror are read back by the reference's sam3_weight_open and the
two loaders must agree on every tensor and every error code.
"""
import struct
from pathlib import Path

import numpy as np
import pytest

from oracle_bind import Oracle, Ref, RefWeightFile, have_ref, ref_weight_write
from sam3_amd import abi
from sam3_amd import weights as W

HERE = Path(__file__).resolve().parent
GOLDEN = HERE / "golden" / "weights_golden.sam3"


def fixture_tensors():
    import sys
    sys.path.insert(0, str(HERE / "golden"))
    from make_golden import WEIGHTS_CONFIG, weight_fixture_tensors
    return weight_fixture_tensors(Oracle().q8_quantize), WEIGHTS_CONFIG


def test_fnv1a_known_answers():
    # FNV-1a 32-bit published test vectors.
    assert W.fnv1a("") == 0x811C9DC5
    assert W.fnv1a("a") == 0xE40C292C
    assert W.fnv1a("foobar") == 0xBF9CF968


def test_reads_reference_written_file():
    tensors, cfg = fixture_tensors()
    with W.WeightFile(GOLDEN) as wf:
        assert wf.n_tensors == len(tensors)
        h = wf.header
        assert int(h["version"]) == 4 and int(h["image_size"]) == cfg["image_size"]
        assert tuple(int(x) for x in h["reserved"]) == (cfg["backbone_type"], cfg["variant"],
                                                        cfg["n_fpn_scales"])
        assert wf.text_backbone == cfg["text_backbone"]
        assert wf.data_start % 4096 == 0
        for name, dt, dims, arr in tensors:
            i = wf.find(name[:127])
            assert i is not None, name
            d = wf.descs[i]
            assert int(d["dtype"]) == dt and list(d["dims"][:len(dims)]) == dims
            assert int(d["data_offset"]) % 64 == 0
            assert bytes(wf.array(i)) == np.ascontiguousarray(arr).tobytes()
            t = wf.to_tensor(i)
            assert t.data == wf.data_base + int(d["data_offset"])
            if dt == abi.Q8_0:
                assert list(t.strides) == [0, 0, 0, 0]
        assert wf.find("m" * 140) is None  # stored truncated to 127 bytes
        assert wf.find("missing") is None


def test_writer_reproduces_reference_file(tmp_path):
    tensors, cfg = fixture_tensors()
    out = tmp_path / "ours.sam3"
    W.write(out, tensors, cfg)
    assert out.read_bytes() == GOLDEN.read_bytes()


def test_hash_table_matches_reference_sizing():
    with W.WeightFile(GOLDEN) as wf:
        n = wf.n_tensors
        cap = len(wf.table)
        assert cap & (cap - 1) == 0 and cap >= 4 * n and cap < 8 * n
        assert sorted(i for i in wf.table if i != W.HASH_EMPTY) == list(range(n))


@pytest.mark.skipif(not have_ref(), reason="oracle/_ref not built")
def test_reference_loader_reads_mirror_files(tmp_path):
    tensors, cfg = fixture_tensors()
    path = tmp_path / "m.sam3"
    W.write(path, tensors, cfg)
    R = Ref()
    rf = RefWeightFile(R, path)
    assert rf.rc == 0
    for name, dt, dims, arr in tensors:
        desc = rf.find(name[:127])
        assert desc
        rc, t = rf.to_tensor(desc)
        assert rc == 0 and t.dtype == dt and list(t.dims)[:len(dims)] == dims
        import ctypes as C
        assert C.string_at(t.data, t.nbytes) == np.ascontiguousarray(arr).tobytes()
    rf.close()


@pytest.mark.skipif(not have_ref(), reason="oracle/_ref not built")
def test_writer_matches_reference_writer_random(tmp_path):
    rng = np.random.default_rng(5)
    R = Ref()
    tensors = []
    for i in range(200):
        n = int(rng.integers(1, 300))
        dt = [abi.F32, abi.F16, abi.I8, abi.Q8_0][i % 4]
        if dt == abi.Q8_0:
            arr = R.q8_quantize(rng.standard_normal(n).astype(np.float32))
        else:
            arr = rng.integers(0, 255, n * {abi.F32: 4, abi.F16: 2, abi.I8: 1}[dt], dtype=np.uint8)
        tensors.append((f"t{i}.{rng.integers(1 << 30)}", dt, [n], arr))
    W.write(tmp_path / "a.sam3", tensors)
    assert ref_weight_write(R, tmp_path / "b.sam3", tensors) == 0
    assert (tmp_path / "a.sam3").read_bytes() == (tmp_path / "b.sam3").read_bytes()
    with W.WeightFile(tmp_path / "a.sam3") as wf:
        rf = RefWeightFile(R, tmp_path / "a.sam3")
        for name, _, _, _ in tensors:
            i = wf.find(name)
            d = rf.find(name)
            assert d
            # same descriptor: address inside the reference's table
            assert d == rf.wf.tensors + i * W.DESC.itemsize
        rf.close()


def _corrupt(tmp_path, mutate):
    data = bytearray(GOLDEN.read_bytes())
    mutate(data)
    p = tmp_path / "bad.sam3"
    p.write_bytes(bytes(data))
    return p


CASES = {
    "bad_magic": lambda d: d.__setitem__(slice(0, 4), b"XXXX"),
    "version5": lambda d: d.__setitem__(slice(4, 8), struct.pack("<I", 5)),
    "table_past_end": lambda d: d.__setitem__(slice(12, 16), struct.pack("<I", 10 ** 6)),
    "data_past_end": lambda d: d.__setitem__(slice(52 + 160, 52 + 168),
                                             struct.pack("<Q", 10 ** 9)),
    "truncated": lambda d: d.__delitem__(slice(40, None)),
}


@pytest.mark.parametrize("case", sorted(CASES))
def test_rejects_malformed_files_like_reference(tmp_path, case):
    p = _corrupt(tmp_path, CASES[case])
    with pytest.raises(W.WeightError) as e:
        W.WeightFile(p)
    assert e.value.code == abi.EMODEL
    if have_ref():
        rf = RefWeightFile(Ref(), p)
        assert rf.rc == abi.EMODEL


def test_missing_file_is_eio(tmp_path):
    with pytest.raises(W.WeightError) as e:
        W.WeightFile(tmp_path / "nope.sam3")
    assert e.value.code == abi.EIO
    if have_ref():
        assert RefWeightFile(Ref(), tmp_path / "nope.sam3").rc == abi.EIO


def test_version3_header(tmp_path):
    """v3 files have a 48-byte header (no text_backbone) and the table at
    offset 48 (weight.c:352-363)."""
    tensors, cfg = fixture_tensors()
    W.write(tmp_path / "v4.sam3", tensors[:3], cfg)
    v4 = (tmp_path / "v4.sam3").read_bytes()
    n = 3
    table = v4[52:52 + 176 * n]
    start4 = (52 + 176 * n + 4095) // 4096 * 4096
    start3 = (48 + 176 * n + 4095) // 4096 * 4096
    v3 = bytearray(v4[:48]) + table
    v3[4:8] = struct.pack("<I", 3)
    v3 += b"\0" * (start3 - len(v3)) + v4[start4:]
    (tmp_path / "v3.sam3").write_bytes(bytes(v3))
    with W.WeightFile(tmp_path / "v3.sam3") as wf:
        assert wf.text_backbone == 0
        for name, _, _, arr in tensors[:3]:
            assert bytes(wf.array(wf.find(name))) == np.ascontiguousarray(arr).tobytes()
    if have_ref():
        rf = RefWeightFile(Ref(), tmp_path / "v3.sam3")
        assert rf.rc == 0 and rf.wf.text_backbone == 0
        rf.close()


def test_vit_layer_load_and_host_fuse(tmp_path):
    """load_vit_layer without a backend: q/k/v stacked on the host keep
    their dtype (Q8_0 stays Q8_0, unlike image_encoder.c:223-254)."""
    from sam3_amd import graph
    O = Oracle()
    ents = graph.vit_layer_entries(0, 64, 256, 900, O.q8_quantize)
    W.write(tmp_path / "l.sam3", ents)
    byname = {n: a for n, _, _, a in ents}
    with W.WeightFile(tmp_path / "l.sam3") as wf:
        G = graph.Graph()
        p = graph.load_vit_layer(G, wf, 0)
        qkv = p["qkv_w"]
        assert qkv.dtype == abi.Q8_0 and list(qkv.dims)[:2] == [192, 64]
        import ctypes as C
        want = b"".join(byname[graph.VIT_PREFIX + graph.VIT_NAMES[k].format(0)].tobytes()
                        for k in ("q_w", "k_w", "v_w"))
        assert C.string_at(qkv.data, qkv.nbytes) == want
        assert p["qkv_b"].dtype == abi.F32 and p["qkv_b"].dims[0] == 192
        assert p["fc1_w"].dtype == abi.Q8_0 and p["ln1_w"].dtype == abi.F32
