"""CPU-side checks of the C ABI (no GPU needed): the library loads, exports
every entry point include/*.h declares, the mirrored structs have sam3.c's
sizes, kernel-path selection, and the argument/dtype error behaviour that
mirrors the reference CPU path (all of these return before any device
call)."""
import ctypes as C
import re
import subprocess
from pathlib import Path

import pytest

from sam3_amd import abi, hip

ROOT = Path(__file__).resolve().parents[1]


@pytest.fixture(autouse=True)
def quiet(env):
    env.set("SAM3_HIP_QUIET", "1")


def declared_entry_points():
    names = set()
    for h in (ROOT / "include").glob("*.h"):
        text = re.sub(r"/\*.*?\*/", "", h.read_text(), flags=re.S)
        for m in re.finditer(r"\b(sam3_hip_\w+)\s*\(", text):
            names.add(m.group(1))
    return sorted(names)


def test_exports_every_declared_symbol():
    lib = hip.load()
    names = declared_entry_points()
    assert len(names) >= 30
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing
    # and the Python binding declares each of them
    assert set(names) <= set(hip.SIGNATURES), set(names) - set(hip.SIGNATURES)


def test_struct_layouts_match_reference_sizes():
    # x86-64 sizes of sam3.c's structs (src/core/tensor.h:24-49, graph.h:77-90)
    assert C.sizeof(abi.Tensor) == 64
    assert C.sizeof(abi.Node) == 104
    assert C.sizeof(abi.Graph) == 104 * 16384 + 8
    assert C.sizeof(abi.BackendOps) == 6 * 8


@pytest.mark.parametrize("args,path", [
    ((abi.BF16, abi.BF16, abi.BF16, 5184, 4096, 1024, hip.B_NT), hip.PATH_MFMA),
    ((abi.BF16, abi.BF16, abi.BF16, 5184, 4096, 1024, 0), hip.PATH_MFMA),
    ((abi.F16, abi.F16, abi.F16, 5184, 1024, 4096, hip.B_NT), hip.PATH_MFMA),
    ((abi.F32, abi.Q8_0, abi.F32, 5184, 1024, 1024, hip.B_NT), hip.PATH_MFMA),
    ((abi.BF16, abi.Q8_0, abi.F32, 5184, 3072, 1024, hip.B_NT), hip.PATH_MFMA),
    ((abi.F32, abi.Q8_0, abi.F32, 1, 1024, 4096, hip.B_NT), hip.PATH_SKINNY),
    ((abi.F32, abi.Q8_0, abi.F32, 77, 256, 256, hip.B_NT), hip.PATH_SKINNY),
    ((abi.F32, abi.Q8_0, abi.F32, 4, 4, 64, 0), hip.PATH_GENERIC),
    ((abi.F32, abi.Q8_0, abi.F32, 512, 512, 512, 0), hip.PATH_MFMA),   # unpacked to f16
    ((abi.F32, abi.F32, abi.F32, 7, 5, 13, 0), hip.PATH_GENERIC),
    ((abi.F16, abi.F16, abi.F16, 19, 23, 70, 0), hip.PATH_GENERIC),
    ((abi.BF16, abi.Q8_0, abi.F32, 8, 8, 8, 0), hip.PATH_GENERIC),
    ((abi.BF16, abi.Q8_0, abi.BF16, 8, 8, 8, 0), hip.PATH_NONE),     # Q8 writes F32
    ((abi.F32, abi.BF16, abi.F32, 8, 8, 8, 0), hip.PATH_NONE),      # mixed dense dtypes
    ((abi.I32, abi.I32, abi.I32, 8, 8, 8, 0), hip.PATH_NONE),
])
def test_path_selection(args, path):
    assert hip.matmul_path(*args) == path


def test_plain_entry_argument_errors():
    lib = hip.load()
    ok = 16  # any non-NULL address: these calls fail before touching it
    assert lib.sam3_hip_matmul(abi.F32, ok, abi.F32, ok, abi.F32, ok, -1, 4, 4, None, 0, None) == abi.EINVAL
    assert lib.sam3_hip_matmul(abi.F32, ok, abi.F32, ok, abi.F32, ok, 0, 4, 4, None, 0, None) == abi.OK
    assert lib.sam3_hip_matmul(abi.F32, None, abi.F32, ok, abi.F32, ok, 4, 4, 4, None, 0, None) == abi.EINVAL
    assert lib.sam3_hip_matmul(abi.F32, ok, abi.F32, ok, abi.F32, ok, 4, 4, 4, None, hip.BIAS, None) == abi.EINVAL
    assert lib.sam3_hip_matmul(abi.F32, ok, abi.BF16, ok, abi.F32, ok, 4, 4, 4, None, 0, None) == abi.EDTYPE
    assert lib.sam3_hip_matmul(abi.I8, ok, abi.I8, ok, abi.I8, ok, 4, 4, 4, None, 0, None) == abi.EDTYPE
    assert lib.sam3_hip_matmul(abi.BF16, ok, abi.BF16, ok, abi.F16, ok, 4, 4, 4, None, 0, None) == abi.EDTYPE
    assert lib.sam3_hip_matmul(abi.F32, ok, abi.Q8_0, ok, abi.Q8_0, ok, 4, 4, 4, None, 0, None) == abi.EDTYPE
    assert lib.sam3_hip_matmul_on_path(9, abi.F32, ok, abi.F32, ok, abi.F32, ok, 4, 4, 4, None, 0, None) == abi.EINVAL
    assert lib.sam3_hip_matmul_batched(abi.BF16, ok, ok, ok, 2, 4, 4, 4, 16, 16, 16, hip.BIAS, None) == abi.EINVAL
    assert lib.sam3_hip_matmul_batched(abi.I32, ok, ok, ok, 2, 4, 4, 4, 16, 16, 16, 0, None) == abi.EDTYPE
    assert lib.sam3_hip_matmul_batched(abi.BF16, ok, ok, ok, 0, 4, 4, 4, 16, 16, 16, 0, None) == abi.OK
    assert lib.sam3_hip_matmul(abi.F32, ok, abi.BF16, ok, abi.F32, ok, 4, 4, 4, None, 0, None) == abi.EDTYPE
    assert b"unsupported dtypes" in lib.sam3_hip_last_error()
    # Q8 batched, quantize, dequantize: argument checks before any device call
    assert lib.sam3_hip_matmul_q8_batched(abi.F32, ok, ok, ok, 2, 4, 4, 33, 16, 36, 16, None, 0, None) == abi.EINVAL
    assert lib.sam3_hip_matmul_q8_batched(abi.I8, ok, ok, ok, 2, 4, 4, 32, 16, 36, 16, None, 0, None) == abi.EDTYPE
    assert lib.sam3_hip_matmul_q8_batched(abi.F32, ok, ok, ok, 2, 4, 4, 32, 16, 36, 16, None, hip.BIAS, None) == abi.EINVAL
    assert lib.sam3_hip_matmul_q8_batched(abi.F32, ok, ok, ok, 0, 4, 4, 32, 16, 36, 16, None, 0, None) == abi.OK
    assert lib.sam3_hip_q8_quantize(None, ok, 5, None) == abi.EINVAL
    assert lib.sam3_hip_q8_quantize(ok, ok, -1, None) == abi.EINVAL
    assert lib.sam3_hip_q8_quantize(ok + 2, ok, 5, None) == abi.EINVAL
    assert lib.sam3_hip_q8_quantize(ok, ok, 0, None) == abi.OK
    assert lib.sam3_hip_q8_dequantize(ok, None, 5, None) == abi.EINVAL
    assert lib.sam3_hip_q8_dequantize(ok, ok, 0, None) == abi.OK


def _node(op, ins, out, params=(0, 0, 0, 0)):
    return abi.make_node(op, ins, out, params)


def _t(dtype, dims):
    return abi.make_tensor(dtype, dims, 4096)  # fake data address: never touched


def test_node_kernel_shape_and_dtype_errors():
    """cpu_kernel_matmul*: NULL, wrong dtype, K mismatch and output size
    mismatch are SAM3_EINVAL (cpu_matmul.c:178-229, cpu_matmul_q8.c:168-213)."""
    lib = hip.load()
    a, b, c = _t(abi.F32, [4, 8]), _t(abi.F32, [9, 3]), _t(abi.F32, [4, 3])
    assert lib.sam3_hip_kernel_matmul(C.byref(_node(abi.OP_MATMUL, [a, b], c)), None) == abi.EINVAL
    b = _t(abi.F32, [8, 3])
    c_bad = _t(abi.F32, [4, 4])
    assert lib.sam3_hip_kernel_matmul(C.byref(_node(abi.OP_MATMUL, [a, b], c_bad)), None) == abi.EINVAL
    assert lib.sam3_hip_kernel_matmul_bf16(C.byref(_node(abi.OP_MATMUL, [a, b], c)), None) == abi.EINVAL
    assert lib.sam3_hip_kernel_matmul_f16(C.byref(_node(abi.OP_MATMUL, [a, b], c)), None) == abi.EINVAL
    q = _t(abi.Q8_0, [8, 3])
    cb = _t(abi.BF16, [4, 3])
    assert lib.sam3_hip_kernel_matmul_q8(C.byref(_node(abi.OP_MATMUL, [a, q], cb)), None) == abi.EINVAL
    n1 = abi.Node()
    n1.n_inputs = 2
    assert lib.sam3_hip_kernel_matmul(C.byref(n1), None) == abi.EINVAL


def test_dispatch_routing_errors():
    """cpu_dispatch_node routing (cpu_dispatch.c:591-686): NONE is a no-op,
    BF16 x Q8_0 and other mixed dtypes are SAM3_EDTYPE, an op without a
    kernel is SAM3_EDTYPE, a node without inputs is SAM3_EINVAL."""
    lib = hip.load()
    d = lib.sam3_hip_dispatch_node
    assert d(C.byref(abi.Node()), None) == abi.OK  # OP_NONE
    none_in = abi.Node()
    none_in.op = abi.OP_MATMUL
    assert d(C.byref(none_in), None) == abi.EINVAL
    ab, q, cb = _t(abi.BF16, [4, 32]), _t(abi.Q8_0, [32, 4]), _t(abi.BF16, [4, 4])
    assert d(C.byref(_node(abi.OP_MATMUL, [ab, q], cb)), None) == abi.EDTYPE
    a32, b16 = _t(abi.F32, [4, 8]), _t(abi.F16, [8, 4])
    assert d(C.byref(_node(abi.OP_MATMUL, [a32, b16], _t(abi.F32, [4, 4]))), None) == abi.EDTYPE
    x = _t(abi.F32, [4, 4])
    assert d(C.byref(_node(abi.OP_SOFTMAX, [x], _t(abi.F32, [4, 4]))), None) == abi.EDTYPE
    assert d(C.byref(_node(abi.OP_MATMUL, [_t(abi.I32, [2, 2]), _t(abi.I32, [2, 2])],
                           _t(abi.I32, [2, 2]))), None) == abi.EDTYPE
    # transposes: params that are not a permutation, and a dtype without an
    # element size (Q8_0 is blocked)
    t3 = _t(abi.F32, [2, 3, 4])
    assert d(C.byref(_node(abi.OP_TRANSPOSE, [t3], _t(abi.F32, [3, 3, 2]), (1, 1, 0, 0))),
             None) == abi.EINVAL
    assert d(C.byref(_node(abi.OP_TRANSPOSE, [_t(abi.Q8_0, [32, 4])], _t(abi.Q8_0, [4, 32]))),
             None) == abi.EDTYPE
    # block ops: bad shapes and dtypes are refused before any launch
    assert d(C.byref(_node(abi.OP_LAYERNORM, [_t(abi.I32, [4, 4])], _t(abi.I32, [4, 4]))),
             None) == abi.EDTYPE
    assert d(C.byref(_node(abi.OP_LAYERNORM, [x, _t(abi.F32, [3])], _t(abi.F32, [4, 4]))),
             None) == abi.EINVAL
    x4 = _t(abi.F32, [1, 5, 2, 8])
    assert d(C.byref(_node(abi.OP_ROPE, [x4, _t(abi.F32, [5, 4]), _t(abi.F32, [4, 4])],
                           _t(abi.F32, [1, 5, 2, 8]))), None) == abi.EINVAL
    assert d(C.byref(_node(abi.OP_ROPE, [x4, _t(abi.BF16, [5, 4]), _t(abi.BF16, [5, 4])],
                           _t(abi.F32, [1, 5, 2, 8]))), None) == abi.EDTYPE
    assert d(C.byref(_node(abi.OP_SLICE, [t3], _t(abi.F32, [2, 2, 4]), (1, 2, 5, 0))),
             None) == abi.EINVAL
    # RESHAPE is a view: the output takes the input's data pointer
    src, dst = _t(abi.F32, [2, 6]), _t(abi.F32, [3, 4])
    src.data = 0x1000
    assert d(C.byref(_node(abi.OP_RESHAPE, [src], dst)), None) == abi.OK
    assert dst.data == 0x1000 and list(dst.strides)[:2] == [4, 1]
    assert d(C.byref(_node(abi.OP_RESHAPE, [src], _t(abi.F32, [5]))), None) == abi.EINVAL
    # shape errors inside a routed matmul
    assert d(C.byref(_node(abi.OP_MATMUL, [_t(abi.F32, [4, 8]), _t(abi.Q8_0, [9, 4])],
                           _t(abi.F32, [4, 4]))), None) == abi.EINVAL


def test_backend_create_without_device_fails_cleanly():
    lib = hip.load()
    if lib.sam3_hip_device_count() > 0:
        pytest.skip("a device is present")
    assert not lib.sam3_hip_backend_create(0)
    assert b"device" in lib.sam3_hip_last_error()
    ops = C.cast(lib.sam3_hip_backend_ops(), C.POINTER(abi.BackendOps)).contents
    assert ops.graph_eval and ops.alloc_tensor and ops.cache_invalidate and ops.arena_reset


def _strip_c_comments(text):
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return re.sub(r"//[^\n]*", "", text)


def test_no_oracle_in_product_path():
    """The product library neither links nor names the CPU checkers (the C
    restatement liboracle.so, and libsam3ref.so built from the reference's
    own sources), and no product source loads them or calls the reference's
    CPU dispatcher. Comments may cite reference functions; code may not."""
    lib = ROOT / "sam3.c_amd" / "sam3_amd" / "libsam3hip.so"
    data = lib.read_bytes()
    for needle in (b"oracle_", b"liboracle", b"libsam3ref", b"sam3ref",
                   b"cpu_dispatch_node", b"cpu_kernel_", b"dlopen"):
        assert needle not in data, needle
    needed = subprocess.run(["readelf", "-d", str(lib)], capture_output=True,
                            text=True, check=True).stdout
    libs = re.findall(r"\(NEEDED\).*\[(.*?)\]", needed)
    assert libs and all(not n.startswith(("liboracle", "libsam3ref")) for n in libs), libs
    banned = ("oracle_bind", "liboracle", "sam3_oracle", "libsam3ref", "oracle/_ref",
              "cpu_dispatch_node(", "cpu_kernel_", "dlopen", "dlsym")
    for p in (ROOT / "sam3.c_amd").rglob("*"):
        if p.suffix in (".py", ".c", ".h", ".hip"):
            text = p.read_text()
            if p.suffix != ".py":
                text = _strip_c_comments(text)
            for b in banned:
                assert b not in text, (p, b)
