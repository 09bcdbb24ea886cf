"""ctypes mirror of the sam3.c types that cross the backend boundary.

The layouts restate, field for field, the C structs the reference's graph
builder hands to a backend, so a tensor or node built here is the same
bytes a sam3.c caller would pass:

* ``enum sam3_error`` / ``enum sam3_dtype`` -- include/sam3/sam3_types.h:25-54
* ``struct sam3_tensor``                    -- src/core/tensor.h:24-49
* ``enum sam3_op`` / ``struct sam3_node``   -- src/core/graph.h:27-83
* ``struct sam3_graph``                     -- src/core/graph.h:86-90
* ``struct sam3_q8_block`` (36 bytes)       -- src/core/quant.h:22-33

The same layouts are declared in C in include/sam3_hip_abi.h.
"""
import ctypes as C

MAX_DIMS = 4          # SAM3_MAX_DIMS
NODE_MAX_INPUTS = 8   # SAM3_NODE_MAX_INPUTS
GRAPH_MAX_NODES = 16384
Q8_BLOCK = 32
Q8_BLOCK_BYTES = 36

# enum sam3_error
OK, EINVAL, ENOMEM, EIO, EBACKEND, EMODEL, EDTYPE, EVIDEO = 0, -1, -2, -3, -4, -5, -6, -7
ERROR_NAMES = {0: "OK", -1: "EINVAL", -2: "ENOMEM", -3: "EIO", -4: "EBACKEND",
               -5: "EMODEL", -6: "EDTYPE", -7: "EVIDEO"}

# enum sam3_dtype
F32, F16, BF16, I32, I8, Q8_0 = range(6)

# enum sam3_op (only the members the matmul path touches are named)
OP_NONE, OP_MATMUL, OP_ADD, OP_MUL, OP_SOFTMAX, OP_RELU, OP_GELU = range(7)
OP_LAYERNORM, OP_CONV2D, OP_RESHAPE, OP_TRANSPOSE, OP_CAST = range(7, 12)
OP_CONCAT, OP_SLICE, OP_EMBED, OP_SIGMOID, OP_UPSAMPLE, OP_ROPE = range(12, 18)
OP_SILU, OP_CONV_TRANSPOSE2D, OP_MAXPOOL2D, OP_SDPA, OP_BIAS_ADD = range(18, 23)


class Tensor(C.Structure):
    _fields_ = [("dtype", C.c_int),
                ("n_dims", C.c_int),
                ("dims", C.c_int * MAX_DIMS),
                ("strides", C.c_int * MAX_DIMS),
                ("data", C.c_void_p),
                ("nbytes", C.c_size_t),
                ("ephemeral", C.c_int),
                ("dbg_force_readback", C.c_int)]


class Node(C.Structure):
    _fields_ = [("op", C.c_int),
                ("inputs", C.POINTER(Tensor) * NODE_MAX_INPUTS),
                ("n_inputs", C.c_int),
                ("output", C.POINTER(Tensor)),
                ("params", C.c_int * 4)]


class Graph(C.Structure):
    _fields_ = [("nodes", Node * GRAPH_MAX_NODES),
                ("n_nodes", C.c_int),
                ("no_readback", C.c_bool)]


assert C.sizeof(Tensor) == 64 and C.sizeof(Node) == 104


def q8_nbytes(nelems):
    """sam3_q8_nbytes (src/core/quant.c:34-37)."""
    return (nelems + Q8_BLOCK - 1) // Q8_BLOCK * Q8_BLOCK_BYTES


def make_tensor(dtype, dims, data_ptr, nbytes=None):
    """Fill a Tensor header the way the reference tests build them by hand
    (tests/test_matmul_q8.c:27-59): row-major strides, non-owning data."""
    t = Tensor()
    t.dtype = dtype
    t.n_dims = len(dims)
    n = 1
    for i, d in enumerate(dims):
        t.dims[i] = d
        n *= d
    for i in range(len(dims), MAX_DIMS):
        t.dims[i] = 1
    s = 1
    for i in reversed(range(len(dims))):
        t.strides[i] = s
        s *= dims[i]
    if dtype == Q8_0:
        # Q8 strides are zeroed by the weight loader (src/core/weight.c:551-555)
        for i in range(MAX_DIMS):
            t.strides[i] = 0
    t.data = data_ptr
    if nbytes is None:
        esz = {F32: 4, F16: 2, BF16: 2, I32: 4, I8: 1}.get(dtype)
        nbytes = q8_nbytes(n) if dtype == Q8_0 else n * esz
    t.nbytes = nbytes
    return t


def make_node(op, inputs, output, params=(0, 0, 0, 0)):
    n = Node()
    n.op = op
    for i, t in enumerate(inputs):
        n.inputs[i] = C.pointer(t) if t is not None else None
    n.n_inputs = len(inputs)
    n.output = C.pointer(output)
    for i, p in enumerate(params):
        n.params[i] = p
    return n


class BackendOps(C.Structure):
    """struct sam3_backend_ops (src/backend/backend.h:31-56)."""
    _fields_ = [("init", C.CFUNCTYPE(C.c_int, C.c_void_p)),
                ("free", C.CFUNCTYPE(None, C.c_void_p)),
                ("alloc_tensor", C.CFUNCTYPE(C.c_int, C.c_void_p, C.POINTER(Tensor))),
                ("graph_eval", C.CFUNCTYPE(C.c_int, C.c_void_p, C.POINTER(Graph))),
                ("arena_reset", C.CFUNCTYPE(None, C.c_void_p)),
                ("cache_invalidate", C.CFUNCTYPE(None, C.c_void_p, C.c_void_p, C.c_size_t))]
