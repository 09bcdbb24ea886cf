/*
 * include/sam3_hip_abi.h - sam3.c types that cross the HIP backend boundary.
 *
 * The HIP backend is a drop-in for sam3.c's backend vtable, so it takes
 * the very structs sam3.c's graph builder hands to every backend. When
 * this header is compiled inside sam3.c (its own headers already
 * included: SAM3_BACKEND_H is defined), sam3.c's definitions are used
 * unchanged. Standalone, this header declares the same types with the
 * same names, field order and sizes:
 *
 *   enum sam3_error, enum sam3_dtype   include/sam3/sam3_types.h:25-54
 *   struct sam3_tensor                 src/core/tensor.h:24-49
 *   enum sam3_op, struct sam3_node     src/core/graph.h:27-83
 *   struct sam3_graph                  src/core/graph.h:86-90
 *   struct sam3_backend(_ops)          src/backend/backend.h:23-62
 *   struct sam3_q8_block (36 bytes)    src/core/quant.h:22-33
 *
 * (paths relative to the sam3.c source tree)
 */
#ifndef SAM3_HIP_ABI_H
#define SAM3_HIP_ABI_H

#include <stdbool.h>
#include <stddef.h>
#include <stdint.h>

#ifndef SAM3_BACKEND_H /* sam3.c's own headers not included: declare them */

#define SAM3_MAX_DIMS 4
#define SAM3_GRAPH_MAX_NODES 16384
#define SAM3_NODE_MAX_INPUTS 8
#define SAM3_DTYPE_COUNT 6
#define SAM3_Q8_BLOCK_SIZE 32

enum sam3_error {
	SAM3_OK       =  0,
	SAM3_EINVAL   = -1,
	SAM3_ENOMEM   = -2,
	SAM3_EIO      = -3,
	SAM3_EBACKEND = -4,
	SAM3_EMODEL   = -5,
	SAM3_EDTYPE   = -6,
	SAM3_EVIDEO   = -7,
};

enum sam3_dtype {
	SAM3_DTYPE_F32,
	SAM3_DTYPE_F16,
	SAM3_DTYPE_BF16,
	SAM3_DTYPE_I32,
	SAM3_DTYPE_I8,
	SAM3_DTYPE_Q8_0,
};

struct sam3_tensor {
	enum sam3_dtype dtype;
	int             n_dims;
	int             dims[SAM3_MAX_DIMS];
	int             strides[SAM3_MAX_DIMS];
	void           *data;
	size_t          nbytes;
	int             ephemeral;
	int             dbg_force_readback;
};

enum sam3_op {
	SAM3_OP_NONE,
	SAM3_OP_MATMUL,
	SAM3_OP_ADD,
	SAM3_OP_MUL,
	SAM3_OP_SOFTMAX,
	SAM3_OP_RELU,
	SAM3_OP_GELU,
	SAM3_OP_LAYERNORM,
	SAM3_OP_CONV2D,
	SAM3_OP_RESHAPE,
	SAM3_OP_TRANSPOSE,
	SAM3_OP_CAST,
	SAM3_OP_CONCAT,
	SAM3_OP_SLICE,
	SAM3_OP_EMBED,
	SAM3_OP_SIGMOID,
	SAM3_OP_UPSAMPLE,
	SAM3_OP_ROPE,
	SAM3_OP_SILU,
	SAM3_OP_CONV_TRANSPOSE2D,
	SAM3_OP_MAXPOOL2D,
	SAM3_OP_SDPA,
	SAM3_OP_BIAS_ADD,
	SAM3_OP_GROUPNORM,
	SAM3_OP_BATCHNORM,
	SAM3_OP_HSWISH,
	SAM3_OP_DIV,
	SAM3_OP_COUNT,
};

struct sam3_node {
	enum sam3_op         op;
	struct sam3_tensor  *inputs[SAM3_NODE_MAX_INPUTS];
	int                  n_inputs;
	struct sam3_tensor  *output;
	int                  params[4];
};

struct sam3_graph {
	struct sam3_node nodes[SAM3_GRAPH_MAX_NODES];
	int              n_nodes;
	bool             no_readback;
};

enum sam3_backend_type {
	SAM3_BACKEND_CPU,
	SAM3_BACKEND_METAL,
};

struct sam3_backend;

struct sam3_backend_ops {
	enum sam3_error (*init)(struct sam3_backend *be);
	void (*free)(struct sam3_backend *be);
	enum sam3_error (*alloc_tensor)(struct sam3_backend *be,
				       struct sam3_tensor *t);
	enum sam3_error (*graph_eval)(struct sam3_backend *be,
				     struct sam3_graph *g);
	void (*arena_reset)(struct sam3_backend *be);
	void (*cache_invalidate)(struct sam3_backend *be,
				 const void *start, size_t len);
};

struct sam3_backend {
	enum sam3_backend_type         type;
	const struct sam3_backend_ops *ops;
};

struct sam3_q8_block {
	float  scale;
	int8_t data[SAM3_Q8_BLOCK_SIZE];
};

struct sam3_arena;

#endif /* !SAM3_BACKEND_H */

#endif /* SAM3_HIP_ABI_H */
