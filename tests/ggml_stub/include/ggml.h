/*
 * TEST-ONLY stand-in for ggml.h: declares just the ggml types, fields and
 * functions that llama-sandbox_amd/ggml_backend/moe_ggml_backend.cpp uses, so
 * that the adapter compiles and runs in this image, which has no ggml tree.
 * Names follow ggml's public API (ggml 0.18.1, commit 6a32c29a7, the version
 * the reference builds against); enum VALUES here are this stand-in's own and
 * are not ggml's ABI.  A real build of the adapter uses ggml's own headers.
 */
#pragma once

#include <stddef.h>
#include <stdint.h>

#define GGML_MAX_DIMS 4
#define GGML_MAX_SRC 10
#define GGML_MAX_OP_PARAMS 64
#define GGML_MAX_NAME 64
#define GGML_UNUSED(x) (void)(x)
#define GGML_ASSERT(x)   \
  do {                   \
    if (!(x)) __builtin_trap(); \
  } while (0)

#ifdef __cplusplus
extern "C" {
#endif

enum ggml_type {
  GGML_TYPE_F32 = 0,
  GGML_TYPE_F16 = 1,
  GGML_TYPE_I32 = 26,
  GGML_TYPE_BF16 = 30,
  GGML_TYPE_MXFP4 = 39,
  GGML_TYPE_COUNT = 40
};

enum ggml_op {
  GGML_OP_NONE = 0,
  GGML_OP_ADD,
  GGML_OP_MUL,
  GGML_OP_MUL_MAT,
  GGML_OP_MUL_MAT_ID,
  GGML_OP_RESHAPE,
  GGML_OP_VIEW,
  GGML_OP_PERMUTE,
  GGML_OP_TRANSPOSE,
  GGML_OP_CLAMP,
  GGML_OP_GLU,
  GGML_OP_SOFT_MAX,
  GGML_OP_COUNT
};

enum ggml_glu_op {
  GGML_GLU_OP_REGLU = 0,
  GGML_GLU_OP_GEGLU = 1,
  GGML_GLU_OP_SWIGLU = 2,
  GGML_GLU_OP_COUNT
};

enum ggml_status {
  GGML_STATUS_ALLOC_FAILED = -2,
  GGML_STATUS_FAILED = -1,
  GGML_STATUS_SUCCESS = 0,
  GGML_STATUS_ABORTED = 1
};

struct ggml_backend_buffer;

struct ggml_tensor {
  enum ggml_type type;
  struct ggml_backend_buffer *buffer;
  int64_t ne[GGML_MAX_DIMS];
  size_t nb[GGML_MAX_DIMS];
  enum ggml_op op;
  int32_t op_params[GGML_MAX_OP_PARAMS / sizeof(int32_t)];
  int32_t flags;
  struct ggml_tensor *src[GGML_MAX_SRC];
  struct ggml_tensor *view_src;
  size_t view_offs;
  void *data;
  char name[GGML_MAX_NAME];
  void *extra;
  char padding[8];
};

struct ggml_cgraph;

const char *ggml_get_name(const struct ggml_tensor *tensor);
size_t ggml_nbytes(const struct ggml_tensor *tensor);
bool ggml_is_contiguous(const struct ggml_tensor *tensor);
enum ggml_glu_op ggml_get_glu_op(const struct ggml_tensor *tensor);
const char *ggml_op_name(enum ggml_op op);
int ggml_graph_n_nodes(struct ggml_cgraph *cgraph);
struct ggml_tensor *ggml_graph_node(struct ggml_cgraph *cgraph, int i);

#ifdef __cplusplus
}
#endif
