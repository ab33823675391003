/*
 * TEST-ONLY stand-in for ggml-backend.h (see ggml.h in this directory): the
 * backend handle types, the device type enum, and the registry functions the
 * adapter calls.
 */
#pragma once

#include "ggml.h"

#ifdef __cplusplus
extern "C" {
#endif

#define GGML_BACKEND_API

typedef struct ggml_backend_buffer_type *ggml_backend_buffer_type_t;
typedef struct ggml_backend_buffer *ggml_backend_buffer_t;
typedef struct ggml_backend *ggml_backend_t;
typedef struct ggml_backend_event *ggml_backend_event_t;
typedef struct ggml_backend_reg *ggml_backend_reg_t;
typedef struct ggml_backend_device *ggml_backend_dev_t;
typedef void *ggml_backend_graph_plan_t;
typedef uint8_t ggml_guid[16];
typedef ggml_guid *ggml_guid_t;

enum ggml_backend_buffer_usage {
  GGML_BACKEND_BUFFER_USAGE_ANY = 0,
  GGML_BACKEND_BUFFER_USAGE_WEIGHTS = 1,
  GGML_BACKEND_BUFFER_USAGE_COMPUTE = 2
};

enum ggml_backend_dev_type {
  GGML_BACKEND_DEVICE_TYPE_CPU,
  GGML_BACKEND_DEVICE_TYPE_GPU,
  GGML_BACKEND_DEVICE_TYPE_IGPU,
  GGML_BACKEND_DEVICE_TYPE_ACCEL
};

struct ggml_backend_dev_caps {
  bool async;
  bool host_buffer;
  bool buffer_from_host_ptr;
  bool events;
};

struct ggml_backend_dev_props {
  const char *name;
  const char *description;
  size_t memory_free;
  size_t memory_total;
  enum ggml_backend_dev_type type;
  struct ggml_backend_dev_caps caps;
};

typedef void (*ggml_backend_set_n_threads_t)(ggml_backend_t backend, int n_threads);

bool ggml_backend_buffer_is_host(ggml_backend_buffer_t buffer);
ggml_backend_t ggml_backend_init_by_type(enum ggml_backend_dev_type type, const char *params);
enum ggml_status ggml_backend_graph_compute(ggml_backend_t backend, struct ggml_cgraph *cgraph);
ggml_backend_dev_t ggml_backend_get_device(ggml_backend_t backend);
ggml_backend_reg_t ggml_backend_dev_backend_reg(ggml_backend_dev_t device);
void *ggml_backend_reg_get_proc_address(ggml_backend_reg_t reg, const char *name);

#ifdef __cplusplus
}
#endif
