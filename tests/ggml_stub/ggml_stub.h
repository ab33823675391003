// TEST-ONLY: what the driver of the backend adapter needs from the stand-in
// ggml runtime (ggml_stub.cpp) beyond ggml's own declarations.
#pragma once

#include "ggml-backend-impl.h"
#include "ggml.h"

#define STUB_NOT_CONTIGUOUS 0x1000   // a ggml_tensor flag bit of the stand-in: ggml_is_contiguous() is false
#define STUB_CPU_SENTINEL 12345.0f   // what the fake CPU delegate writes into a split's MUL node

extern "C" {
struct ggml_cgraph *stub_graph(struct ggml_tensor **nodes, int n);
void stub_graph_free(struct ggml_cgraph *g);
extern int stub_cpu_calls;
extern int stub_cpu_threads;
}
