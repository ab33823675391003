// moe-server: nano-glm's MoE backend on the gfx950 MoE block.
//
//   moe-server -m <first-file.gguf> [--host 127.0.0.1] [--port 5711] [--device 0] [--budget-mb N]
//
// Serves protocol v2 (nano-glm/lib/moe_proto.h:45-157) through the library's
// moe_server_* entry points; the options follow nano-glm's moe-server
// (nano-glm/apps/moe-server/main.cpp:73-96) where they apply to one GPU.
#include "../../include/moe_block.h"

#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <string>

int main(int argc, char **argv) {
  std::string model, host = "127.0.0.1";
  int port = 5711, device = 0;
  long long budget_mb = -1;
  for (int i = 1; i < argc; i++) {
    const char *a = argv[i];
    if (!strcmp(a, "-m") && i + 1 < argc) model = argv[++i];
    else if (!strcmp(a, "--host") && i + 1 < argc) host = argv[++i];
    else if (!strcmp(a, "--port") && i + 1 < argc) port = atoi(argv[++i]);
    else if (!strcmp(a, "--device") && i + 1 < argc) device = atoi(argv[++i]);
    else if (!strcmp(a, "--budget-mb") && i + 1 < argc) budget_mb = atoll(argv[++i]);
    else {
      model.clear();
      break;
    }
  }
  if (model.empty()) {
    fprintf(stderr,
            "Usage: moe-server -m <first-file.gguf> [options]\n"
            "  --host <ip>        bind address (default 127.0.0.1)\n"
            "  --port <n>         port (default 5711; 0 = any free port)\n"
            "  --device <n>       GPU (default 0)\n"
            "  --budget-mb <n>    cap on resident expert bytes (default: none)\n");
    return 2;
  }
  const uint64_t budget = budget_mb < 0 ? UINT64_MAX : (uint64_t)budget_mb << 20;
  moe_server *srv = nullptr;
  char err[512];
  moe_status st = moe_server_open(model.c_str(), device, budget, &srv, err, sizeof err);
  if (st != MOE_OK) {
    fprintf(stderr, "moe-server: %s: %s\n", moe_status_str(st), err);
    return 1;
  }
  int bound = 0;
  st = moe_server_listen(srv, host.c_str(), port, &bound);
  if (st != MOE_OK) {
    fprintf(stderr, "moe-server: %s\n", moe_server_last_error(srv));
    moe_server_close(srv);
    return 1;
  }
  fprintf(stderr, "moe-server: listening on %s:%d\n", host.c_str(), bound);
  st = moe_server_serve(srv, -1);
  if (st != MOE_OK) fprintf(stderr, "moe-server: %s\n", moe_server_last_error(srv));
  moe_server_close(srv);
  return st == MOE_OK ? 0 : 1;
}
