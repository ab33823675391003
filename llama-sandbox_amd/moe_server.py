"""moe-server for nano-glm's trunk, backed by the gfx950 MoE block.

    python llama-sandbox_amd/moe_server.py -m <first-file.gguf> [--host 127.0.0.1] [--port 5711]

Speaks protocol v2 (nano-glm/lib/moe_proto.h:45-157): a hello per
connection, then one request per MoE layer and batch, answered with the
routed experts' combined rows.  The options follow nano-glm's moe-server
(nano-glm/apps/moe-server/main.cpp:73-96) where they apply to one GPU.
"""
import argparse
import os
import sys

sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))
import moe_block as mb  # noqa: E402


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("-m", dest="model", required=True, help="GGUF model (first file of a split model)")
    ap.add_argument("--host", default="127.0.0.1", help="bind address (default 127.0.0.1)")
    ap.add_argument("--port", type=int, default=5711, help="port (default 5711, 0 = any free port)")
    ap.add_argument("--device", type=int, default=0, help="GPU (default 0)")
    ap.add_argument("--budget-mb", type=int, default=-1, help="cap on resident expert bytes (default: none)")
    a = ap.parse_args(argv)
    budget = 2 ** 64 - 1 if a.budget_mb < 0 else a.budget_mb << 20
    with mb.MoeServer(a.model, a.device, budget) as srv:
        port = srv.listen(a.host, a.port)
        print(f"moe-server: listening on {a.host}:{port}", file=sys.stderr, flush=True)
        srv.serve(-1)
    return 0


if __name__ == "__main__":
    sys.exit(main())
