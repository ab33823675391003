"""The moe-server protocol v2 structs of the C-ABI on CPU: sizes and field
offsets as nano-glm/lib/moe_proto.h:94-157 fixes them, and the server's
no-device error (the exchanges themselves run in test_gpu_server.py)."""
import ctypes

import pytest

import moe_block as mb


def test_wire_struct_layouts():
    assert ctypes.sizeof(mb.WireHelloRequest) == 24 and mb.WireHelloRequest.payload_bytes.offset == 16
    assert ctypes.sizeof(mb.WireHelloResponse) == 80 and mb.WireHelloResponse.payload_bytes.offset == 72
    assert mb.WireHelloResponse.arch.offset == 16 and mb.WireHelloResponse.expert_scale.offset == 56
    assert ctypes.sizeof(mb.WireRequest) == 40 and mb.WireRequest.payload_bytes.offset == 32
    assert ctypes.sizeof(mb.WireResponse) == 56 and mb.WireResponse.payload_bytes.offset == 48
    assert mb.WireResponse.t_parse_us.offset == 32
    assert mb.WIRE_MAGIC.to_bytes(4, "little") == b"NMOE"


def test_server_open_without_a_device(tmp_path):
    import torch
    if torch.cuda.is_available():
        pytest.skip("a GPU is present; the no-device path is exercised on CPU-only hosts")
    with pytest.raises(mb.MoeError) as ei:
        mb.MoeServer(str(tmp_path / "absent.gguf"))
    assert ei.value.status == mb.MOE_ERR_NO_DEVICE


def test_moe_server_binary_usage_and_no_device(tmp_path):
    """The C++ moe-server: usage on bad arguments (exit 2); on a host without
    a gfx950 device, a clear error (exit 1)."""
    import os
    import subprocess
    exe = os.path.join(os.path.dirname(mb.LIB_PATH), "moe-server")
    assert os.path.exists(exe), "moe-server is built with the library"
    r = subprocess.run([exe], capture_output=True, text=True, timeout=60)
    assert r.returncode == 2 and "Usage: moe-server -m" in r.stderr
    import torch
    if torch.cuda.is_available():
        pytest.skip("a GPU is present")
    r = subprocess.run([exe, "-m", str(tmp_path / "absent.gguf"), "--port", "0"], capture_output=True, text=True,
                       timeout=60)
    assert r.returncode == 1 and "no usable gfx950 device" in r.stderr
