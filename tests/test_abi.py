"""CPU-side checks of the C-ABI library: it is built, loads, and exports every
entry point include/moe_block.h declares.  No compute calls (no GPU here)."""
import ctypes
import os
import re
import subprocess

import pytest

import moe_block as mb

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(REPO, "include", "moe_block.h")


def declared_functions():
    src = open(HEADER).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    return sorted(set(re.findall(r"\b(moe_[a-z0-9_]+)\s*\(", src)))


def test_header_declares_the_binding_exports():
    assert declared_functions() == sorted(mb.EXPORTS)


def test_library_exports_every_declared_symbol():
    lib = ctypes.CDLL(mb.LIB_PATH)
    for name in declared_functions():
        assert hasattr(lib, name), name
    out = subprocess.run(["nm", "-D", "--defined-only", mb.LIB_PATH], capture_output=True, text=True,
                         check=True).stdout
    exported = {line.split()[-1] for line in out.splitlines() if " T " in line}
    missing = [n for n in declared_functions() if n not in exported]
    assert not missing, missing


def test_library_is_gfx950_only():
    # the offload bundle ids embedded in our own build name every GPU target
    blob = open(mb.LIB_PATH, "rb").read()
    targets = set(re.findall(rb"amdgcn-amd-amdhsa--(gfx[0-9a-z]+)", blob))
    assert targets == {b"gfx950"}, targets


def test_status_strings_and_no_device_error():
    lib = mb.load_library()
    assert lib.moe_status_str(mb.MOE_ERR_OUT_OF_BUDGET).decode().startswith("layer does not fit")
    assert lib.moe_status_str(0).decode() == "ok"
    import torch
    if torch.cuda.is_available():
        pytest.skip("a GPU is present; the no-device path is exercised on CPU-only hosts")
    with pytest.raises(mb.MoeError) as ei:
        mb.MoeBlock(0)
    assert ei.value.status == mb.MOE_ERR_NO_DEVICE


def test_product_binding_does_not_import_the_oracle():
    pkg = os.path.join(REPO, "llama-sandbox_amd")
    for root, _, files in os.walk(pkg):
        for f in files:
            if f.endswith((".py", ".hip", ".h", ".cpp")):
                text = open(os.path.join(root, f)).read()
                assert "import oracle" not in text and "moe_oracle" not in text, f


def test_header_is_c99_and_links(tmp_path):
    """include/moe_block.h is a C header: a C99 program (-pedantic -Werror)
    includes it, links against the library and sees the wire structs at the
    protocol's sizes."""
    src = tmp_path / "use.c"
    src.write_text('#include "moe_block.h"\n#include <stdio.h>\n'
                   "int main(void) {\n"
                   "  moe_node n = {0}; moe_split s = {0}; moe_gguf_layer g = {0}; (void)s; (void)g;\n"
                   "  printf(\"%zu %zu %zu %zu %d\\n\", sizeof(moe_wire_hello_request), sizeof(moe_wire_hello_response),\n"
                   "         sizeof(moe_wire_request), sizeof(moe_wire_response), n.op);\n"
                   "  return moe_status_str(MOE_ERR_FORMAT)[0] == 0;\n}\n")
    exe = tmp_path / "use"
    libdir = os.path.dirname(mb.LIB_PATH)
    subprocess.run(["gcc", "-std=c99", "-Wall", "-Wextra", "-pedantic", "-Werror", "-I", os.path.join(REPO, "include"),
                    str(src), "-o", str(exe), "-L", libdir, "-lmoe_block", f"-Wl,-rpath,{libdir}"], check=True)
    r = subprocess.run([str(exe)], capture_output=True, text=True, check=True)
    assert r.stdout.split() == ["24", "80", "40", "56", "0"]
