"""CPU checks of the drop-in boundary: the built library loads and exports
every symbol include/hawking_hip.h declares, and the Python binding declares
a prototype for each (no compute calls: there is no GPU here)."""
import sys
import os
import re
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "hawking_hip.h")
LIB = os.path.join(ROOT, "hawking_amd", "lib", "libhawking_hip.so")


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    names = re.findall(r"^\s*(?:const\s+)?[A-Za-z_][A-Za-z0-9_]*\s*\**\s+\**(hk_[a-z0-9_]+)\s*\(", text, re.M)
    return sorted(set(names))


def test_header_declares_the_boundary():
    names = declared_functions()
    for must in ("hk_ctx_create", "hk_gemv", "hk_gemv_batch", "hk_decode_rows", "hk_router_softmax_topk", "hk_moe_block",
                 "hk_router_noaux_tc", "hk_moe_decode_layer", "hk_moe_decode_stack", "hk_last_error"):
        assert must in names


@pytest.mark.skipif(not os.path.exists(LIB), reason="library not built (run python -m hawking_amd.build)")
def test_library_exports_every_declared_symbol():
    out = subprocess.run(["nm", "-D", "--defined-only", LIB], capture_output=True, text=True).stdout
    exported = set(re.findall(r"\bT (hk_[a-z0-9_]+)", out))
    assert set(declared_functions()) <= exported
    # Load it with the dynamic loader in a child process: loading the HIP
    # runtime into this (GPU-less) test process and forking afterwards is not
    # safe, so the in-process check stays out of the CPU suite.
    code = ("import ctypes,sys; L=ctypes.CDLL(sys.argv[1]); "
            "m=[n for n in sys.argv[2:] if not hasattr(L,n)]; print(','.join(m)); sys.exit(1 if m else 0)")
    r = subprocess.run([sys.executable, "-c", code, LIB, *declared_functions()], capture_output=True, text=True)
    assert r.returncode == 0, r.stdout + r.stderr


def test_python_binding_covers_the_header():
    from hawking_amd import _lib
    assert set(declared_functions()) == set(_lib.exported_symbols())


@pytest.mark.skipif(not os.path.exists(LIB), reason="library not built")
def test_library_is_gfx950_only(tmp_path):
    fb = tmp_path / "fatbin.bin"
    r = subprocess.run(["objcopy", f"--dump-section", f".hip_fatbin={fb}", LIB], capture_output=True, text=True)
    assert r.returncode == 0, r.stderr
    out = subprocess.run(["/opt/rocm/llvm/bin/clang-offload-bundler", "--list", "--type=o", f"--input={fb}"],
                         capture_output=True, text=True)
    assert out.returncode == 0, out.stderr
    targets = [t for t in out.stdout.split() if "amdgcn" in t]
    assert targets and all(t.endswith("gfx950") for t in targets)


def test_missing_library_fails_loudly(monkeypatch, tmp_path):
    from hawking_amd import _lib
    monkeypatch.setattr(_lib, "LIB_PATH", str(tmp_path / "nope.so"))
    monkeypatch.setattr(_lib, "_lib", None)
    with pytest.raises(RuntimeError, match="not built"):
        _lib.lib()
