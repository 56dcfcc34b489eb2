"""The C ABI without a GPU: the library loads, exports every symbol include/unholy_amd.h declares and the C++ drop-in
entry points of include/unholy/kernels/*.hpp, and rejects invalid shapes with a message before touching the device."""
import ctypes
import pathlib
import re
import subprocess

import pytest

from unholy_amd import _lib

ROOT = pathlib.Path(__file__).resolve().parents[1]


def test_library_exports_every_declared_symbol():
    protos = _lib.parse_header()
    assert len(protos) >= 50
    lib = _lib.lib()  # binds every prototype; a missing export raises here
    for name in protos:
        assert hasattr(lib, name)


def _exported_cpp():
    out = subprocess.run(["nm", "-D", "-C", "--defined-only", str(_lib.LIB_PATH)], capture_output=True, text=True,
                         check=True).stdout
    return out


def test_cpp_drop_in_entry_points_exported():
    syms = _exported_cpp()
    names = set()
    for hdr in (ROOT / "include" / "unholy" / "kernels").glob("*.hpp"):
        text = re.sub(r"//[^\n]*", "", hdr.read_text())
        for m in re.finditer(r"^(?:void|int|bool|unsigned long long)\s+(\w+)\s*\(", text, flags=re.M):
            names.add(m.group(1))
    assert {"mx_repack", "mx_grouped_gemv", "mx_grouped_gemm", "moe_scatter", "gemm_w8a8", "route"} <= names
    for n in names:
        assert re.search(rf"unholy::kernels::{n}\(", syms), n


@pytest.mark.parametrize("call", [
    ("uh_mx_grouped_gemv_q", (8, 8, 100, 8, 1, 8, 8, 8, 16, 16, None, None, None, None, None, 1,
                              None, None, None, None, None, None, 0.0), "K % 128"),
    ("uh_mx_repack_to", (None, None, None, None, 15, 64, None), "N % 16"),
    ("uh_act_quant_fp8", (None, 128, None, None, 2, 128, 48, None), "block"),
    ("uh_moe_plan", (None, None, 2000, 1, None, None, None, None, None, 1, None, 128), "E must be"),
    ("uh_moe_dispatch_small", (None, None, 40, 6, 256, 240, 300, 16, None, None, None, None, None, None, None, None,
                               None, 0.0, None, None, None, None, None, 0, None), "T <= 32"),
])
def test_shape_errors_are_reported(call):
    name, args, msg = call
    f = getattr(_lib.lib(), name)
    rc = f(*args)
    assert rc == -1
    assert msg in _lib.last_error()


def test_cpp_dropin_caller_compiles_and_links(tmp_path):
    """A C++ caller compiles against include/unholy/kernels/*.hpp and links every drop-in symbol it uses from
    libunholy_amd.so (tests/cpp/build.sh into a temporary path; running it needs a GPU: tests/test_gpu_dropin.py)."""
    import subprocess
    root = pathlib.Path(__file__).resolve().parent.parent
    out = tmp_path / "dropin_link"
    r = subprocess.run([str(root / "tests" / "cpp" / "build.sh"), str(out)], capture_output=True, text=True,
                       timeout=300)
    assert r.returncode == 0, r.stderr[-2000:]
    assert out.exists()
