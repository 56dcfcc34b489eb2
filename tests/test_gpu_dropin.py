"""The drop-in boundary from a compiled C++ caller: tests/cpp/dropin_link.cpp includes include/unholy/kernels/*.hpp,
links libunholy_amd.so, runs the reference's native-MXFP4 expert sequence (src/model/forward_ref.hip:455-470)
through the C++ entry points and compares it bit for bit with uh_mx_moe_forward (T = 8 on the grouped GEMV, T = 200
on the grouped GEMM, and T = 64 in the gfx12 verify order: mx_grouped_gemm with max_rows = T, mx_swiglu,
mx_grouped_gemm). The binary is built in-tree by __graft_entry__.build() (tests/cpp/build.sh)."""
import pathlib
import subprocess

import pytest

pytestmark = pytest.mark.gpu

BIN = pathlib.Path(__file__).resolve().parent / "cpp" / "dropin_link"


def test_cpp_dropin_sequence_matches_forward():
    assert BIN.exists(), "build the C++ caller first: tests/cpp/build.sh (run by __graft_entry__.build())"
    r = subprocess.run([str(BIN)], capture_output=True, text=True, timeout=120)
    print(r.stdout, r.stderr)
    assert r.returncode == 0 and "dropin_link: OK" in r.stdout
