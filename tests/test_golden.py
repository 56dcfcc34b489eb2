"""Golden fixtures (tests/golden/*.npz, written by tests/golden/make_golden.py from the CPU oracle): the oracle must
still reproduce them bit for bit (CPU), and the HIP kernels must match them through the C ABI (GPU)."""
import pathlib

import numpy as np
import pytest

import oracle
from tests.helpers import from_bf16, max_rel

G = pathlib.Path(__file__).resolve().parent / "golden"


def load(name):
    return dict(np.load(G / name, allow_pickle=False))


def test_oracle_reproduces_mx_gemv():
    f = load("mx_gemv.npz")
    q, qs = oracle.act_quant_fp8(f["x"])
    assert np.array_equal(q, f["q"]) and np.array_equal(qs, f["qs"])
    tw, ts = oracle.repack(f["w"], f["s"], 64, 512)
    assert np.array_equal(tw, f["tw"]) and np.array_equal(ts, f["ts"])
    y16, y32 = oracle.gemm_a8w4(q, qs, f["w"], f["s"], 64)
    assert np.array_equal(y16, f["y16"]) and np.array_equal(y32, f["y32"])


def test_oracle_reproduces_routing():
    f = load("routing.npz")
    sel, wt = oracle.route_softmax(f["logits"], 6)
    assert np.array_equal(sel, f["sel"]) and np.array_equal(wt, f["wt"])
    d = oracle.dispatch(sel, wt, 256, tile_rows=16)
    for k in ("eidx", "ewt", "row_expert", "pidx", "tiles", "plan"):
        assert np.array_equal(d[k], f[k]), k


def _experts(f, E=8):
    return [{k: f[f"{k}_{e}"] for k in ("w1", "s1", "w3", "s3", "w2", "s2")} for e in range(E)]


def test_oracle_reproduces_moe_ffn():
    f = load("moe_ffn.npz")
    sel, wt = oracle.route_softmax(f["logits"], 3)
    assert np.array_equal(sel, f["sel"])
    out, pair = oracle.moe_forward(f["x"], sel, wt, _experts(f), 256, 128, 10.0)
    assert np.array_equal(out, f["out"]) and np.array_equal(pair, f["pair"])


def test_oracle_reproduces_fp8_dense():
    f = load("fp8_dense.npz")
    aq, sa = oracle.act_quant_fp8_f32s(f["a"])
    assert np.array_equal(aq, f["aq"]) and np.array_equal(sa, f["sa"])
    c16, c32 = oracle.gemm_w8a8(aq, sa, f["wq"], f["sw"])
    assert np.array_equal(c16, f["c16"]) and np.array_equal(c32, f["c32"])


# ---- the kernels against the fixtures ---------------------------------------------------------------------------------
@pytest.mark.gpu
def test_gpu_matches_golden():
    from unholy_amd import call
    from unholy_amd.device import DeviceBuffer, pointer_table, synchronize

    def dev(a):
        return DeviceBuffer.from_array(np.ascontiguousarray(a))

    f = load("mx_gemv.npz")
    q, qs = DeviceBuffer(3 * 512), DeviceBuffer(3 * 4)
    call("uh_act_quant_fp8", dev(f["x"]), 512, q, qs, 3, 512, 128, None)
    assert np.array_equal(q.download((3, 512), np.uint8), f["q"])
    tw, ts = DeviceBuffer(64 * 256), DeviceBuffer(64 * 16)
    call("uh_mx_repack_to", dev(f["w"]), dev(f["s"]), tw, ts, 64, 512, None)
    assert np.array_equal(tw.download(f["tw"].shape, np.uint8), f["tw"])
    wtab, stab = pointer_table([tw]), pointer_table([ts])
    out = DeviceBuffer(3 * 64 * 2)
    tiles = dev(np.array([[0, 0, 3]], np.int32))
    call("uh_mx_grouped_gemv_q", q, qs, 512, tiles, 1, wtab, stab, out, 64, 64, None, None, None, None, None, 16,
         None, None, None, None, None, None, 0.0)
    y = out.download((3, 64), np.uint16)
    assert max_rel(from_bf16(y), from_bf16(f["y16"])) <= 1e-2

    f = load("moe_ffn.npz")
    ex = _experts(f)
    bufs = [dev(e[k]) for k in ("w1", "s1", "w3", "s3", "w2", "s2") for e in ex]
    tab = pointer_table(bufs)
    T, E, K, D, I = 5, 8, 3, 256, 128
    ws_bytes = call("uh_mx_moe_workspace_size", T, K, E, D, I)
    ws, out = DeviceBuffer(ws_bytes), DeviceBuffer(T * D * 2)
    sel = DeviceBuffer(T * K * 4)
    call("uh_mx_moe_forward", dev(f["x"]), dev(f["logits"]), T, K, E, D, I, tab, 10.0, ws, ws_bytes, out, sel,
         None, None)
    synchronize()
    assert np.array_equal(sel.download((T, K), np.int32), f["sel"])
    assert max_rel(from_bf16(out.download((T, D), np.uint16)), from_bf16(f["out"])) <= 1e-2

    f = load("fp8_dense.npz")
    c = DeviceBuffer(2 * 256 * 2)
    call("uh_gemm_fp8_f32s", dev(f["aq"]), dev(f["sa"]), dev(f["wq"]), dev(f["sw"]), c, 256, 2, 256, 256, None)
    assert max_rel(from_bf16(c.download((2, 256), np.uint16)), from_bf16(f["c16"])) <= 1e-2
