"""GPU parity of the fused activation producers: rmsnorm_quant_slices (rmsnorm + act_quant_fp8 in one launch) and
quant_remote_tokens (act_quant_fp8 of gathered rows below a device-side count), bit-exact against the CPU oracle."""
import ctypes

import numpy as np
import pytest

import oracle
from tests.helpers import randn_bf16
from unholy_amd import call
from unholy_amd.device import DeviceBuffer

pytestmark = pytest.mark.gpu


def dev(a):
    return DeviceBuffer.from_array(np.ascontiguousarray(a))


# (rows, dim, pad): slices per row = clamp(64 / rows, 1, dim / 256) -> 16, 8, 1, 28, 4 and 4 of them; an odd row
# stride (pad 3) takes the one-value-per-thread path, the others the 16-byte one.
@pytest.mark.parametrize("rows,dim,pad", [(1, 4096, 0), (8, 4096, 64), (300, 4096, 0), (1, 7168, 0), (16, 1024, 8),
                                          (16, 1024, 3)])
def test_rmsnorm_quant_slices_bit_exact(rows, dim, pad):
    rng = np.random.default_rng(rows + dim)
    ld = dim + pad
    x = randn_bf16(rng, (rows, ld), scale=3.0)
    w = randn_bf16(rng, (dim,))
    x[0, :128] = 0  # an all-zero input block (a zero output block: the 1e-4 amax floor)
    eps = 1e-6
    y_ref, q_ref, qs_ref = oracle.rmsnorm_quant(np.ascontiguousarray(x[:, :dim]), w, eps)
    y = DeviceBuffer(rows * ld * 2)
    q, qs = DeviceBuffer(rows * dim), DeviceBuffer(rows * dim // 128)
    launched = ctypes.c_int(-1)
    call("uh_rmsnorm_quant_slices", dev(x), ld, dev(w), y, ld, q, qs, rows, dim, eps, ctypes.byref(launched), None)
    assert launched.value == 1
    got = y.download((rows, ld), np.uint16)[:, :dim]
    print(f"rmsnorm_quant rows={rows} dim={dim}: y bit-identical {np.mean(got == y_ref):.6f}")
    assert np.array_equal(got, y_ref)
    assert np.array_equal(q.download((rows, dim), np.uint8), q_ref)
    assert np.array_equal(qs.download((rows, dim // 128), np.uint8), qs_ref)


def test_rmsnorm_quant_slices_applicability():
    """Where the reference's returns false, nothing is launched; without q only y is written."""
    rng = np.random.default_rng(5)
    x, w = randn_bf16(rng, (4, 1000)), randn_bf16(rng, (1000,))
    dx, dw = dev(x), dev(w)
    launched = ctypes.c_int(-1)
    call("uh_rmsnorm_quant_slices", dx, 1000, dw, DeviceBuffer(8000), 1000, None, None, 4, 1000, 1e-6,
         ctypes.byref(launched), None)
    assert launched.value == 0  # 1000 values: not whole 256-value slices
    x2 = randn_bf16(rng, (2, 512))
    dx2 = dev(x2)
    call("uh_rmsnorm_quant_slices", dx2, 512, dev(w[:512]), dx2, 512, None, None, 2, 512, 1e-6,
         ctypes.byref(launched), None)
    assert launched.value == 0  # in place
    y = DeviceBuffer(2 * 512 * 2)
    call("uh_rmsnorm_quant_slices", dx2, 512, dev(w[:512]), y, 512, None, None, 2, 512, 1e-6,
         ctypes.byref(launched), None)
    assert launched.value == 1
    assert np.array_equal(y.download((2, 512), np.uint16), oracle.rmsnorm_quant(x2, w[:512], 1e-6, quant=False))


@pytest.mark.parametrize("U,T,dim", [(17, 40, 4096), (1, 1, 1024), (0, 8, 512), (32, 32, 7168)])
def test_quant_remote_tokens(U, T, dim):
    rng = np.random.default_rng(U * 3 + T)
    x = randn_bf16(rng, (T, dim), scale=2.0)
    u2t = np.sort(rng.choice(T, size=U, replace=False)).astype(np.int32) if U else np.zeros(1, np.int32)
    plan = np.array([6 * T, 0, 0, 0, U], np.int32)  # P, remote0, local tiles, remote tiles, n_remote_tokens
    q = dev(np.full((T, dim), 0xAB, np.uint8))
    s = dev(np.full((T, dim // 128), 0xCD, np.uint8))
    call("uh_quant_remote_tokens", dev(x), dim, dev(u2t), dev(plan), q, s, T, None)
    qg, sg = q.download((T, dim), np.uint8), s.download((T, dim // 128), np.uint8)
    if U:
        q_ref, s_ref = oracle.act_quant_fp8(x[u2t])
        assert np.array_equal(qg[:U], q_ref)
        assert np.array_equal(sg[:U], s_ref)
    assert (qg[U:] == 0xAB).all() and (sg[U:] == 0xCD).all()  # rows past the device count untouched


@pytest.mark.parametrize("rows,dim", [(1, 4096), (8, 1000), (300, 4096), (3, 7168), (16, 130)])
def test_rmsnorm_slices(rows, dim):
    """rmsnorm_slices (any dim, no quantization) bit-exact against the oracle."""
    rng = np.random.default_rng(rows * 7 + dim)
    x, w = randn_bf16(rng, (rows, dim), scale=2.0), randn_bf16(rng, (dim,))
    y = DeviceBuffer(rows * dim * 2)
    call("uh_rmsnorm_slices", dev(x), dim, dev(w), y, dim, rows, dim, 1e-6, None)
    assert np.array_equal(y.download((rows, dim), np.uint16), oracle.rmsnorm_quant(x, w, 1e-6, quant=False))


@pytest.mark.parametrize("T,hc,dim,inplace", [(8, 4, 4096, False), (8, 4, 4096, True), (3, 2, 1000, True),
                                              (40, 1, 512, False)])
def test_hc_post_slices(T, hc, dim, inplace):
    rng = np.random.default_rng(T + hc + dim)
    x, res = randn_bf16(rng, (T, dim)), randn_bf16(rng, (T, hc, dim))
    post = rng.random((T, hc)).astype(np.float32)
    comb = rng.random((T, hc, hc)).astype(np.float32)
    dres = dev(res)
    out = dres if inplace else DeviceBuffer(res.nbytes)
    call("uh_hc_post_slices", dev(x), dres, dev(post), dev(comb), out, T, hc, dim, None)
    assert np.array_equal(out.download(res.shape, np.uint16), oracle.hc_post(x, res, post, comb))


def test_moe_trace():
    rng = np.random.default_rng(2)
    sel = rng.integers(0, 256, 6 * 37, dtype=np.int32)
    dst = DeviceBuffer(sel.size)
    call("uh_moe_trace", dev(sel), sel.size, dst, None)
    assert np.array_equal(dst.download(sel.size, np.uint8), sel.astype(np.uint8))
