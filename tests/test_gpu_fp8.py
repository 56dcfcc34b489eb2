"""GPU parity of the fp8 e4m3 block-scaled dense GEMM / GEMV and the reference-order a8w4 GEMM."""
import numpy as np
import pytest

import oracle
from tests.helpers import from_bf16, max_rel, mx_weights, randn_bf16, rel_l2
from unholy_amd import call
from unholy_amd.device import DeviceBuffer

pytestmark = pytest.mark.gpu


def dev(a):
    return DeviceBuffer.from_array(np.ascontiguousarray(a))


def _weights_f32s(rng, N, K):
    w = (rng.standard_normal((N, K), dtype=np.float32) * np.float32(0.02)).astype(np.float32)
    dw = dev(w)
    q, s = DeviceBuffer(N * K), DeviceBuffer(((N + 127) // 128) * (K // 128) * 4)
    call("uh_quant_weight_fp8_f32s", dw, q, s, N, K, None)
    return q.download((N, K), np.uint8), s.download(((N + 127) // 128, K // 128), np.float32), w


# 16 < M <= 256 with N % 32 == 0 takes the row-tile kernel: one to four 2,048-input chunks, ragged last chunks (K = 640,
# 2,176), one 32-column block (N = 32), a weight-scale row shared by fewer than 128 columns (N = 96), 1 to 8 row tiles;
# (200, 4096, 1024): the 64-column form over 7 row tiles. Past 256 rows the tiled GEMM, whose last row tile leaves a
# wave one or no live 32-row block: 300 (44 rows), 400 (16 rows), 480 (96 rows).
@pytest.mark.parametrize("M,N,K", [(1, 4096, 4096), (5, 384, 1024), (64, 512, 1024), (300, 256, 512), (3, 136, 384),
                                   (1000, 768, 1024), (129, 200, 256), (17, 32, 640), (33, 1024, 8192), (64, 96, 6144),
                                   (48, 256, 2176), (40, 200, 512), (200, 128, 1024), (256, 96, 2176), (129, 64, 384),
                                   (200, 4096, 1024), (400, 256, 512), (480, 384, 768)])
def test_fp8_f32_scales(M, N, K):
    """BASELINE config 4 form: A bf16 -> e4m3 per 1x128 with fp32 scales; W e4m3 with fp32 128x128 scales."""
    rng = np.random.default_rng(M + N)
    x = randn_bf16(rng, (M, K))
    wq, ws, w = _weights_f32s(rng, N, K)
    # the weight quantizer against its definition: s = max(amax, 1e-4) * fp32(1/448), codes e4m3(w / s)
    blk = np.abs(w[:128, :128]).max()
    assert ws[0, 0] == np.float32(max(blk, np.float32(1e-4))) * np.float32(1.0 / 448.0)
    q, sa = DeviceBuffer(M * K), DeviceBuffer(M * (K // 128) * 4)
    call("uh_act_quant_fp8_f32s", dev(x), K, q, sa, M, K, 128, None)
    q_ref, sa_ref = oracle.act_quant_fp8_f32s(x)
    assert np.array_equal(q.download((M, K), np.uint8), q_ref)
    assert np.array_equal(sa.download((M, K // 128), np.float32), sa_ref)
    c = DeviceBuffer(M * N * 2)
    call("uh_gemm_fp8_f32s", q, sa, dev(wq), dev(ws), c, N, M, N, K, None)
    got = from_bf16(c.download((M, N), np.uint16))
    ref16, _ = oracle.gemm_w8a8(q_ref, sa_ref, wq, ws)
    ref64 = oracle.gemm_w8a8_f64(q_ref, sa_ref, wq, ws)
    mr = max_rel(got, from_bf16(ref16))
    print(f"fp8 f32s M={M}: max_rel {mr:.3e} rel_l2 {rel_l2(got, from_bf16(ref16)):.3e} "
          f"vs f64 {max_rel(got, ref64):.3e}")
    assert mr <= 1e-2


@pytest.mark.parametrize("M,N,K,pad", [(1, 4096, 4096, 0), (5, 136, 384, 64), (16, 1024, 1024, 8), (3, 200, 256, 0)])
def test_fp8_f32s_fused_quant_is_bit_identical(M, N, K, pad):
    """gemm_fp8_f32s_x (act_quant_fp8_f32s fused into the GEMV, M <= 16) against the two calls it replaces: the same
    bf16 outputs bit for bit, also with a row stride wider than K and a ragged N; and past 16 rows it refuses."""
    rng = np.random.default_rng(7 * M + N)
    ldx = K + pad
    x = randn_bf16(rng, (M, ldx))
    x[:, 0:128] = 0  # an all-zero block: the 1e-4 amax floor
    x[0, 130] = np.uint16(0x4480)  # 1024.0: a block whose scale a single value sets
    wq, ws, _ = _weights_f32s(rng, N, K)
    dx, dwq, dws = dev(x), dev(wq), dev(ws)
    q, sa = DeviceBuffer(M * K), DeviceBuffer(M * (K // 128) * 4)
    call("uh_act_quant_fp8_f32s", dx, ldx, q, sa, M, K, 128, None)
    c_ref = DeviceBuffer(M * N * 2)
    call("uh_gemm_fp8_f32s", q, sa, dwq, dws, c_ref, N, M, N, K, None)
    c = DeviceBuffer(M * N * 2)
    call("uh_gemm_fp8_f32s_x", dx, ldx, dwq, dws, c, N, M, N, K, None)
    got, ref = c.download((M, N), np.uint16), c_ref.download((M, N), np.uint16)
    print(f"fp8 f32s fused M={M} N={N} K={K}: bit-identical fraction {np.mean(got == ref):.6f}")
    assert np.array_equal(got, ref)
    with pytest.raises(Exception, match="M <= 16"):
        call("uh_gemm_fp8_f32s_x", dx, ldx, dwq, dws, c, N, 17, N, K, None)


# (40, 16384, 2048) and (48, 20480, 1152) leave >= 512 workgroups of 64 columns: the wide form (two chunks, the second
# ragged at K = 1152).
@pytest.mark.parametrize("M,N,K,pad", [(17, 512, 1024, 0), (64, 1024, 2048, 8), (40, 4096, 1024, 0), (64, 128, 256, 0),
                                       (33, 640, 4096, 64), (40, 16384, 2048, 0), (48, 20480, 1152, 0)])
def test_fp8_f32s_row_tiles_ldc(M, N, K, pad):
    """gemm_fp8_f32s at 16 < M <= 64 (the row-tile kernel) with a C row stride wider than N: against the oracle within
    the bf16 bar, and C columns past N untouched."""
    rng = np.random.default_rng(5 * M + K)
    ldx, ldc = K + pad, N + 8
    x = randn_bf16(rng, (M, ldx))
    wq, ws, _ = _weights_f32s(rng, N, K)
    q, sa = DeviceBuffer(M * K), DeviceBuffer(M * (K // 128) * 4)
    call("uh_act_quant_fp8_f32s", dev(x), ldx, q, sa, M, K, 128, None)
    q_ref, sa_ref = oracle.act_quant_fp8_f32s(x[:, :K])
    c = dev(np.full((M, ldc), 0x7FC1, np.uint16))
    call("uh_gemm_fp8_f32s", q, sa, dev(wq), dev(ws), c, ldc, M, N, K, None)
    g = c.download((M, ldc), np.uint16)
    assert np.all(g[:, N:] == 0x7FC1)
    ref16, _ = oracle.gemm_w8a8(q_ref, sa_ref, wq, ws)
    mr = max_rel(from_bf16(g[:, :N]), from_bf16(ref16))
    print(f"fp8 f32s row tiles M={M} N={N} K={K} ldc={ldc}: max_rel {mr:.3e}")
    assert mr <= 1e-2


# M > 64 takes the tiled GEMM: 64-column tiles while 128-column ones would make fewer than 256 workgroups
# (M = 200, 1000), else 128 columns (M = 1024, N = 4096).
@pytest.mark.parametrize("M,N,K", [(1, 4096, 4096), (8, 1024, 512), (33, 256, 1024), (200, 512, 512), (17, 200, 640),
                                   (1000, 768, 1024), (1024, 4096, 256), (400, 256, 512)])
def test_fp8_e8m0_scales(M, N, K):
    """The reference's W8A8 contract (gemm_w8a8 / gemv_w8a8 / gemm_w8a8_wmma): e8m0 scales on both sides."""
    rng = np.random.default_rng(M * 3 + K)
    x = randn_bf16(rng, (M, K))
    q_ref, sa_ref = oracle.act_quant_fp8(x)
    wq = rng.integers(0, 256, (N, K), dtype=np.uint8)
    wq[(wq & 0x7F) == 0x7F] = 0  # no NaN codes
    sw = rng.integers(118, 126, ((N + 127) // 128, K // 128), dtype=np.uint8)
    ref16, _ = oracle.gemm_w8a8(q_ref, sa_ref, wq, sw)
    ref = from_bf16(ref16)
    names = ["uh_gemm_w8a8", "uh_gemm_w8a8_wmma"] + (["uh_gemv_w8a8"] if M <= 32 else [])
    outs = []
    for name in names:
        c = DeviceBuffer(M * N * 2)
        call(name, dev(q_ref), dev(sa_ref), dev(wq), dev(sw), c, N, M, N, K, None)
        outs.append(c.download((M, N), np.uint16))
        assert max_rel(from_bf16(outs[-1]), ref) <= 1e-2, name
    for o in outs[1:]:  # every W8A8 entry point gives the same values (a row's result does not depend on M)
        assert np.array_equal(o, outs[0])


@pytest.mark.parametrize("tiled", [False, True])
def test_gemm_a8w4_reference_order_bit_exact(tiled):
    rng = np.random.default_rng(9)
    M, N, K = 7, 256, 512
    x = randn_bf16(rng, (M, K))
    q, qs = oracle.act_quant_fp8(x)
    w, s = mx_weights(rng, N, K)
    if tiled:
        w, s = oracle.repack(w, s, N, K)
    ref16, _ = oracle.gemm_a8w4(q, qs, w, s, N, tiled=tiled)
    c = DeviceBuffer(M * N * 2)
    call("uh_gemm_a8w4_tiled" if tiled else "uh_gemm_a8w4", dev(q), dev(qs), dev(w), dev(s), c, N, M, N, K, None)
    assert np.array_equal(c.download((M, N), np.uint16), ref16)


def _w8a8_weights(rng, N, K):
    wq = rng.integers(0, 256, (N, K), dtype=np.uint8)
    wq[(wq & 0x7F) == 0x7F] = 0  # no NaN codes
    sw = rng.integers(118, 126, ((N + 127) // 128, K // 128), dtype=np.uint8)
    return wq, sw


def test_gemv_w8a8_parts():
    """Ref gemv.hpp:40-52: three column ranges (one ragged) on one input in one launch, each against the oracle and
    bit-identical to gemv_w8a8 on that range alone."""
    rng = np.random.default_rng(21)
    M, K, Ns = 5, 1024, (384, 256, 200)
    x = randn_bf16(rng, (M, K))
    q, sa = oracle.act_quant_fp8(x)
    dq, dsa = dev(q), dev(sa)
    ws = [_w8a8_weights(rng, n, K) for n in Ns]
    dws = [(dev(w), dev(s)) for w, s in ws]
    ldc = [n + 8 for n in Ns]
    outs = [DeviceBuffer(M * l * 2) for l in ldc]
    wp = np.array([d[0].ptr for d in dws], np.uint64)
    sp = np.array([d[1].ptr for d in dws], np.uint64)
    cp = np.array([o.ptr for o in outs], np.uint64)
    ldc_a, n_a = np.array(ldc, np.int32), np.array(Ns, np.int32)  # host arrays: alive across the call
    call("uh_gemv_w8a8_parts", dq, dsa, wp.ctypes.data, sp.ctypes.data, cp.ctypes.data, ldc_a.ctypes.data,
         n_a.ctypes.data, 3, M, K, None)
    for (w, s), (dw, ds), n, l, o in zip(ws, dws, Ns, ldc, outs):
        got = o.download((M, l), np.uint16)[:, :n]
        ref16, _ = oracle.gemm_w8a8(q, sa, w, s)
        assert max_rel(from_bf16(got), from_bf16(ref16)) <= 1e-2
        single = DeviceBuffer(M * n * 2)
        call("uh_gemv_w8a8", dq, dsa, dw, ds, single, n, M, n, K, None)
        assert np.array_equal(single.download((M, n), np.uint16), got)


@pytest.mark.parametrize("M", [1, 3, 32])
def test_gemv_w8a8_glu(M):
    """Ref gemv.hpp:56-57 (the shared expert's gate / up): gate and up against the oracle, and the codes / scales
    exactly act_quant_fp8(bf16(SwiGLU(gate, up))) of the outputs the launch wrote (forward_ref.hip:1231-1244's
    alternative path: swiglu + act_quant_fp8)."""
    rng = np.random.default_rng(M + 40)
    I, K, limit = 512, 1024, 10.0
    x = randn_bf16(rng, (M, K), 2.0)
    q, sa = oracle.act_quant_fp8(x)
    (w1, s1), (w3, s3) = _w8a8_weights(rng, I, K), _w8a8_weights(rng, I, K)
    g, u = DeviceBuffer(M * I * 2), DeviceBuffer(M * I * 2)
    hq, hs = DeviceBuffer(M * I), DeviceBuffer(M * I // 128)
    counters = DeviceBuffer(I // 128 * 4)
    counters.zero()
    call("uh_gemv_w8a8_glu", dev(q), dev(sa), dev(w1), dev(s1), g, I, dev(w3), dev(s3), u, I, I, M, K, limit, hq, hs,
         counters, None)
    gg, uu = g.download((M, I), np.uint16), u.download((M, I), np.uint16)
    for got, (w, s) in ((gg, (w1, s1)), (uu, (w3, s3))):
        assert max_rel(from_bf16(got), from_bf16(oracle.gemm_w8a8(q, sa, w, s)[0])) <= 1e-2
    q_ref, s_ref = oracle.act_quant_fp8(oracle.swiglu(gg, uu, None, limit))
    assert np.array_equal(hq.download((M, I), np.uint8), q_ref)
    assert np.array_equal(hs.download((M, I // 128), np.uint8), s_ref)
    assert not counters.download(I // 128, np.uint32).any()


def test_fp8_gemm_refuses_narrow_ldc():
    """A C row stride below N is refused before any launch (every kernel of the dense dispatch would write past it)."""
    M, N, K = 40, 256, 512
    q, sa = DeviceBuffer(M * K), DeviceBuffer(M * (K // 128) * 4)
    w, sw = DeviceBuffer(N * K), DeviceBuffer((N // 128) * (K // 128) * 4)
    c = DeviceBuffer(M * N * 2)
    with pytest.raises(Exception, match="ldc < N"):
        call("uh_gemm_fp8_f32s", q, sa, w, sw, c, N - 32, M, N, K, None)
