"""GPU parity of the MXFP4 expert path against the CPU oracle, through the C ABI.

Bar: bit-exact for layout, quantization codes/scales, routing and permutation; bf16 outputs of the expert GEMMs
within max-rel 1e-2 (denominator floored at 2^-8 rms) of the oracle's reference-order fp32 path, and the GEMV's fp32
outputs within 1e-3 max-rel of the fp64 oracle on the same quantized operands.
"""
import ctypes

import numpy as np
import pytest

import oracle
from tests.helpers import from_bf16, max_abs_rms, max_rel, mx_weights, randn_bf16, rel_l2, to_bf16
from unholy_amd import call
from unholy_amd._lib import UhError
from unholy_amd.device import DeviceBuffer, pointer_table, synchronize

pytestmark = pytest.mark.gpu


def dev(a):
    return DeviceBuffer.from_array(np.ascontiguousarray(a))


def test_check_dequant_exhaustive():
    bad = ctypes.c_ulonglong(0)
    total = ctypes.c_ulonglong(0)
    call("uh_mx_check_dequant", ctypes.byref(bad), ctypes.byref(total))
    print(f"MFMA decode check: {bad.value} mismatches of {total.value}")
    assert total.value > 200_000
    assert bad.value == 0


def test_check_fp8_encode_exhaustive():
    """The hardware e4m3 encode used by the quantizers equals the software round-to-nearest-even encode (itself
    pinned against brute force in the oracle tests) on every fp32 value the encoders feed it."""
    bad = ctypes.c_ulonglong(0)
    total = ctypes.c_ulonglong(0)
    call("uh_check_fp8_encode", ctypes.byref(bad), ctypes.byref(total))
    print(f"e4m3 encode check: {bad.value} mismatches of {total.value}")
    assert total.value == 2 * (0x43E00000 + 1)
    assert bad.value == 0


def test_exp_f32_matches_oracle_bit_for_bit():
    """The kernels' e^x (SwiGLU silu, softmax / sigmoid router weights) equals the oracle's bit for bit: every bf16
    value, and every 61st fp32 bit pattern of both signs up to the overflow / underflow cut-offs, plus the specials
    (the oracle's e^x is pinned within 2 ulp of float64 e^x in the CPU tests)."""
    bfv = (np.arange(65536, dtype=np.uint32) << 16).view(np.float32)
    pos = np.arange(0, 0x42B30000, 61, dtype=np.uint32).view(np.float32)
    x = np.concatenate([bfv, pos, -pos, np.array([np.inf, -np.inf, 1e30, -1e30], np.float32)])
    dx, dy = DeviceBuffer.from_array(x), DeviceBuffer(x.nbytes)
    call("uh_exp_f32_array", dx, dy, x.size, None)
    got = dy.download(x.shape, np.float32)
    want = oracle.exp_f32(x)
    same = (got.view(np.uint32) == want.view(np.uint32)) | (np.isnan(got) & np.isnan(want))
    print(f"exp_f32: {np.count_nonzero(~same)} of {x.size} differ")
    assert same.all()


def test_check_bf16_encode_exhaustive():
    """The hardware bf16 rounding the kernels use for fp32 -> bf16 equals the software round-to-nearest-even (the
    reference's rounding) at every non-NaN fp32 input, and every NaN input gives a NaN (payloads may differ; they are
    counted apart and printed)."""
    bad = ctypes.c_ulonglong(0)
    nan_bad = ctypes.c_ulonglong(0)
    call("uh_check_bf16_encode", ctypes.byref(bad), ctypes.byref(nan_bad))
    print(f"bf16 rounding check: {bad.value} mismatches at non-NaN inputs, {nan_bad.value} at NaN inputs")
    assert bad.value == 0


@pytest.mark.parametrize("N,K", [(16, 64), (64, 256), (2048, 4096)])
def test_repack_matches_oracle(N, K):
    rng = np.random.default_rng(1)
    w, s = mx_weights(rng, N, K, 0, 254)
    tw_ref, ts_ref = oracle.repack(w, s, N, K)
    dw, ds = dev(w), dev(s)
    tw, ts = DeviceBuffer(w.nbytes), DeviceBuffer(s.nbytes)
    call("uh_mx_repack_to", dw.ptr, ds.ptr, tw.ptr, ts.ptr, N, K, None)
    assert np.array_equal(tw.download(tw_ref.shape, np.uint8), tw_ref)
    assert np.array_equal(ts.download(ts_ref.shape, np.uint8), ts_ref)
    # in place, with the caller's tmp
    tmp = DeviceBuffer(w.nbytes + s.nbytes)
    call("uh_mx_repack", dw.ptr, ds.ptr, N, K, tmp.ptr, None)
    assert np.array_equal(dw.download(tw_ref.shape, np.uint8), tw_ref)
    assert np.array_equal(ds.download(ts_ref.shape, np.uint8), ts_ref)


@pytest.mark.parametrize("block", [32, 64, 128])
def test_act_quant_bit_exact(block):
    rng = np.random.default_rng(2)
    x = randn_bf16(rng, (37, 1024), 3.0)
    x[0, :block] = 0  # amax floor
    x[1, :block] = randn_bf16(rng, (block,), 1e-7)  # tiny block
    q_ref, s_ref = oracle.act_quant_fp8(x, block)
    dx = dev(x)
    q, s = DeviceBuffer(q_ref.nbytes), DeviceBuffer(s_ref.nbytes)
    call("uh_act_quant_fp8", dx.ptr, 1024, q.ptr, s.ptr, 37, 1024, block, None)
    assert np.array_equal(q.download(q_ref.shape, np.uint8), q_ref)
    assert np.array_equal(s.download(s_ref.shape, np.uint8), s_ref)
    call("uh_fake_quant_fp8", dx.ptr, 1024, 37, 1024, block, None)
    assert np.array_equal(dx.download(x.shape, np.uint16), oracle.fake_quant_fp8(x, block))
    q32_ref, s32_ref = oracle.act_quant_fp8_f32s(x, block)
    dx.upload(x)
    s32 = DeviceBuffer(s32_ref.nbytes)
    call("uh_act_quant_fp8_f32s", dx.ptr, 1024, q.ptr, s32.ptr, 37, 1024, block, None)
    assert np.array_equal(q.download(q32_ref.shape, np.uint8), q32_ref)
    assert np.array_equal(s32.download(s32_ref.shape, np.float32), s32_ref)


@pytest.mark.parametrize("block,ldx", [(32, 1024), (64, 1024), (128, 1024), (32, 1029)])
def test_fake_quant_fp4_bit_exact(block, ldx):
    """e2m1 fake quantization in place (ref_elem.hip:43-59) against the oracle, bit for bit: random rows, an all-zero
    and a sub-floor block, every rounding midpoint, values clamped at +-6 x scale; 16-byte rows and an odd stride (the
    2-byte path). Columns past `cols` in the strided rows stay untouched."""
    rng = np.random.default_rng(block + ldx)
    rows, cols = 37, 1024
    full = randn_bf16(rng, (rows, ldx), 3.0)
    x = full[:, :cols]
    x[0, :block] = 0
    x[1, :block] = to_bf16(np.full(block, 1e-39, np.float32))
    ties = np.array([0.25, 0.75, 1.25, 1.75, 2.5, 3.5, 5.0, -0.25, -2.5, -5.0, 6.0, -6.0], np.float32)
    x[2, :len(ties)] = to_bf16(ties)
    x[3, :block] = to_bf16(np.linspace(-70, 70, block, dtype=np.float32))
    ref = oracle.fake_quant_fp4(np.ascontiguousarray(x), block)
    dx = dev(full)
    call("uh_fake_quant_fp4", dx.ptr, ldx, rows, cols, block, None)
    got = dx.download(full.shape, np.uint16)
    assert np.array_equal(got[:, :cols], ref)
    assert np.array_equal(got[:, cols:], full[:, cols:])
    with pytest.raises(UhError, match="block % 8"):
        call("uh_fake_quant_fp4", dx.ptr, ldx, rows, cols, 12, None)


def test_xform_in_gathered_rows():
    rng = np.random.default_rng(3)
    T, K, P, E = 9, 512, 20, 4
    x = randn_bf16(rng, (T, K))
    x_rows = rng.integers(0, T, P).astype(np.int32)
    row_expert = rng.integers(0, E, P).astype(np.int32)
    present = DeviceBuffer(16)
    tab = pointer_table([present, None, present, present])  # expert 1 not resident: its rows skipped
    gathered = x[x_rows]
    fq_ref = oracle.fake_quant_fp8(gathered)
    q_ref, s_ref = oracle.act_quant_fp8(gathered)
    dx, dr, de = dev(x), dev(x_rows), dev(row_expert)
    xa = DeviceBuffer(P * K * 2)
    xa.zero()
    call("uh_mx_xform_in", dx.ptr, K, de.ptr, tab.ptr, xa.ptr, P, K, None, dr.ptr)
    q, s = DeviceBuffer(P * K), DeviceBuffer(P * K // 128)
    q.zero()
    s.zero()
    call("uh_mx_xform_in_fp8", dx.ptr, K, de.ptr, tab.ptr, q.ptr, s.ptr, P, K, None, dr.ptr)
    got, gq, gs = xa.download((P, K), np.uint16), q.download((P, K), np.uint8), s.download((P, K // 128), np.uint8)
    live = row_expert != 1
    assert np.array_equal(got[live], fq_ref[live])
    assert np.array_equal(gq[live], q_ref[live]) and np.array_equal(gs[live], s_ref[live])
    assert not got[~live].any() and not gq[~live].any()


def _expert_tables(experts, keys):
    bufs = {k: [dev(ex[k]) if ex is not None else None for ex in experts] for k in keys}
    tabs = {k: pointer_table(bufs[k]) for k in keys}
    return bufs, tabs


def _make_experts(rng, E, N, K, names=("w", "s")):
    out = []
    for _ in range(E):
        w, s = mx_weights(rng, N, K)
        tw, ts = oracle.repack(w, s, N, K)
        out.append({names[0]: tw, names[1]: ts})
    return out


def test_single_gemv_config0():
    """x [1, 4096] ~ N(0,1), W [2048, 4096] MXFP4 with e8m0 in [119, 125], seed 0."""
    rng = np.random.default_rng(0)
    N, K = 2048, 4096
    x = randn_bf16(rng, (1, K))
    w, s = mx_weights(rng, N, K)
    tw, ts = oracle.repack(w, s, N, K)
    q, qs = oracle.act_quant_fp8(x)
    ref16, ref32 = oracle.gemm_a8w4(q, qs, w, s, N)
    ref64 = oracle.gemm_a8w4_f64(q, qs, w, s, N)
    dq, dqs, dw, ds = dev(q), dev(qs), dev(tw), dev(ts)
    wt, st = pointer_table([dw]), pointer_table([ds])
    tiles = dev(np.array([[0, 0, 1]], np.int32))
    out = DeviceBuffer(N * 2)
    call("uh_mx_grouped_gemv_q", dq.ptr, dqs.ptr, K, tiles.ptr, 1, wt.ptr, st.ptr, out.ptr, N, N, None, None,
         None, None, None, 1, None, None, None, None, None, None, 0.0)
    out32 = DeviceBuffer(N * 4)
    call("uh_mx_grouped_gemv_q_f32out", dq.ptr, dqs.ptr, K, tiles.ptr, 1, wt.ptr, st.ptr, out32.ptr, N, N, None,
         None, 1)
    got = from_bf16(out.download((1, N), np.uint16))
    got32 = out32.download((1, N), np.float32)
    mr, mr64 = max_rel(got, from_bf16(ref16)), max_rel(got32, ref64)
    print(f"config0: max_rel vs ref {mr:.3e}, rel_l2 {rel_l2(got, from_bf16(ref16)):.3e}, fp32 vs fp64 {mr64:.3e}, "
          f"bit-identical {np.mean(out.download((1, N), np.uint16) == ref16):.4f}")
    assert mr <= 1e-2
    assert mr64 <= 1e-3
    # the drop-in form: bf16 fake-quantized xa -> the same MFMA operands
    xa = DeviceBuffer(K * 2)
    call("uh_mx_xform_in", dev(x), K, dev(np.zeros(1, np.int32)), st.ptr, xa.ptr, 1, K, None, None)
    out2 = DeviceBuffer(N * 2)
    call("uh_mx_grouped_gemv", xa.ptr, K, tiles.ptr, 1, wt.ptr, st.ptr, out2.ptr, N, N, None, None, None, None, None,
         8, None, None, None, None, 0.0, None)
    assert np.array_equal(out2.download((1, N), np.uint16), out.download((1, N), np.uint16))


@pytest.mark.parametrize("abf16", [False, True])
def test_grouped_gemv_glu(abf16):
    """Tiles of 1-16 rows over several experts, w1 and w3 in one launch with the SwiGLU epilogue."""
    rng = np.random.default_rng(5)
    E, K, N, limit = 5, 1024, 512, 10.0
    rows = [3, 16, 1, 0, 11]
    P = sum(rows)
    tiles, row_expert, r0 = [], [], 0
    for e, c in enumerate(rows):
        if c:
            tiles.append([e, r0, c])
        row_expert += [e] * c
        r0 += c
    tiles.append([2, 0, 0])  # an empty tile past the live count
    ntiles_live = len(tiles) - 1
    row_expert = np.array(row_expert, np.int32)
    w1 = _make_experts(rng, E, N, K)
    w3 = _make_experts(rng, E, N, K)
    w1raw = [oracle.unrepack(ex["w"], ex["s"], N, K) for ex in w1]
    w3raw = [oracle.unrepack(ex["w"], ex["s"], N, K) for ex in w3]
    x = randn_bf16(rng, (P, K))
    q, qs = oracle.act_quant_fp8(x)
    rw = rng.random(P).astype(np.float32)
    g_ref = np.zeros((P, N), np.uint16)
    u_ref = np.zeros((P, N), np.uint16)
    for t in tiles[:ntiles_live]:
        e, a, c = t
        g_ref[a:a + c] = oracle.gemm_a8w4(q[a:a + c], qs[a:a + c], *w1raw[e], N)[0]
        u_ref[a:a + c] = oracle.gemm_a8w4(q[a:a + c], qs[a:a + c], *w3raw[e], N)[0]
    b1, t1 = _expert_tables(w1, ("w", "s"))
    b3, t3 = _expert_tables(w3, ("w", "s"))
    dtiles = dev(np.array(tiles, np.int32))
    ntd = dev(np.array([ntiles_live], np.int32))
    g, u, hh = DeviceBuffer(P * N * 2), DeviceBuffer(P * N * 2), DeviceBuffer(P * N * 2)
    de, drw = dev(row_expert), dev(rw)
    if abf16:
        xa = dev(oracle.fake_quant_fp8(x))
        call("uh_mx_grouped_gemv", xa.ptr, K, dtiles.ptr, len(tiles), t1["w"].ptr, t1["s"].ptr, g.ptr, N, N, None,
             ntd.ptr, t3["w"].ptr, t3["s"].ptr, u.ptr, 16, drw.ptr, de.ptr, t1["s"].ptr, hh.ptr, limit, None)
    else:
        hq, hs = DeviceBuffer(P * N), DeviceBuffer(P * N // 128)
        call("uh_mx_grouped_gemv_q", dev(q), dev(qs), K, dtiles.ptr, len(tiles), t1["w"].ptr, t1["s"].ptr,
             g.ptr, N, N, None, ntd.ptr, t3["w"].ptr, t3["s"].ptr, u.ptr, 16, drw.ptr, de.ptr, t1["s"].ptr, hh.ptr,
             hq.ptr, hs.ptr, limit)
    synchronize()
    gg, uu, hgot = (b.download((P, N), np.uint16) for b in (g, u, hh))
    assert max_rel(from_bf16(gg), from_bf16(g_ref)) <= 1e-2
    assert max_rel(from_bf16(uu), from_bf16(u_ref)) <= 1e-2
    # The epilogue on the kernel's own g / u: swiglu + fake quant as the reference's mx_swiglu.
    h_ref = oracle.fake_quant_fp8(oracle.swiglu(gg, uu, rw, limit))
    frac = np.mean(hgot == h_ref)
    print(f"glu abf16={abf16}: hh bit-identical fraction {frac:.6f}")
    assert max_rel(from_bf16(hgot), from_bf16(h_ref)) <= 1e-2
    assert frac > 0.999
    if not abf16:
        # codes x scales are exactly the fake-quantized values (the codes themselves are act_quant's of the
        # SwiGLU output, so for rows where it is bit-identical they equal the oracle's codes too)
        codes, scales = hq.download((P, N), np.uint8), hs.download((P, N // 128), np.uint8)
        deq = oracle.e4m3_to_f32(codes) * np.ldexp(1.0, scales.astype(np.int32) - 127).repeat(128, axis=1)
        assert np.array_equal(deq.astype(np.float32), from_bf16(hgot))
        q2, s2 = oracle.act_quant_fp8(oracle.swiglu(gg, uu, rw, limit))
        same = (hgot == h_ref).all(axis=1)
        assert np.array_equal(codes[same], q2[same]) and np.array_equal(scales[same], s2[same])


def test_gemv_x_fused_quant_is_bit_identical():
    """uh_mx_grouped_gemv_x (act_quant of gathered token rows in the GEMV's staging) == xform_in_fp8 + gemv_q."""
    rng = np.random.default_rng(21)
    E, K, N, T, limit = 3, 2048, 256, 9, 10.0
    rows = [4, 7, 2]
    P = sum(rows)
    tiles, row_expert, r0 = [], [], 0
    for e, c in enumerate(rows):
        tiles.append([e, r0, c])
        row_expert += [e] * c
        r0 += c
    x = randn_bf16(rng, (T, K), 2.0)
    x_rows = rng.integers(0, T, P).astype(np.int32)
    w1, w3 = _make_experts(rng, E, N, K), _make_experts(rng, E, N, K)
    b1, t1 = _expert_tables(w1, ("w", "s"))
    b3, t3 = _expert_tables(w3, ("w", "s"))
    rw = rng.random(P).astype(np.float32)
    dx, dr, de, drw, dt = dev(x), dev(x_rows), dev(np.array(row_expert, np.int32)), dev(rw), dev(np.array(tiles, np.int32))
    q, qs = DeviceBuffer(P * K), DeviceBuffer(P * K // 128)
    call("uh_mx_xform_in_fp8", dx, K, de, t1["s"], q, qs, P, K, None, dr)
    outs = []
    for fused in (False, True):
        hq, hs, g = DeviceBuffer(P * N), DeviceBuffer(P * N // 128), DeviceBuffer(P * N * 2)
        if fused:
            call("uh_mx_grouped_gemv_x", dx, K, dr, K, dt, 3, t1["w"], t1["s"], g, N, N, None, None, t3["w"], t3["s"],
                 None, 16, drw, de, t1["s"], None, hq, hs, limit)
        else:
            call("uh_mx_grouped_gemv_q", q, qs, K, dt, 3, t1["w"], t1["s"], g, N, N, None, None, t3["w"], t3["s"],
                 None, 16, drw, de, t1["s"], None, hq, hs, limit)
        outs.append((g.download((P, N), np.uint16), hq.download((P, N), np.uint8), hs.download((P, N // 128), np.uint8)))
    for a, b in zip(*outs):
        assert np.array_equal(a, b)


def _gemm_case(rng, rows, E, K, N):
    tiles, row_expert, r0 = [], [], 0
    for e, c in enumerate(rows):
        for i in range(0, c, 128):
            tiles.append([e, r0 + i, min(128, c - i)])
        row_expert += [e] * c
        r0 += c
    return np.array(tiles, np.int32), np.array(row_expert, np.int32), sum(rows)


def test_gemm_fp32_accuracy_k4096(gemm_arith):
    """The prefill GEMM at the model's inner size (K = 4096, 96 rows of one expert): fp32 outputs against the fp64
    oracle on the same quantized operands, with the bars of test_grouped_gemm_prefill_tiles."""
    rng = np.random.default_rng(77)
    K, N, R = 4096, 256, 96
    x = randn_bf16(rng, (R, K))
    q, qs = oracle.act_quant_fp8(x)
    w, s_ = mx_weights(rng, N, K)
    tw, ts = oracle.repack(w, s_, N, K)
    ref64 = oracle.gemm_a8w4_f64(q, qs, w, s_, N)
    dw, ds, dq, dqs = dev(tw), dev(ts), dev(q), dev(qs)  # alive until the kernel has run (download syncs)
    wt, st = pointer_table([dw]), pointer_table([ds])
    tiles = dev(np.array([[0, 0, R]], np.int32))
    out = DeviceBuffer(R * N * 4)
    call("uh_mx_grouped_gemm_q_f32out", dq, dqs, K, tiles, 1, wt.ptr, st.ptr, out, N, N, None, None)
    got = out.download((R, N), np.float32)
    m, l2, ma = max_rel(got, ref64), rel_l2(got, ref64), max_abs_rms(got, ref64)
    same = np.mean(got == oracle.gemm_a8w4(q, qs, w, s_, N)[1])  # fp32 values of the reference's order
    print(f"gemm K=4096 {gemm_arith}: max_rel {m:.3e} rel_l2 {l2:.3e} max|err|/rms {ma:.3e}, fp32 bit-identical "
          f"to the reference order {same:.4f}")
    if gemm_arith == "exact":  # (95% of the fp32 values equal the reference order's; the rest differ by an ulp)
        assert m <= 1e-3
    else:
        assert l2 <= 1e-3 and ma <= 1e-4


@pytest.mark.parametrize("amode", ["q", "bf16", "x"])
def test_grouped_gemm_prefill_tiles(amode, gemm_arith):
    """The 128-row MFMA GEMM: tiles of 1..128 rows (and one expert split over two tiles), w1 and w3 in two launches
    (no epilogue) and in one launch with the SwiGLU epilogue, against the oracle; fp32 outputs against fp64.
    Tolerances: bf16 outputs max-rel <= 1e-2 (per element, floor 2^-8 rms) on either arithmetic. fp32 outputs against
    fp64: exact dequantization (the default) max-rel <= 1e-3 per element; the block-scaled MFMA speed mode (its sums
    are not exact; not a parity arithmetic) rel L2
    <= 1e-3 -- the reference's own criterion for its fast MXFP4 GEMM (tools/kernel_test/mx_moe.hip:3) -- and
    max |err| <= 1e-4 rms. Only amode q runs the pipelined kernel whose arithmetic gemm_arith selects."""
    if amode != "q" and gemm_arith != "exact":
        pytest.skip("the arithmetic switch only concerns the e4m3-code kernel")
    rng = np.random.default_rng(33)
    E, K, N, T, limit = 4, 1024, 256, 300, 10.0
    rows = [96, 1, 200, 37]
    tiles, row_expert, P = _gemm_case(rng, rows, E, K, N)
    x = randn_bf16(rng, (T, K), 2.0)
    x_rows = rng.integers(0, T, P).astype(np.int32)
    q, qs = oracle.act_quant_fp8(x[x_rows])
    w1, w3 = _make_experts(rng, E, N, K), _make_experts(rng, E, N, K)
    b1, t1 = _expert_tables(w1, ("w", "s"))
    b3, t3 = _expert_tables(w3, ("w", "s"))
    rw = rng.random(P).astype(np.float32)
    g_ref = np.zeros((P, N), np.uint16)
    g64 = np.zeros((P, N))
    for e, a0, c in tiles:
        w, s_ = oracle.unrepack(w1[e]["w"], w1[e]["s"], N, K)
        g_ref[a0:a0 + c] = oracle.gemm_a8w4(q[a0:a0 + c], qs[a0:a0 + c], w, s_, N)[0]
        g64[a0:a0 + c] = oracle.gemm_a8w4_f64(q[a0:a0 + c], qs[a0:a0 + c], w, s_, N)
    dq, dqs, dt, de, drw = dev(q), dev(qs), dev(tiles), dev(row_expert), dev(rw)
    dx, dr = dev(x), dev(x_rows)
    g, u = DeviceBuffer(P * N * 2), DeviceBuffer(P * N * 2)
    nt = len(tiles)
    if amode == "q":
        call("uh_mx_grouped_gemm_q", dq, dqs, K, dt, nt, t1["w"], t1["s"], g, N, N, None, None, t3["w"], t3["s"], u, 128,
             None, None, None, None, None, None, 0.0)
    elif amode == "bf16":
        xa = dev(oracle.fake_quant_fp8(x[x_rows]))
        call("uh_mx_grouped_gemm", xa, K, dt, nt, t1["w"], t1["s"], g, N, N, None, None, t3["w"], t3["s"], u, 128)
    else:
        call("uh_mx_grouped_gemm_x", dx, K, dr, K, dt, nt, t1["w"], t1["s"], g, N, N, None, None, t3["w"], t3["s"], u,
             None, None, None, None, None, None, 0.0)
    gg, uu = g.download((P, N), np.uint16), u.download((P, N), np.uint16)
    mr = max_rel(from_bf16(gg), from_bf16(g_ref))
    print(f"gemm {amode} {gemm_arith}: max_rel {mr:.3e} bit-identical {np.mean(gg == g_ref):.4f}")
    assert mr <= 1e-2
    if gemm_arith == "exact":  # one MFMA per 32-block: the reference's order of roundings
        assert np.mean(gg == g_ref) >= 0.999
    if amode == "q":  # fp32 outputs against the fp64 oracle
        g32 = DeviceBuffer(P * N * 4)
        call("uh_mx_grouped_gemm_q_f32out", dq, dqs, K, dt, nt, t1["w"], t1["s"], g32, N, N, None, None)
        got32 = g32.download((P, N), np.float32)
        m32, l32, a32 = max_rel(got32, g64), rel_l2(got32, g64), max_abs_rms(got32, g64)
        print(f"gemm q {gemm_arith} fp32 vs fp64: max_rel {m32:.3e} rel_l2 {l32:.3e} max|err|/rms {a32:.3e}")
        if gemm_arith == "exact":
            assert m32 <= 1e-3
        else:
            assert l32 <= 1e-3 and a32 <= 1e-4
    # the SwiGLU epilogue in one launch: its g / u, and hh / hq / hs against the transform of those
    hq, hs, hh, g2, u2 = DeviceBuffer(P * N), DeviceBuffer(P * N // 128), DeviceBuffer(P * N * 2), DeviceBuffer(P * N * 2), DeviceBuffer(P * N * 2)
    if amode == "q":
        call("uh_mx_grouped_gemm_q", dq, dqs, K, dt, nt, t1["w"], t1["s"], g2, N, N, None, None, t3["w"], t3["s"], u2,
             128, drw, de, t1["s"], hh, hq, hs, limit)
    elif amode == "bf16":
        call("uh_mx_grouped_gemm_glu", xa, K, dt, nt, t1["w"], t1["s"], t3["w"], t3["s"], N, drw, de, t1["s"], hh,
             limit, None, None)
    else:
        call("uh_mx_grouped_gemm_x", dx, K, dr, K, dt, nt, t1["w"], t1["s"], g2, N, N, None, None, t3["w"], t3["s"], u2,
             drw, de, t1["s"], hh, hq, hs, limit)
    synchronize()
    if amode != "bf16":
        assert np.array_equal(g2.download((P, N), np.uint16), gg) and np.array_equal(u2.download((P, N), np.uint16), uu)
    h_ref = oracle.fake_quant_fp8(oracle.swiglu(gg, uu, rw, limit))
    hgot = hh.download((P, N), np.uint16)
    print(f"gemm glu {amode}: hh bit-identical {np.mean(hgot == h_ref):.6f}")
    assert np.mean(hgot == h_ref) > 0.999 and max_rel(from_bf16(hgot), from_bf16(h_ref)) <= 1e-2
    if amode != "bf16":
        codes, scales = hq.download((P, N), np.uint8), hs.download((P, N // 128), np.uint8)
        deq = oracle.e4m3_to_f32(codes) * np.ldexp(1.0, scales.astype(np.int32) - 127).repeat(128, axis=1)
        assert np.array_equal(deq.astype(np.float32), from_bf16(hgot))


@pytest.mark.parametrize("K,N", [(1024, 384), (512, 256)])
def test_grouped_gemm_max_rows_routes_to_gemv(K, N):
    """mx_grouped_gemm with max_rows <= 64 (the reference's verify steps pass the step's token count,
    forward_ref.hip:455-470) runs the grouped GEMV over 128-row tiles of up to 64 rows; the outputs must equal the
    128-row GEMM's (max_rows = 128) bit for bit, with one and with two projections, and match the oracle (max-rel <=
    1e-2 per element). N = 384 also runs the GEMM's half column block (N % 256 == 128)."""
    rng = np.random.default_rng(71)
    E = 5
    rows = [1, 17, 64, 0, 40]
    tiles, row_expert, P = _gemm_case(rng, rows, E, K, N)
    x = randn_bf16(rng, (P, K), 1.5)
    xa = oracle.fake_quant_fp8(x)
    q, qs = oracle.act_quant_fp8(x)
    w1, w3 = _make_experts(rng, E, N, K), _make_experts(rng, E, N, K)
    b1, t1 = _expert_tables(w1, ("w", "s"))
    b3, t3 = _expert_tables(w3, ("w", "s"))
    g_ref = np.zeros((P, N), np.uint16)
    for e, a0, c in tiles:
        w, s_ = oracle.unrepack(w1[e]["w"], w1[e]["s"], N, K)
        g_ref[a0:a0 + c] = oracle.gemm_a8w4(q[a0:a0 + c], qs[a0:a0 + c], w, s_, N)[0]
    dxa, dt = dev(xa), dev(tiles)
    ntd = dev(np.array([len(tiles)], np.int32))
    outs = {}
    for max_rows in (128, 64, 40):
        g, u, g1 = DeviceBuffer(P * N * 2), DeviceBuffer(P * N * 2), DeviceBuffer(P * N * 2)
        call("uh_mx_grouped_gemm", dxa, K, dt, len(tiles) + 3, t1["w"], t1["s"], g, N, N, None, ntd, t3["w"], t3["s"],
             u, max_rows)
        call("uh_mx_grouped_gemm", dxa, K, dt, len(tiles), t1["w"], t1["s"], g1, N, N, None, None, None, None, None,
             max_rows)
        synchronize()
        outs[max_rows] = [b.download((P, N), np.uint16) for b in (g, u, g1)]
    mr = max_rel(from_bf16(outs[128][0]), from_bf16(g_ref))
    print(f"K={K} N={N}: GEMM vs oracle max_rel {mr:.3e}, bit-identical {np.mean(outs[128][0] == g_ref):.5f}")
    assert mr <= 1e-2 and np.array_equal(outs[128][0], outs[128][2])
    for max_rows in (64, 40):  # 40: tiles of up to 64 rows still run whole (16-row groups)
        for a, b in zip(outs[max_rows], outs[128]):
            assert np.array_equal(a, b), max_rows


def test_grouped_gemm_k64_half_block():
    """K % 64 == 0 with K % 128 != 0 (the reference's bound, mx_moe.hip:1045) and N % 256 == 128 on plain bf16 rows:
    the 64-input-stage GEMM against an fp64 product of the bf16 rows and the decoded weights (max-rel <= 1e-2 per
    element; the rows are not fake-quantized here, so each 32-block's sum rounds once in fp32)."""
    rng = np.random.default_rng(72)
    E, K, N = 3, 192, 384
    rows = [5, 130, 33]
    tiles, row_expert, P = _gemm_case(rng, rows, E, K, N)
    x = randn_bf16(rng, (P, K))
    w1 = _make_experts(rng, E, N, K)
    b1, t1 = _expert_tables(w1, ("w", "s"))
    ref = np.zeros((P, N))
    xf = from_bf16(x).astype(np.float64)
    for e, a0, c in tiles:
        wd = oracle.mx_dequant(w1[e]["w"], w1[e]["s"], N, K, tiled=True).astype(np.float64)
        ref[a0:a0 + c] = xf[a0:a0 + c] @ wd.T
    g = DeviceBuffer(P * N * 2)
    call("uh_mx_grouped_gemm", dev(x), K, dev(tiles), len(tiles), t1["w"], t1["s"], g, N, N, None, None, None, None,
         None, 128)
    synchronize()
    got = from_bf16(g.download((P, N), np.uint16))
    mr = max_rel(got, ref)
    print(f"K={K} N={N} bf16 rows: max_rel {mr:.3e} vs fp64")
    assert mr <= 1e-2
