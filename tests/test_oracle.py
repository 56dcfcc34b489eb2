"""Pins the CPU oracle (oracle/uh_oracle.cpp) against the reference's own host code (oracle/_ref: half.hpp codecs and
expert_pack.cpp's repack, compiled from the reference sources), closed forms, brute force and invariants, so that a
plausible mistake (a dropped term, a wrong sign or index, a transposed operand) fails at least one check."""
import math

import numpy as np
import pytest

import oracle
from tests.helpers import from_bf16, mx_weights, randn_bf16, to_bf16

GRID_E2M1 = [0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0]


def e4m3_closed(c):
    c = int(c)  # numpy uint8 arithmetic would wrap e - 7
    s = -1.0 if c & 0x80 else 1.0
    e, m = (c >> 3) & 15, c & 7
    return s * (m * 2.0 ** -9 if e == 0 else (1 + m / 8) * 2.0 ** (e - 7))


E4M3_FINITE = [c for c in range(256) if (c & 0x7F) != 0x7F]


# ---- codecs --------------------------------------------------------------------------------------------------------------
def test_e4m3_decode_all_codes():
    lib = oracle.lib()
    for c in range(256):
        got = lib.or_e4m3_to_f32(c)
        if (c & 0x7F) == 0x7F:
            assert got == (-480.0 if c & 0x80 else 480.0)  # the device decode has no NaN case (dev.hip.hpp:59-63)
        else:
            assert got == e4m3_closed(c), c


def test_e2m1_e8m0_decode():
    lib = oracle.lib()
    for n in range(16):
        assert lib.or_e2m1_to_f32(n) == (-1 if n & 8 else 1) * GRID_E2M1[n & 7]
    assert lib.or_e8m0_to_f32(0) == 0.0  # device semantics: the exponent field shifted in (dev.hip.hpp:96)
    for v in range(1, 255):
        assert lib.or_e8m0_to_f32(v) == 2.0 ** (v - 127)


def test_codecs_match_reference_host_code():
    ref = oracle.ref_lib()
    if ref is None:
        pytest.skip("oracle/_ref not built (the reference tree is only present in the build container)")
    lib = oracle.lib()
    for c in E4M3_FINITE:
        assert lib.or_e4m3_to_f32(c) == ref.ref_e4m3_to_float(c)
    for n in range(16):
        assert lib.or_e2m1_to_f32(n) == ref.ref_e2m1_to_float(n)
    for v in range(1, 255):
        assert lib.or_e8m0_to_f32(v) == ref.ref_e8m0_to_float(v)
    for b in range(0, 65536, 97):
        x, y = lib.or_bf16_to_f32(b), ref.ref_bf16_to_float(b)
        assert (math.isnan(x) and math.isnan(y)) or x == y


def test_bf16_round_to_nearest_even():
    rng = np.random.default_rng(0)
    x = rng.standard_normal(100000).astype(np.float32) * np.float32(1000)
    u = x.view(np.uint32)
    # ties: exactly halfway between two bf16 values, both parities
    ties = np.array([0x3F808000, 0x3F818000, 0xBF808000, 0x7F7F8000], np.uint32).view(np.float32)
    got = oracle.f32_to_bf16(np.concatenate([x, ties]))
    want = to_bf16(np.concatenate([x, ties]))
    assert np.array_equal(got, want)
    assert list(got[-4:]) == [0x3F80, 0x3F82, 0xBF80, 0x7F80]  # even stays, odd rounds up, overflow -> inf
    nan = oracle.f32_to_bf16(np.array([np.nan], np.float32))[0]
    assert (nan & 0x7F80) == 0x7F80 and (nan & 0x40)  # quiet NaN
    assert np.all(from_bf16(got[:-4]) == from_bf16(want[:-4]))
    del u


def test_e4m3_encode_rne_against_brute_force():
    vals = np.array([e4m3_closed(c) for c in E4M3_FINITE], np.float64)
    order = np.argsort(vals, kind="stable")
    grid, codes = vals[order], np.array(E4M3_FINITE)[order]
    # every representable value round-trips
    for c in E4M3_FINITE:
        v = e4m3_closed(c)
        got = int(oracle.lib().or_f32_to_e4m3(v))
        assert got == c or (v == 0 and got in (0, 0x80)), (c, got)
    # midpoints round to the even mantissa; random values to the nearest
    rng = np.random.default_rng(1)
    x = np.concatenate([(grid[1:] + grid[:-1]) / 2, rng.uniform(-448, 448, 20000), rng.uniform(-0.02, 0.02, 20000)])
    x = x.astype(np.float32)
    got = oracle.f32_to_e4m3(x)
    for xi, g in zip(x.astype(np.float64), got):
        d = np.abs(grid - xi)
        best = np.flatnonzero(d == d.min())
        cand = [int(codes[b]) for b in best]
        if len(cand) > 1:  # a tie: the even mantissa (code bit 0 clear)
            cand = [c for c in cand if (c & 1) == 0]
        gv = e4m3_closed(int(g))
        assert any(e4m3_closed(c) == gv for c in cand), (xi, g, cand)


def test_pow2_ceil_scale():
    rng = np.random.default_rng(2)
    lib = oracle.lib()
    for v in np.concatenate([rng.uniform(1e-6, 10, 2000), 2.0 ** np.arange(-20, 20)]).astype(np.float32):
        m, e = math.frexp(float(v))  # kernel.py _pow2_ceil: e - (m == 0.5)
        want = e - (1 if m == 0.5 else 0)
        assert lib.or_pow2_ceil_e8m0(float(v)) == want + 127


# ---- quantization ---------------------------------------------------------------------------------------------------------
@pytest.mark.parametrize("block", [32, 64, 128])
def test_act_quant_closed_form(block):
    rng = np.random.default_rng(3)
    x = randn_bf16(rng, (9, 512), 2.0)
    x[0, :block] = 0
    x[1, :block] = to_bf16(np.full(block, 448.0 * 2 ** -5, np.float32))  # amax / 448 an exact power of two
    q, s = oracle.act_quant_fp8(x, block)
    xf = from_bf16(x).astype(np.float64).reshape(9, -1, block)
    amax = np.maximum(np.abs(xf).max(-1), np.float32(1e-4))
    se = np.ceil(np.log2(amax.astype(np.float32) * np.float32(1 / 448))).astype(int) + 127
    assert np.array_equal(s.astype(int), se)
    assert s[1, 0] == 127 - 5
    deq = np.vectorize(e4m3_closed)(q).reshape(9, -1, block) * 2.0 ** (s.astype(int) - 127)[..., None]
    err = np.abs(deq - xf)
    half_ulp = np.maximum(np.abs(xf), 2.0 ** -6 * 2.0 ** (s.astype(int) - 127)[..., None]) * 2.0 ** -4
    assert np.all(err <= half_ulp * (1 + 1e-12))
    assert np.all(np.abs(np.vectorize(e4m3_closed)(q)) <= 448)
    fq = oracle.fake_quant_fp8(x, block)
    assert np.array_equal(from_bf16(fq).reshape(9, -1, block), deq.astype(np.float32))


def test_act_quant_fp32_scales():
    rng = np.random.default_rng(4)
    x = randn_bf16(rng, (4, 256))
    q, s = oracle.act_quant_fp8_f32s(x)
    xf = from_bf16(x).reshape(4, 2, 128)
    want = np.maximum(np.abs(xf).max(-1), np.float32(1e-4)) * np.float32(1 / 448)
    assert np.array_equal(s, want.astype(np.float32))
    deq = np.vectorize(e4m3_closed)(q).reshape(4, 2, 128) * s[..., None]
    assert np.all(np.abs(deq - xf) <= np.abs(xf) * 2 ** -4 + s[..., None] * 2 ** -9)


# ---- layout ----------------------------------------------------------------------------------------------------------------
@pytest.mark.parametrize("N,K", [(16, 64), (48, 256), (2048, 128)])
def test_repack_matches_reference_and_inverts(N, K):
    rng = np.random.default_rng(5)
    w, s = mx_weights(rng, N, K, 0, 254)
    tw, ts = oracle.repack(w, s, N, K)
    w2, s2 = oracle.unrepack(tw, ts, N, K)
    assert np.array_equal(w2, w) and np.array_equal(s2, s)
    # explicit index formula (ref_gemm.hip:95-96, 152-153)
    for n, kbyte in [(0, 0), (N - 1, K // 2 - 1), (17 % N, 33 % (K // 2))]:
        k = 2 * kbyte
        chunk = (k // 64) * (N // 16) + n // 16
        assert tw[chunk * 512 + (n % 16) * 32 + (k % 64) // 2] == w[n, kbyte]
        b = k // 32
        assert ts[((b // 2) * (N // 16) + n // 16) * 32 + (n % 16) * 2 + b % 2] == s[n, b]
    ref = oracle.ref_lib()
    if ref is not None:
        rw, rs = np.empty_like(tw), np.empty_like(ts)
        ref.ref_repack_matrix(w.ctypes.data, s.ctypes.data, rw.ctypes.data, rs.ctypes.data, N, K)
        assert np.array_equal(rw, tw) and np.array_equal(rs, ts)


def test_mx_dequant_exhaustive_codes_and_scales():
    # every byte value x every scale of interest, against e2m1 * 2^(s-127)
    N, K = 16, 512
    w = np.tile(np.arange(256, dtype=np.uint8), N)[: N * K // 2].reshape(N, K // 2)
    for s0 in (1, 100, 127, 200, 254):
        s = np.full((N, K // 32), s0, np.uint8)
        d = oracle.mx_dequant(w, s, N, K)
        lo = np.array([GRID_E2M1[b & 7] * (-1 if b & 8 else 1) for b in range(256)])
        hi = np.array([GRID_E2M1[(b >> 4) & 7] * (-1 if b & 0x80 else 1) for b in range(256)])
        want = np.stack([lo[w], hi[w]], -1).reshape(N, K) * 2.0 ** (s0 - 127)
        with np.errstate(over="ignore"):
            assert np.array_equal(d, want.astype(np.float32))


# ---- GEMMs -----------------------------------------------------------------------------------------------------------------
def _a8w4_f64_numpy(q, qs, w, s):
    a = np.vectorize(e4m3_closed)(q) * np.repeat(2.0 ** (qs.astype(int) - 127), 128, axis=1)
    lo = np.array([GRID_E2M1[b & 7] * (-1 if b & 8 else 1) for b in range(256)])
    hi = np.array([GRID_E2M1[(b >> 4) & 7] * (-1 if b & 0x80 else 1) for b in range(256)])
    N = w.shape[0]
    wv = np.stack([lo[w], hi[w]], -1).reshape(N, -1) * np.repeat(2.0 ** (s.astype(int) - 127), 32, axis=1)
    return a @ wv.T


def test_gemm_a8w4_brute_force_and_layouts():
    rng = np.random.default_rng(6)
    M, N, K = 5, 48, 256
    q, qs = oracle.act_quant_fp8(randn_bf16(rng, (M, K)))
    w, s = mx_weights(rng, N, K)
    c16, c32 = oracle.gemm_a8w4(q, qs, w, s, N)
    exact = _a8w4_f64_numpy(q, qs, w, s)
    assert np.max(np.abs(c32 - exact)) <= 1e-6 * np.max(np.abs(exact))
    assert np.array_equal(c16, oracle.f32_to_bf16(c32))
    assert np.allclose(oracle.gemm_a8w4_f64(q, qs, w, s, N), exact, rtol=1e-12, atol=1e-12 * np.abs(exact).max())
    tw, ts = oracle.repack(w, s, N, K)
    t16, t32 = oracle.gemm_a8w4(q, qs, tw, ts, N, tiled=True)
    assert np.array_equal(t32, c32)  # same operands, same order
    # a transposed / misindexed scale would move the result: perturb one weight scale and see exactly one column move
    s2 = s.copy()
    s2[7, 3] += 1
    _, d32 = oracle.gemm_a8w4(q, qs, w, s2, N)
    moved = np.flatnonzero(np.any(d32 != c32, axis=0))
    assert list(moved) == [7]


@pytest.mark.parametrize("f32", [False, True])
def test_gemm_w8a8_brute_force(f32):
    rng = np.random.default_rng(7)
    M, N, K = 4, 256, 384
    x = randn_bf16(rng, (M, K))
    if f32:
        q, sa = oracle.act_quant_fp8_f32s(x)
        sw = rng.uniform(1e-4, 1e-3, (2, K // 128)).astype(np.float32)
        sa_d, sw_d = sa.astype(np.float64), sw.astype(np.float64)
    else:
        q, sa = oracle.act_quant_fp8(x)
        sw = rng.integers(118, 126, (2, K // 128), dtype=np.uint8)
        sa_d, sw_d = 2.0 ** (sa.astype(int) - 127), 2.0 ** (sw.astype(int) - 127)
    wq = rng.integers(0, 256, (N, K), dtype=np.uint8)
    wq[(wq & 0x7F) == 0x7F] = 0
    a = np.vectorize(e4m3_closed)(q) * np.repeat(sa_d, 128, axis=1)
    wv = np.vectorize(e4m3_closed)(wq) * np.repeat(np.repeat(sw_d, 128, axis=0), 128, axis=1)[:N]
    exact = a @ wv.T
    c16, c32 = oracle.gemm_w8a8(q, sa, wq, sw)
    assert np.max(np.abs(c32 - exact)) <= 2e-6 * np.max(np.abs(exact))
    assert np.allclose(oracle.gemm_w8a8_f64(q, sa, wq, sw), exact, rtol=1e-12, atol=1e-12 * np.abs(exact).max())


def test_gemm_grouped_fp8w_brute_force():
    """The grouped fp8-weight GEMM against numpy in fp64 from the formats' closed forms: group g of row m meets
    weight rows g R .. g R + R - 1, each scaled by its 128 x 128 block's e8m0 (a block straddling two groups when
    R % 128 != 0); the reference-order fp32 chain within fp32 rounding of the exact sums, its bf16 the RNE of it."""
    rng = np.random.default_rng(11)
    for M, G, R, K in ((3, 3, 200, 256), (2, 1, 128, 384), (1, 4, 64, 128)):
        a = randn_bf16(rng, (M, G, K))
        w = rng.integers(0, 256, (G * R, K), dtype=np.uint8)
        w[(w & 0x7F) == 0x7F] = 0
        sw = rng.integers(118, 130, ((G * R + 127) // 128, K // 128), dtype=np.uint8)
        wv = np.vectorize(e4m3_closed)(w) * np.repeat(np.repeat(2.0 ** (sw.astype(int) - 127), 128, axis=0),
                                                      128, axis=1)[:G * R]
        exact = np.einsum("mgk,grk->mgr", from_bf16(a).astype(np.float64), wv.reshape(G, R, K))
        c16, c32 = oracle.gemm_grouped_fp8w(a, w, sw, G, R)
        assert np.max(np.abs(c32 - exact)) <= 2e-6 * np.max(np.abs(exact))
        assert np.array_equal(c16, to_bf16(c32))
        c64 = oracle.gemm_grouped_fp8w_f64(a, w, sw, G, R)
        assert np.allclose(c64, exact, rtol=1e-12, atol=1e-12 * np.abs(exact).max())


def test_rmsnorm_quant_closed_form():
    """rmsnorm against fp64 w x / sqrt(mean(x^2) + eps): within the two roundings the reference applies (x * r to fp32,
    w * t to bf16); the output's quantization is act_quant_fp8 of it."""
    rng = np.random.default_rng(13)
    for rows, dim, eps in ((3, 4096, 1e-6), (2, 512, 1e-2), (1, 7168, 1e-6)):
        x = randn_bf16(rng, (rows, dim), scale=4.0)
        w = randn_bf16(rng, (dim,))
        y, q, qs = oracle.rmsnorm_quant(x, w, eps)
        xf, wf = from_bf16(x).astype(np.float64), from_bf16(w).astype(np.float64)
        exact = wf * xf / np.sqrt((xf ** 2).mean(axis=1, keepdims=True) + eps)
        err = np.abs(from_bf16(y) - exact)
        assert np.all(err <= 2.0 ** -8 * np.abs(exact) + 1e-30)
        q_ref, qs_ref = oracle.act_quant_fp8(y)
        assert np.array_equal(q, q_ref) and np.array_equal(qs, qs_ref)
        assert np.array_equal(oracle.rmsnorm_quant(x, w, eps, quant=False), y)


def _ulp32(v):
    """The fp32 ulp at |v| (float64 values), subnormal spacing below 2^-126."""
    e = np.floor(np.log2(np.maximum(np.abs(v), 2.0 ** -126)))
    return np.exp2(e - 23)


def test_exp_f32_within_2_ulp():
    """The library's e^x (IEEE operations only, shared bit for bit by the kernels and the oracle) against float64
    e^x: every 97th fp32 bit pattern of [-103.97, 88.72], every bf16 value, and the special cases."""
    hi = np.float32(88.7228394).view(np.uint32)
    lo = np.float32(103.972084).view(np.uint32)
    pos = np.arange(0, int(hi), 97, dtype=np.uint32).view(np.float32)
    neg = -np.arange(0, int(lo), 97, dtype=np.uint32).view(np.float32)
    bfv = (np.arange(65536, dtype=np.uint32) << 16).view(np.float32)
    bfv = bfv[np.isfinite(bfv) & (bfv < 88.72) & (bfv > -103.97)]
    for x in (pos, neg, bfv):
        y = oracle.exp_f32(x).astype(np.float64)
        want = np.exp(x.astype(np.float64))
        err = np.abs(y - want) / _ulp32(want)
        assert err.max() <= 2.0, (err.max(), x[np.argmax(err)])
    special = np.array([0.0, -0.0, 1.0, 89.0, 1e30, -104.0, -1e30, np.inf, -np.inf], np.float32)
    y = oracle.exp_f32(special)
    assert y[0] == 1.0 and y[1] == 1.0 and abs(y[2] - np.e) <= 2.4e-7
    assert np.isposinf(y[3]) and np.isposinf(y[4]) and np.isposinf(y[7])
    assert y[5] == 0.0 and y[6] == 0.0 and y[8] == 0.0
    assert np.isnan(oracle.exp_f32(np.array([np.nan], np.float32))[0])


# ---- MoE pieces ------------------------------------------------------------------------------------------------------------
@pytest.mark.parametrize("limit", [10.0, 0.0])
def test_swiglu_closed_form(limit):
    rng = np.random.default_rng(8)
    g, u = randn_bf16(rng, (6, 256), 8.0), randn_bf16(rng, (6, 256), 8.0)
    w = rng.random(6).astype(np.float32)
    h = oracle.swiglu(g, u, w, limit)
    gf, uf = from_bf16(g).astype(np.float64), from_bf16(u).astype(np.float64)
    if limit > 0:
        gf, uf = np.minimum(gf, limit), np.clip(uf, -limit, limit)
    want = w[:, None] * (gf / (1 + np.exp(-gf))) * uf
    assert np.all(np.abs(from_bf16(h) - want) <= np.abs(want) * 2 ** -8 + 1e-30)
    if limit > 0:
        assert np.all(np.abs(from_bf16(h)) <= limit * limit * 1.01)


def test_routers_brute_force():
    rng = np.random.default_rng(9)
    T, E, K = 40, 64, 6
    logits = rng.standard_normal((T, E)).astype(np.float32) * 2
    logits[0, 3] = logits[0, 50] = 50.0  # tie on the top key: lower id first
    bias = rng.standard_normal(E).astype(np.float32) * 0.3
    sel, wt = oracle.route_softmax(logits, K)
    assert list(sel[0, :2]) == [3, 50]
    for t in range(T):
        want = np.argsort(-logits[t].astype(np.float64), kind="stable")[:K]
        assert np.array_equal(sel[t], want)
        p = np.exp(logits[t].astype(np.float64) - logits[t].max())
        np.testing.assert_allclose(wt[t], p[want] / p[want].sum(), rtol=4e-6)  # fp32 rounding of l - m
    def check_topk(chosen, key, ordered):
        # fp32 keys against fp64 ones: the picks are the top K up to 1e-6 (near-ties may order either way)
        rest = np.setdiff1d(np.arange(E), chosen)
        assert key[chosen].min() >= key[rest].max() - 1e-6
        if ordered:
            assert np.all(np.diff(key[chosen]) <= 1e-6)

    sel, wt = oracle.route_ds(logits, bias, K, 2.0)
    score = np.sqrt(np.where(logits > 20, logits, np.log1p(np.exp(logits.astype(np.float64)))))
    for t in range(T):
        check_topk(sel[t], score[t] + bias, True)
        np.testing.assert_allclose(wt[t], score[t][sel[t]] / score[t][sel[t]].sum() * 2.0, rtol=1e-6)
    t2e = rng.integers(0, E, (100, K)).astype(np.int32)
    ids = rng.integers(0, 100, T).astype(np.int32)
    sel, _ = oracle.route_ds(logits, bias, K, 1.0, tid2eid=t2e, ids=ids)
    assert np.array_equal(sel, t2e[ids])  # hash layers take the table
    sel, wt = oracle.route_glm(logits, bias, K, 1.5)
    sig = 1 / (1 + np.exp(-logits.astype(np.float64)))
    for t in range(T):
        check_topk(sel[t], sig[t] + bias, False)
        assert np.all(np.diff(sel[t]) > 0)  # reported in ascending expert id
        np.testing.assert_allclose(wt[t], sig[t][sel[t]] / sig[t][sel[t]].sum() * 1.5, rtol=1e-6)


@pytest.mark.parametrize("tile_rows", [1, 8, 128])
def test_dispatch_invariants(tile_rows):
    rng = np.random.default_rng(10)
    T, E, K = 50, 16, 4
    sel = np.stack([rng.permutation(E)[:K] for _ in range(T)]).astype(np.int32)
    wt = rng.random((T, K)).astype(np.float32)
    resident = (rng.random(E) > 0.3).astype(np.uint8)
    d = oracle.dispatch(sel, wt, E, tile_rows, resident=resident)
    P = T * K
    assert d["plan"][0] == P and np.bincount(sel.ravel(), minlength=E).tolist() == d["count"].tolist()
    # resident experts first, each group in ascending id
    order = [e for e in range(E) if resident[e]] + [e for e in range(E) if not resident[e]]
    assert d["plan"][1] == sum(d["count"][e] for e in range(E) if resident[e])
    pos = 0
    for e in order:
        assert d["off"][e] == pos
        rows = np.arange(pos, pos + d["count"][e])
        assert np.all(d["row_expert"][rows] == e)
        assert np.all(np.diff(d["eidx"][rows]) > 0)  # tokens ascending within an expert
        pos += d["count"][e]
    for t in range(T):
        ex = d["row_expert"][d["pidx"][t]]
        assert np.all(np.diff(ex) > 0)  # each token's pairs in ascending expert order
        assert sorted(ex.tolist()) == sorted(sel[t].tolist())
        assert np.all(d["eidx"][d["pidx"][t]] == t)
        for j, p in enumerate(d["pidx"][t]):
            assert d["ewt"][p] == wt[t][list(sel[t]).index(d["row_expert"][p])]
    covered = sorted(r for e_, r0, n in d["tiles"] for r in range(r0, r0 + n))
    assert covered == list(range(d["plan"][1]))
    assert all(1 <= n <= tile_rows for _, _, n in d["tiles"])


def test_combine_fixed_order():
    rng = np.random.default_rng(11)
    T, K, D = 5, 3, 64
    pair = randn_bf16(rng, (T * K, D))
    pidx = rng.permutation(T * K).reshape(T, K).astype(np.int32)
    shared = randn_bf16(rng, (T, D))
    out = oracle.moe_combine(pair, pidx, shared)
    acc = np.zeros((T, D), np.float32)
    for j in range(K):
        acc = acc + from_bf16(pair[pidx[:, j]])
    acc = acc + from_bf16(shared)
    assert np.array_equal(out, to_bf16(acc))


def test_moe_forward_composition():
    """The routed-expert FFN against an independent fp64 composition of the same quantized steps (act_quant ->
    a8w4 -> SwiGLU -> act_quant -> a8w4 -> sum): differences only from fp32 sums and bf16 roundings."""
    rng = np.random.default_rng(12)
    T, E, K, D, I, limit = 6, 8, 3, 256, 128, 10.0
    experts = []
    for _ in range(E):
        ex = {}
        for (wn, sn), (n, k) in ((("w1", "s1"), (I, D)), (("w3", "s3"), (I, D)), (("w2", "s2"), (D, I))):
            ex[wn], ex[sn] = mx_weights(rng, n, k)
        experts.append(ex)
    x = randn_bf16(rng, (T, D))
    sel, wt = oracle.route_softmax(rng.standard_normal((T, E)).astype(np.float32), K)
    out, _ = oracle.moe_forward(x, sel, wt, experts, D, I, limit, tiled=False)
    want = np.zeros((T, D))
    for t in range(T):
        for j in range(K):
            ex = experts[sel[t, j]]
            q, qs = oracle.act_quant_fp8(x[t:t + 1])
            # the reference keeps g and u as bf16 tensors (forward_ref.hip:297-300)
            g = from_bf16(to_bf16(_a8w4_f64_numpy(q, qs, ex["w1"], ex["s1"]).astype(np.float32))).astype(np.float64)
            u = from_bf16(to_bf16(_a8w4_f64_numpy(q, qs, ex["w3"], ex["s3"]).astype(np.float32))).astype(np.float64)
            gc, uc = np.minimum(g, limit), np.clip(u, -limit, limit)
            h = wt[t, j] * gc / (1 + np.exp(-gc)) * uc
            q2, s2 = oracle.act_quant_fp8(to_bf16(h.astype(np.float32)))
            want[t] += _a8w4_f64_numpy(q2, s2, ex["w2"], ex["s2"])[0]
    got = from_bf16(out).astype(np.float64)
    rel = np.linalg.norm(got - want) / np.linalg.norm(want)
    assert rel < 5e-3, rel  # bf16 pair rows and output (2^-9 each) and the rare fp8 code flip they cause


def _fake_quant_fp4_closed(x_bf16, block):
    """An independent statement of e2m1 fake quantization (ref_elem.hip:43-59): per block, sc = the smallest power of
    two >= max(amax, 6 * 2^-126) / 6 (from frexp, no logarithms), each value clamped to +-6 after division by sc and
    moved to the nearest e2m1 grid value, a tie going to the even code (codes 0..7 = 0, .5, 1, 1.5, 2, 3, 4, 6)."""
    grid = np.array([0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0])
    xf = from_bf16(x_bf16).astype(np.float64)
    rows, cols = xf.shape
    out = np.empty_like(xf)
    for r in range(rows):
        for b in range(cols // block):
            v = xf[r, b * block:(b + 1) * block]
            amax = max(np.abs(v).max(), 6.0 * 2.0 ** -126)
            m, e = np.frexp(np.float32(amax) * np.float32(1 / 6))  # the kernel's fp32 product, then 2^ceil(log2)
            sc = 2.0 ** (e - 1) if m == 0.5 else 2.0 ** e
            y = np.clip(v / sc, -6.0, 6.0)
            d = np.abs(np.abs(y)[:, None] - grid[None, :])
            best = d.min(axis=1, keepdims=True)
            cand = d == best
            # a tie is between neighbouring codes, exactly one of them even
            even = np.argmax(cand & (np.arange(8) % 2 == 0), axis=1)
            code = np.where(cand.sum(axis=1) > 1, even, np.argmax(cand, axis=1))
            out[r, b * block:(b + 1) * block] = np.copysign(grid[code], y) * sc
    return out.astype(np.float32)


@pytest.mark.parametrize("block", [32, 64, 128])
def test_fake_quant_fp4_closed_form(block):
    rng = np.random.default_rng(40 + block)
    x = randn_bf16(rng, (7, 256), 3.0)
    x[0, :block] = 0                                    # all-zero block: the amax floor
    x[1, :block] = to_bf16(np.full(block, 1e-39, np.float32))  # below the floor
    ties = np.array([0.25, 0.75, 1.25, 1.75, 2.5, 3.5, 5.0, -0.25, -2.5, -5.0, 6.0, -6.0], np.float32)
    x[2, :len(ties)] = to_bf16(ties)                  # amax 6 -> sc = 1: every tie at its midpoint
    x[3, :block] = to_bf16(np.linspace(-70, 70, block, dtype=np.float32))
    got = from_bf16(oracle.fake_quant_fp4(x, block))
    want = _fake_quant_fp4_closed(x, block)
    assert np.array_equal(got.view(np.uint32) & 0x7FFFFFFF, want.view(np.uint32) & 0x7FFFFFFF)
    assert np.array_equal(np.signbit(got) & (got != 0), np.signbit(want) & (want != 0))
    # the ties row: midpoints to the even code
    assert got[2, :len(ties)].tolist() == [0.0, 1.0, 1.0, 2.0, 2.0, 4.0, 4.0, -0.0, -2.0, -4.0, 6.0, -6.0]
