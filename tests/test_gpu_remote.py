"""GPU parity of the remote-expert kernels (the compact transport around experts held elsewhere), at one GPU's
share: the exchange itself needs a second device, so the remote side's buffers are device buffers here. Every
output bit-exact against the CPU oracle; extents past the device-side counts untouched."""
import ctypes

import numpy as np
import pytest

import oracle
from tests.helpers import randn_bf16
from unholy_amd import call
from unholy_amd.device import DeviceBuffer, synchronize

pytestmark = pytest.mark.gpu


def dev(a):
    return DeviceBuffer.from_array(np.ascontiguousarray(a))


def filled(shape, dtype, v):
    return dev(np.full(shape, v, dtype))


def _routed(rng, T, E, K, frac, tile_rows=16):
    sel = np.stack([rng.permutation(E)[:K] for _ in range(T)]).astype(np.int32)
    wt = rng.random((T, K)).astype(np.float32)
    resident = (rng.random(E) >= frac).astype(np.uint8)
    return sel, wt, resident, oracle.dispatch(sel, wt, E, tile_rows, resident)


@pytest.mark.parametrize("T,E,K,frac", [(1, 8, 2, 1.0), (40, 64, 6, 0.3), (1500, 256, 6, 0.5), (300, 256, 6, 0.0),
                                         (4097, 256, 6, 0.5), (9000, 64, 4, 0.2)])
def test_remote_tokens(T, E, K, frac):
    rng = np.random.default_rng(T + E)
    _, _, _, d = _routed(rng, T, E, K, frac)
    P, r0 = T * K, d["plan"][1]
    ref = oracle.remote_tokens(d["pidx"], d["eidx"], r0)
    plan = dev(d["plan"])
    tok2u, u2t = filled(T, np.int32, -7), filled(T, np.int32, -7)
    p2u, u2p = filled(P, np.int32, -7), filled((T, K), np.int32, -7)
    call("uh_remote_tokens", dev(d["pidx"]), dev(d["eidx"]), T, K, plan, tok2u, u2t, p2u, u2p, None)
    U = ref["U"]
    print(f"remote_tokens T={T} E={E}: U={U} remote0={r0}")
    assert plan.download(5, np.int32)[4] == U
    assert np.array_equal(tok2u.download(T, np.int32), ref["tok2u"])
    assert np.array_equal(u2t.download(T, np.int32)[:U], ref["u2t"])
    assert (u2t.download(T, np.int32)[U:] == -7).all()
    got_p2u = p2u.download(P, np.int32)
    assert np.array_equal(got_p2u[r0:], ref["p2u"][r0:]) and (got_p2u[:r0] == -7).all()
    assert np.array_equal(u2p.download((T, K), np.int32)[:U], ref["u2p"])


@pytest.mark.parametrize("T,D,hc", [(40, 4096, 0), (40, 4096, 4), (7, 1000, 2), (1, 512, 1)])
def test_remote_combine_and_partial_combines(T, D, hc):
    rng = np.random.default_rng(T * 3 + D + hc)
    E, K = 64, 6
    _, _, _, d = _routed(rng, T, E, K, 0.4)
    P, r0 = T * K, d["plan"][1]
    ref_rt = oracle.remote_tokens(d["pidx"], d["eidx"], r0)
    U = ref_rt["U"]
    plan = d["plan"].copy()
    plan[4] = U
    pair_out = randn_bf16(rng, (P, D))
    shared = randn_bf16(rng, (T, D))
    dplan, dpidx, dtok2u = dev(plan), dev(d["pidx"]), dev(ref_rt["tok2u"])
    dpair, dshared = dev(pair_out), dev(shared)
    if D % 8 == 0:
        partial = filled((max(U, 1), D), np.uint16, 0x7FC1)
        call("uh_remote_combine", dpair, dev(ref_rt["u2p"] if U else np.zeros((1, K), np.int32)), dplan, partial, K,
             D, T, None)
        ref_partial = oracle.remote_combine(pair_out, ref_rt["u2p"])
        assert np.array_equal(partial.download((max(U, 1), D), np.uint16)[:U], ref_partial)
    else:  # remote_combine needs whole 16-byte rows; the partial rows come from the oracle
        ref_partial = oracle.remote_combine(pair_out, ref_rt["u2p"])
        partial = dev(ref_partial if U else np.zeros((1, D), np.uint16))
    x = randn_bf16(rng, (T, max(hc, 1), D))
    post = rng.random((T, max(hc, 1))).astype(np.float32)
    comb = rng.random((T, max(hc, 1), max(hc, 1))).astype(np.float32)
    ref = oracle.moe_combine_partial(pair_out, d["pidx"], r0, ref_rt["tok2u"], ref_partial, shared,
                                     x if hc else None, post if hc else None, comb if hc else None)
    ref_out, ref_x = ref if hc else (ref, None)
    # the link form: the partial read from its own rows
    out, dx = DeviceBuffer(T * D * 2), dev(x)
    call("uh_moe_combine_partial_link", dpair, dpidx, dplan, dtok2u, partial, dshared, out, T, K, D,
         dx if hc else None, dev(post) if hc else None, dev(comb) if hc else None, hc, None)
    got = out.download((T, D), np.uint16)
    print(f"combine_partial_link T={T} D={D} hc={hc}: bit-identical {np.mean(got == ref_out):.6f}")
    assert np.array_equal(got, ref_out)
    if hc:
        assert np.array_equal(dx.download(x.shape, np.uint16), ref_x)
    # the copy form: the partial rows placed at rows remote0.. of pair_out first
    if D % 8 == 0:
        call("uh_copy_remote_partial", partial, dpair, dplan, D, T, None)
        full = dpair.download((P, D), np.uint16)
        assert np.array_equal(full[r0:r0 + U], ref_partial)
        assert np.array_equal(full[:r0], pair_out[:r0]) and np.array_equal(full[r0 + U:], pair_out[r0 + U:])
        out2 = DeviceBuffer(T * D * 2)
        call("uh_moe_combine_partial", dpair, dpidx, dplan, dtok2u, dshared, out2, T, K, D, None)
        assert np.array_equal(out2.download((T, D), np.uint16), ref_out)


def test_stage_and_copies():
    rng = np.random.default_rng(11)
    T, E, K, D = 30, 64, 6, 1024
    _, _, _, d = _routed(rng, T, E, K, 0.5)
    P, r0 = T * K, d["plan"][1]
    rt = oracle.remote_tokens(d["pidx"], d["eidx"], r0)
    U = rt["U"]
    plan = d["plan"].copy()
    plan[4] = U
    nrt = plan[3]
    dplan = dev(plan)
    rtiles = np.zeros((P + E, 3), np.int32)
    rtiles[:nrt] = d["remote_tiles"]
    plan_dst, tiles_dst = filled(5, np.int32, -1), filled((P + E, 3), np.int32, -1)
    w_dst, e_dst = filled(P, np.float32, -1.0), filled(P, np.int32, -1)
    call("uh_stage_remote", dplan, dev(rtiles), dev(d["ewt"]), dev(d["row_expert"]), plan_dst, tiles_dst, w_dst,
         e_dst, P, None)
    assert np.array_equal(plan_dst.download(5, np.int32), plan)
    td = tiles_dst.download((P + E, 3), np.int32)
    assert np.array_equal(td[:nrt], d["remote_tiles"]) and (td[nrt:] == -1).all()
    for got, want, fill in ((w_dst.download(P, np.float32), d["ewt"], -1.0),
                            (e_dst.download(P, np.int32), d["row_expert"], -1)):
        assert np.array_equal(got[r0:], want[r0:]) and (got[:r0] == fill).all()
    w2, e2 = filled(P, np.float32, -1.0), filled(P, np.int32, -1)
    call("uh_copy_remote_meta", dev(d["ewt"]), dev(d["row_expert"]), w2, e2, dplan, P, None)
    assert np.array_equal(w2.download(P, np.float32), w_dst.download(P, np.float32))
    assert np.array_equal(e2.download(P, np.int32), e_dst.download(P, np.int32))
    src = randn_bf16(rng, (P, D))
    dst = filled((P, D), np.uint16, 0x1234)
    call("uh_copy_remote_rows", dev(src), dst, dplan, D, P, None)
    got = dst.download((P, D), np.uint16)
    assert np.array_equal(got[r0:], src[r0:]) and (got[:r0] == 0x1234).all()
    x = randn_bf16(rng, (T, D))
    xd = filled((T, D), np.uint16, 0x4321)
    call("uh_copy_remote_tokens", dev(x), D, dev(rt["u2t"] if U else np.zeros(1, np.int32)), dplan, xd, T, None)
    got = xd.download((T, D), np.uint16)
    assert np.array_equal(got[:U], x[rt["u2t"]]) and (got[U:] == 0x4321).all()


@pytest.mark.parametrize("T,E,K,frac,tile_rows,dim", [(8, 256, 6, 0.5, 8, 4096), (32, 64, 8, 0.3, 4, 1024),
                                                      (1, 16, 2, 1.0, 8, 512), (20, 256, 6, 0.0, 16, 4096)])
def test_dispatch_small_remote(T, E, K, frac, tile_rows, dim):
    """moe_dispatch_small with a resident mask and every remote-side output, against the host-order dispatch,
    remote_tokens, the remote tokens' rows and their act_quant_fp8."""
    rng = np.random.default_rng(T + E + K)
    sel, wt, resident, d = _routed(rng, T, E, K, frac, tile_rows)
    P, r0 = T * K, d["plan"][1]
    rt = oracle.remote_tokens(d["pidx"], d["eidx"], r0)
    U = rt["U"]
    mt = P + E
    x = randn_bf16(rng, (T, dim), scale=2.0)
    o = {n: filled(s, t, v) for n, s, t, v in [
        ("plan", 5, np.int32, -1), ("tiles", (mt, 3), np.int32, -1), ("rtiles", (mt, 3), np.int32, -1),
        ("eidx", P, np.int32, -1), ("ewt", P, np.float32, -1), ("rex", P, np.int32, -1), ("pidx", (T, K), np.int32, -1),
        ("tok2u", T, np.int32, -9), ("u2t", T, np.int32, -9), ("p2u", P, np.int32, -9), ("u2p", (T, K), np.int32, -9),
        ("plan_dst", 5, np.int32, -1), ("tiles_dst", (mt, 3), np.int32, -1), ("w_dst", P, np.float32, -1),
        ("e_dst", P, np.int32, -1), ("x_dst", (T, dim), np.uint16, 0x5555), ("q", (T, dim), np.uint8, 0xAB),
        ("qs", (T, dim // 128), np.uint8, 0xCD), ("flag", 1, np.uint32, 0)]}
    call("uh_moe_dispatch_small_remote", dev(sel), dev(wt), T, K, E, P, mt, tile_rows, o["plan"], o["tiles"],
         o["rtiles"], o["eidx"], o["ewt"], o["rex"], o["pidx"], dev(resident), None, None, 0.0, 1, 1, o["tok2u"],
         o["u2t"], o["p2u"], o["u2p"], o["plan_dst"], o["tiles_dst"], o["w_dst"], o["e_dst"], dev(x), dim,
         o["x_dst"], o["q"], o["qs"], o["flag"], 77, None)
    synchronize()
    g = lambda n, s, t: o[n].download(s, t)  # noqa: E731
    plan = g("plan", 5, np.int32)
    want_plan = d["plan"].copy()
    want_plan[4] = U
    print(f"dispatch_small_remote T={T} E={E}: remote0={r0} U={U} plan={plan.tolist()}")
    assert np.array_equal(plan, want_plan)
    assert np.array_equal(g("plan_dst", 5, np.int32), want_plan)
    nl, nr = plan[2], plan[3]
    assert np.array_equal(g("tiles", (mt, 3), np.int32)[:nl], d["tiles"][:nl])
    assert np.array_equal(g("rtiles", (mt, 3), np.int32)[:nr], d["remote_tiles"])
    assert np.array_equal(g("tiles_dst", (mt, 3), np.int32)[:nr], d["remote_tiles"])
    for n, key, t in (("eidx", "eidx", np.int32), ("ewt", "ewt", np.float32), ("rex", "row_expert", np.int32)):
        assert np.array_equal(g(n, P, t), d[key]), n
    assert np.array_equal(g("pidx", (T, K), np.int32), d["pidx"])
    for n, key, t, fill in (("w_dst", "ewt", np.float32, -1), ("e_dst", "row_expert", np.int32, -1)):
        v = g(n, P, t)
        assert np.array_equal(v[r0:], d[key][r0:]) and (v[:r0] == fill).all(), n
    assert np.array_equal(g("tok2u", T, np.int32), rt["tok2u"])
    assert np.array_equal(g("u2t", T, np.int32)[:U], rt["u2t"])
    assert np.array_equal(g("p2u", P, np.int32)[r0:], rt["p2u"][r0:])
    assert np.array_equal(g("u2p", (T, K), np.int32)[:U], rt["u2p"])
    xd = g("x_dst", (T, dim), np.uint16)
    assert np.array_equal(xd[:U], x[rt["u2t"]]) and (xd[U:] == 0x5555).all()
    q, qs = g("q", (T, dim), np.uint8), g("qs", (T, dim // 128), np.uint8)
    if U:
        q_ref, s_ref = oracle.act_quant_fp8(x[rt["u2t"]])
        assert np.array_equal(q[:U], q_ref) and np.array_equal(qs[:U], s_ref)
    assert (q[U:] == 0xAB).all() and (qs[U:] == 0xCD).all()
    assert g("flag", 1, np.uint32)[0] == 77


def test_dispatch_small_remote_rejects_inconsistent_args():
    from unholy_amd._lib import UhError
    b = DeviceBuffer(4096)
    with pytest.raises(UhError, match="remote without a resident mask"):
        call("uh_moe_dispatch_small_remote", b, b, 2, 2, 8, 4, 12, 8, b, b, b, b, b, b, b, None, None, None, 0.0, 1, 0,
             None, None, None, None, b, b, b, b, None, 0, None, None, None, None, 0, None)
    with pytest.raises(UhError, match="need qin"):
        call("uh_moe_dispatch_small_remote", b, b, 2, 2, 8, 4, 12, 8, b, b, b, b, b, b, b, b, None, None, 0.0, 1, 0,
             None, None, None, None, b, b, b, b, b, 128, b, None, None, None, 0, None)


@pytest.mark.parametrize("T,K", [(40, 4096), (1, 1024), (300, 2048)])
def test_xform_in_q_matches_gathered_rows(T, K):
    """The remote side's input transform from compact fp8 tokens equals mx_xform_in / mx_xform_in_fp8 on the pair
    rows gathered from the tokens, bit for bit, and the oracle's fake_quant_fp8 / act_quant_fp8 of those rows; rows of
    experts absent from the table and rows below remote0 untouched."""
    rng = np.random.default_rng(T + K)
    E, Kp = 64, 6
    _, _, resident, d = _routed(rng, T, E, Kp, 0.5)
    P, r0 = T * Kp, d["plan"][1]
    rt = oracle.remote_tokens(d["pidx"], d["eidx"], r0)
    U = rt["U"]
    x = randn_bf16(rng, (T, K), scale=3.0)
    plan = d["plan"].copy()
    plan[4] = U
    dplan, dx = dev(plan), dev(x)
    q, qs = DeviceBuffer(max(U, 1) * K), DeviceBuffer(max(U, 1) * K // 128)
    call("uh_quant_remote_tokens", dx, K, dev(rt["u2t"] if U else np.zeros(1, np.int32)), dplan, q, qs, T, None)
    # the remote side holds the non-resident experts, except expert `gone` (its rows must stay untouched)
    held = resident == 0
    gone = int(np.nonzero(held)[0][0]) if held.any() else -1
    if gone >= 0:
        held[gone] = False
    s_tab = DeviceBuffer.from_array(np.where(held, 0x1000, 0).astype(np.uint64))
    p2u = np.full(P, 0, np.int32)
    p2u[r0:] = rt["p2u"][r0:]
    dp2u, drex = dev(p2u), dev(d["row_expert"])
    xa = filled((P, K), np.uint16, 0x7E57)
    call("uh_mx_xform_in_q", q, qs, dp2u, dplan, drex, s_tab, xa, P, K, None)
    got = xa.download((P, K), np.uint16)
    live = np.zeros(P, bool)
    live[r0:] = held[d["row_expert"][r0:]]
    gathered = x[d["eidx"]]
    print(f"xform_in_q T={T} K={K}: U={U} rebuilt rows {live.sum()}")
    assert np.array_equal(got[live], oracle.fake_quant_fp8(gathered[live]))
    assert (got[~live] == 0x7E57).all()
    xa2 = filled((P, K), np.uint16, 0x7E57)  # mx_xform_in on the gathered rows, restricted to the same rows
    tab2 = DeviceBuffer.from_array(np.where(held, 0x1000, 0).astype(np.uint64))
    call("uh_mx_xform_in", dx, K, drex, tab2, xa2, P, K, None, dev(d["eidx"]))
    assert np.array_equal(xa2.download((P, K), np.uint16)[live], got[live])
    qo, qso = filled((P, K), np.uint8, 0xEE), filled((P, K // 128), np.uint8, 0xEE)
    call("uh_mx_xform_in_q_fp8", q, qs, dp2u, dplan, drex, s_tab, qo, qso, P, K, None)
    q_ref, s_ref = oracle.act_quant_fp8(gathered[live]) if live.any() else (None, None)
    gq, gs = qo.download((P, K), np.uint8), qso.download((P, K // 128), np.uint8)
    if live.any():
        assert np.array_equal(gq[live], q_ref) and np.array_equal(gs[live], s_ref)
    assert (gq[~live] == 0xEE).all() and (gs[~live] == 0xEE).all()


@pytest.mark.parametrize("T,E,K,tile_rows,frac", [(4096, 256, 6, 128, 0.5), (100, 16, 4, 8, 0.25), (33, 64, 8, 16, 1.0)])
def test_dispatch_multi_kernel_resident(T, E, K, tile_rows, frac):
    """moe_count + moe_plan(resident) + moe_scatter against the host-order dispatch: resident rows first, then the
    others, each expert-ascending; local and remote tiles; remote0."""
    rng = np.random.default_rng(T + 1)
    sel, wt, resident, d = _routed(rng, T, E, K, frac, tile_rows)
    P = T * K
    mt = P // tile_rows + E + 1
    count = DeviceBuffer(E * 4)
    count.zero()
    off, fill, plan = DeviceBuffer(E * 4), DeviceBuffer(E * 4), DeviceBuffer(20)
    lt, rtl = DeviceBuffer(mt * 12), DeviceBuffer(mt * 12)
    eidx, ewt, rex, pidx = (DeviceBuffer(P * 4) for _ in range(4))
    dsel, dwt = dev(sel), dev(wt)
    call("uh_moe_count", dsel, T, K, count, E, None, None)
    call("uh_moe_plan", count, dev(resident), E, P, plan, lt, rtl, off, fill, mt, None, tile_rows)
    call("uh_moe_scatter", dsel, dwt, T, K, off, fill, eidx, ewt, rex, pidx, None)
    p = plan.download(5, np.int32)
    print(f"multi-kernel resident T={T}: plan={p.tolist()}")
    assert np.array_equal(p[:4], d["plan"][:4])
    assert np.array_equal(off.download(E, np.int32), d["off"])
    assert np.array_equal(eidx.download(P, np.int32), d["eidx"])
    assert np.array_equal(ewt.download(P, np.float32), d["ewt"])
    assert np.array_equal(rex.download(P, np.int32), d["row_expert"])
    assert np.array_equal(pidx.download((T, K), np.int32), d["pidx"])
    assert np.array_equal(lt.download((mt, 3), np.int32)[:p[2]], d["tiles"][:p[2]])
    assert np.array_equal(rtl.download((mt, 3), np.int32)[:p[3]], d["remote_tiles"])


def test_dispatch_small_resident_without_remote():
    """The resident split alone (remote off): plan, local and remote tiles, rows; no staging outputs needed."""
    rng = np.random.default_rng(99)
    T, E, K, tile_rows = 16, 128, 6, 8
    sel, wt, resident, d = _routed(rng, T, E, K, 0.5, tile_rows)
    P, mt = T * K, T * K + E
    o = {n: filled(s, t, -1) for n, s, t in [("plan", 5, np.int32), ("tiles", (mt, 3), np.int32),
                                             ("rtiles", (mt, 3), np.int32), ("eidx", P, np.int32),
                                             ("ewt", P, np.float32), ("rex", P, np.int32), ("pidx", (T, K), np.int32)]}
    call("uh_moe_dispatch_small_remote", dev(sel), dev(wt), T, K, E, P, mt, tile_rows, o["plan"], o["tiles"],
         o["rtiles"], o["eidx"], o["ewt"], o["rex"], o["pidx"], dev(resident), None, None, 0.0, 0, 0, None, None, None,
         None, None, None, None, None, None, 0, None, None, None, None, 0, None)
    p = o["plan"].download(5, np.int32)
    assert np.array_equal(p, d["plan"])
    assert np.array_equal(o["tiles"].download((mt, 3), np.int32)[:p[2]], d["tiles"][:p[2]])
    assert np.array_equal(o["rtiles"].download((mt, 3), np.int32)[:p[3]], d["remote_tiles"])
    assert np.array_equal(o["pidx"].download((T, K), np.int32), d["pidx"])
    assert np.array_equal(o["eidx"].download(P, np.int32), d["eidx"])


@pytest.mark.parametrize("T,ldo_pad", [(8, 0), (40, 128)])
def test_grouped_gemv_sums(T, ldo_pad):
    """mx_grouped_gemv with MxSums on the remote side (its tiles are the remote experts' rows): out is the plain
    GEMV's bit for bit, and sums.dst is remote_combine of those output rows (the oracle's)."""
    from tests.test_gpu_mx import _expert_tables, _make_experts
    from unholy_amd.device import pointer_table  # noqa: F401
    rng = np.random.default_rng(T + ldo_pad)
    E, Kp, N, K = 16, 4, 256, 512
    _, _, _, d = _routed(rng, T, E, Kp, 0.5, tile_rows=8)
    P, r0 = T * Kp, d["plan"][1]
    rt = oracle.remote_tokens(d["pidx"], d["eidx"], r0)
    U = rt["U"]
    plan = d["plan"].copy()
    plan[4] = U
    rtiles = d["remote_tiles"]
    nt = len(rtiles)
    assert nt > 0 and U > 0
    _, tabs = _expert_tables(_make_experts(rng, E, N, K), ("w", "s"))
    xa = dev(oracle.fake_quant_fp8(randn_bf16(rng, (P, K))))
    ldo = N + ldo_pad
    dtiles = dev(rtiles.astype(np.int32))
    out_a, out_b = filled((P, ldo), np.uint16, 0), filled((P, ldo), np.uint16, 0)
    call("uh_mx_grouped_gemv", xa, K, dtiles, nt, tabs["w"], tabs["s"], out_a, ldo, N, None, None, None, None, None, 8,
         None, None, None, None, 0.0, None)
    dst = filled((U, N), np.uint16, 0x7777)
    call("uh_mx_grouped_gemv_sums", xa, K, dtiles, nt, tabs["w"], tabs["s"], out_b, ldo, N, None, None, 8,
         dev(rt["u2p"]), dev(plan), Kp, dst, None)
    a, b = out_a.download((P, ldo), np.uint16), out_b.download((P, ldo), np.uint16)
    assert np.array_equal(a, b)
    ref = oracle.remote_combine(np.ascontiguousarray(b[:, :N]), rt["u2p"])
    got = dst.download((U, N), np.uint16)
    print(f"gemv sums T={T} ldo={ldo}: U={U}, tiles={nt}, bit-identical {np.mean(got == ref):.6f}")
    assert np.array_equal(got, ref)
