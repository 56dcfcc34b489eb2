"""Pins of the oracle's remote-expert functions (no GPU): remote_tokens against an independent numpy statement of
its definition; the partial combine against moe_combine where the two sum in the same order (each token's only
remote pick is its last one and crosses remote_combine unchanged), and against fp64 sums in general; the mHC
post-mix against its closed form."""
import numpy as np
import pytest

import oracle
from tests.helpers import randn_bf16


def _routed(rng, T, E, K, remote_frac):
    sel = np.stack([rng.permutation(E)[:K] for _ in range(T)]).astype(np.int32)
    wt = rng.random((T, K)).astype(np.float32)
    resident = (rng.random(E) >= remote_frac).astype(np.uint8)
    return sel, wt, resident, oracle.dispatch(sel, wt, E, 16, resident)


@pytest.mark.parametrize("T,E,K,frac", [(1, 8, 2, 0.5), (40, 64, 6, 0.3), (300, 256, 6, 0.0), (50, 16, 4, 1.0)])
def test_remote_tokens_matches_numpy(T, E, K, frac):
    rng = np.random.default_rng(T + K)
    sel, _, resident, d = _routed(rng, T, E, K, frac)
    r0 = d["plan"][1]
    got = oracle.remote_tokens(d["pidx"], d["eidx"], r0)
    remote_pick = resident[sel] == 0                       # [T, K]: the pick's expert is not held here
    flag = remote_pick.any(axis=1)
    assert np.array_equal(d["pidx"] >= r0, np.take_along_axis(remote_pick, np.argsort(sel, axis=1), axis=1))
    u = np.cumsum(flag) - 1
    assert got["U"] == flag.sum()
    assert np.array_equal(got["tok2u"], np.where(flag, u, -1))
    assert np.array_equal(got["u2t"], np.nonzero(flag)[0])
    assert np.array_equal(got["p2u"][r0:], u[d["eidx"][r0:]])
    exp_u2p = np.where(d["pidx"] >= r0, d["pidx"], -1)[flag]
    assert np.array_equal(got["u2p"], exp_u2p)


def test_partial_combine_reduces_to_moe_combine():
    rng = np.random.default_rng(3)
    T, E, K, D = 24, 32, 4, 256
    resident = np.ones(E, np.uint8)
    resident[E - 4:] = 0  # the four highest experts are remote
    sel = np.empty((T, K), np.int32)
    for t in range(T):  # K-1 resident picks and, for odd tokens, one remote pick
        loc = rng.permutation(E - 4)[:K]
        sel[t] = loc if t % 2 == 0 else np.append(loc[:K - 1], E - 4 + t % 4)
    wt = rng.random((T, K)).astype(np.float32)
    d = oracle.dispatch(sel, wt, E, 16, resident)
    r0 = d["plan"][1]
    pair_out = randn_bf16(rng, (T * K, D))
    shared = randn_bf16(rng, (T, D))
    rt = oracle.remote_tokens(d["pidx"], d["eidx"], r0)
    partial = oracle.remote_combine(pair_out, rt["u2p"])
    assert np.array_equal(partial, pair_out[rt["u2p"].max(axis=1)])  # one row: unchanged through the sum
    got = oracle.moe_combine_partial(pair_out, d["pidx"], r0, rt["tok2u"], partial, shared)
    assert np.array_equal(got, oracle.moe_combine(pair_out, d["pidx"], shared))


def test_partial_combine_close_to_fp64_and_hc_post():
    rng = np.random.default_rng(5)
    T, E, K, D, hc = 10, 16, 6, 64, 4
    sel, wt, resident, d = _routed(rng, T, E, K, 0.5)
    r0 = d["plan"][1]
    pair_out = randn_bf16(rng, (T * K, D))
    shared = randn_bf16(rng, (T, D))
    rt = oracle.remote_tokens(d["pidx"], d["eidx"], r0)
    partial = oracle.remote_combine(pair_out, rt["u2p"])
    f = oracle.bf16_to_f32(pair_out).astype(np.float64)
    exact = f[d["pidx"]].sum(axis=1) + oracle.bf16_to_f32(shared)
    x = randn_bf16(rng, (T, hc, D))
    post = rng.random((T, hc)).astype(np.float32)
    comb = rng.random((T, hc, hc)).astype(np.float32)
    out, xo = oracle.moe_combine_partial(pair_out, d["pidx"], r0, rt["tok2u"], partial, shared, x, post, comb)
    o = oracle.bf16_to_f32(out).astype(np.float64)
    assert np.abs(o - exact).max() <= 2e-2 * np.abs(exact).max()
    xf = oracle.bf16_to_f32(x).astype(np.float64)
    want = post[:, :, None] * o[:, None, :] + np.einsum("tij,tid->tjd", comb.astype(np.float64), xf)
    np.testing.assert_allclose(oracle.bf16_to_f32(xo), want, rtol=8e-3, atol=1e-6)
    # hc = 1, post 1, comb 0: the stream becomes the output exactly
    one = oracle.moe_combine_partial(pair_out, d["pidx"], r0, rt["tok2u"], partial, shared, x[:, :1],
                                     np.ones((T, 1), np.float32), np.zeros((T, 1, 1), np.float32))
    assert np.array_equal(one[1][:, 0], out)


def test_hc_post_closed_forms():
    rng = np.random.default_rng(8)
    T, hc, D = 5, 4, 96
    x = randn_bf16(rng, (T, D))
    res = randn_bf16(rng, (T, hc, D))
    eye = np.broadcast_to(np.eye(hc, dtype=np.float32), (T, hc, hc))
    assert np.array_equal(oracle.hc_post(x, res, np.zeros((T, hc), np.float32), eye), res)  # comb = I, post = 0
    one = oracle.hc_post(x, res[:, :1], np.ones((T, 1), np.float32), np.zeros((T, 1, 1), np.float32))
    assert np.array_equal(one[:, 0], x)  # hc = 1, post = 1, comb = 0
    post = rng.random((T, hc)).astype(np.float32)
    comb = rng.random((T, hc, hc)).astype(np.float32)
    got = oracle.bf16_to_f32(oracle.hc_post(x, res, post, comb))
    want = (post[:, :, None] * oracle.bf16_to_f32(x).astype(np.float64)[:, None, :]
            + np.einsum("tij,tid->tjd", comb.astype(np.float64), oracle.bf16_to_f32(res).astype(np.float64)))
    np.testing.assert_allclose(got, want, rtol=8e-3, atol=1e-6)
