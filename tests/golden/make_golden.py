"""Writes the small golden fixtures under tests/golden/ from the CPU oracle (the reference's arithmetic restated in
oracle/uh_oracle.cpp). The reference commits no fixtures for this path (its kernel tests draw random data at run
time), so these are the portable known-answer vectors: inputs from numpy's PCG64 with fixed seeds, outputs from the
oracle. Regenerate with `python tests/golden/make_golden.py`; tests/test_golden.py checks the oracle still
reproduces them and the GPU tests check the kernels against them.
"""
import pathlib
import sys

import numpy as np

HERE = pathlib.Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parents[1]))

import oracle  # noqa: E402
from tests.helpers import mx_weights, randn_bf16  # noqa: E402


def main():
    rng = np.random.default_rng(20261201)
    # 1. one MXFP4 GEMV / small GEMM (configs[0] in miniature): x [3, 512], W [64, 512]
    N, K = 64, 512
    x = randn_bf16(rng, (3, K))
    w, s = mx_weights(rng, N, K)
    q, qs = oracle.act_quant_fp8(x)
    tw, ts = oracle.repack(w, s, N, K)
    y16, y32 = oracle.gemm_a8w4(q, qs, w, s, N)
    np.savez_compressed(HERE / "mx_gemv.npz", x=x, w=w, s=s, q=q, qs=qs, tw=tw, ts=ts, y16=y16, y32=y32)
    # 2. routing + dispatch (configs[1] shape: 8 tokens, 256 experts, top 6)
    logits = rng.standard_normal((8, 256)).astype(np.float32)
    sel, wt = oracle.route_softmax(logits, 6)
    d = oracle.dispatch(sel, wt, 256, tile_rows=16)
    np.savez_compressed(HERE / "routing.npz", logits=logits, sel=sel, wt=wt, eidx=d["eidx"], ewt=d["ewt"],
                        row_expert=d["row_expert"], pidx=d["pidx"], tiles=d["tiles"], plan=d["plan"])
    # 3. a whole routed-expert FFN, miniature: T 5, E 8, top 3, D 256, I 128, limit 10
    T, E, KT, D, I = 5, 8, 3, 256, 128
    arrs = {}
    experts = []
    for e in range(E):
        ex = {}
        for (wn, sn), (n, k) in ((("w1", "s1"), (I, D)), (("w3", "s3"), (I, D)), (("w2", "s2"), (D, I))):
            ww, ss = mx_weights(rng, n, k)
            ex[wn], ex[sn] = oracle.repack(ww, ss, n, k)
            arrs[f"{wn}_{e}"], arrs[f"{sn}_{e}"] = ex[wn], ex[sn]
        experts.append(ex)
    x = randn_bf16(rng, (T, D))
    logits = rng.standard_normal((T, E)).astype(np.float32)
    sel, wt = oracle.route_softmax(logits, KT)
    out, pair = oracle.moe_forward(x, sel, wt, experts, D, I, 10.0)
    np.savez_compressed(HERE / "moe_ffn.npz", x=x, logits=logits, sel=sel, wt=wt, out=out, pair=pair, **arrs)
    # 4. fp8 dense with fp32 scales (configs[4] form), M 2, N 256, K 256
    a = randn_bf16(rng, (2, 256))
    aq, sa = oracle.act_quant_fp8_f32s(a)
    wq = rng.integers(0, 256, (256, 256), dtype=np.uint8)
    wq[(wq & 0x7F) == 0x7F] = 0
    sw = rng.uniform(1e-4, 1e-3, (2, 2)).astype(np.float32)
    c16, c32 = oracle.gemm_w8a8(aq, sa, wq, sw)
    np.savez_compressed(HERE / "fp8_dense.npz", a=a, aq=aq, sa=sa, wq=wq, sw=sw, c16=c16, c32=c32)
    print("wrote", sorted(p.name for p in HERE.glob("*.npz")))


if __name__ == "__main__":
    main()
