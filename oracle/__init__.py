"""ctypes binding of the CPU oracle (oracle/uh_oracle.cpp) and of oracle/_ref (the reference's own host code).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg, as the
checker or the timed CPU baseline, never by the product (unholy_amd/). Every function takes and returns numpy
arrays; see uh_oracle.cpp for the reference file:line each one restates.
"""
from __future__ import annotations

import ctypes
import pathlib
import subprocess

import numpy as np

HERE = pathlib.Path(__file__).resolve().parent
LIB_PATH = HERE / "liboracle.so"
REF_PATH = HERE / "_ref" / "libuh_ref.so"

_P = ctypes.c_void_p
_I = ctypes.c_int
_F = ctypes.c_float

_SIGS = {
    "or_bf16_to_f32": (_F, [ctypes.c_uint16]),
    "or_f32_to_bf16": (ctypes.c_uint16, [_F]),
    "or_e4m3_to_f32": (_F, [ctypes.c_uint8]),
    "or_f32_to_e4m3": (ctypes.c_uint8, [_F]),
    "or_e8m0_to_f32": (_F, [ctypes.c_uint8]),
    "or_e2m1_to_f32": (_F, [ctypes.c_uint32]),
    "or_exp_f32_array": (None, [_P, _P, ctypes.c_size_t]),
    "or_pow2_ceil_e8m0": (ctypes.c_uint8, [_F]),
    "or_f32_to_bf16_array": (None, [_P, _P, ctypes.c_size_t]),
    "or_f32_to_e4m3_array": (None, [_P, _P, ctypes.c_size_t]),
    "or_act_quant_fp8": (None, [_P, _I, _P, _P, _I, _I, _I]),
    "or_fake_quant_fp8": (None, [_P, _I, _I, _I, _I]),
    "or_fake_quant_fp4": (None, [_P, _I, _I, _I, _I]),
    "or_act_quant_fp8_f32s": (None, [_P, _I, _P, _P, _I, _I, _I]),
    "or_repack": (None, [_P, _P, _P, _P, _I, _I]),
    "or_unrepack": (None, [_P, _P, _P, _P, _I, _I]),
    "or_mx_dequant": (None, [_P, _P, _P, _I, _I, _I]),
    "or_gemm_a8w4": (None, [_P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _I]),
    "or_gemm_a8w4_f64": (None, [_P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _I]),
    "or_gemm_w8a8": (None, [_P, _P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I]),
    "or_gemm_w8a8_f64": (None, [_P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I]),
    "or_gemm_grouped_fp8w": (None, [_P, _P, _P, _P, _P, _I, _I, _I, _I, _I]),
    "or_gemm_grouped_fp8w_f64": (None, [_P, _P, _P, _P, _I, _I, _I, _I, _I]),
    "or_rmsnorm_quant": (None, [_P, _I, _P, _P, _I, _P, _P, _I, _I, _F]),
    "or_swiglu": (None, [_P, _P, _P, _P, _I, _I, _F]),
    "or_route_ds": (None, [_P, _P, _P, _P, _P, _P, _I, _I, _I, _F, _P, _I]),
    "or_route_glm": (None, [_P, _P, _P, _P, _I, _I, _I, _F]),
    "or_route_softmax": (None, [_P, _P, _P, _I, _I, _I]),
    "or_dispatch": (_I, [_P, _P, _I, _I, _I, _P, _I, _P, _P, _P, _P, _P, _P, _P, _I, _P, _P]),
    "or_moe_combine": (None, [_P, _P, _P, _P, _I, _I, _I]),
    "or_remote_tokens": (_I, [_P, _P, _I, _I, _I, _I, _P, _P, _P, _P]),
    "or_remote_combine": (None, [_P, _P, _I, _I, _I, _P]),
    "or_hc_post": (None, [_P, _P, _P, _P, _P, _I, _I, _I]),
    "or_moe_combine_partial": (None, [_P, _P, _I, _P, _P, _P, _P, _I, _I, _I, _P, _P, _P, _I]),
    "or_moe_forward": (None, [_P, _P, _P, _I, _I, _I, _I, _I, _P, _P, _P, _P, _P, _P, _I, _F, _P, _P, _I, _P, _I, _P, _P]),
}

_lib = None
_ref = None


def build() -> None:
    """Compiles liboracle.so (and oracle/_ref when the reference tree is present)."""
    subprocess.run(["make", "-s", "-C", str(HERE), "all"], check=True)
    if pathlib.Path("/root/reference/src/core/half.hpp").exists():
        subprocess.run(["make", "-s", "-C", str(HERE), "ref"], check=True)


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            build()
        l = ctypes.CDLL(str(LIB_PATH))
        for name, (rt, at) in _SIGS.items():
            f = getattr(l, name)
            f.restype, f.argtypes = rt, at
        _lib = l
    return _lib


def ref_lib() -> ctypes.CDLL | None:
    """The reference's host code (half.hpp codecs, expert_pack repack), or None where it was not built."""
    global _ref
    if _ref is None and REF_PATH.exists():
        l = ctypes.CDLL(str(REF_PATH))
        for name in ("ref_bf16_to_float", "ref_e4m3_to_float", "ref_e8m0_to_float", "ref_e2m1_to_float"):
            getattr(l, name).restype = _F
        l.ref_bf16_to_float.argtypes = [ctypes.c_uint16]
        l.ref_e4m3_to_float.argtypes = [ctypes.c_uint8]
        l.ref_e8m0_to_float.argtypes = [ctypes.c_uint8]
        l.ref_e2m1_to_float.argtypes = [ctypes.c_uint8]
        l.ref_repack_matrix.argtypes = [_P, _P, _P, _P, _I, _I]
        l.ref_unrepack_matrix.argtypes = [_P, _P, _P, _P, _I, _I]
        l.ref_xxh64.restype, l.ref_xxh64.argtypes = ctypes.c_uint64, [_P, ctypes.c_size_t, ctypes.c_uint64]
        l.ref_read_header.restype, l.ref_read_header.argtypes = _I, [ctypes.c_char_p, _P]
        l.ref_header_size.restype, l.ref_header_size.argtypes = _I, []
        _ref = l
    return _ref


def _p(a):
    return None if a is None else a.ctypes.data


def _c(a, dtype):
    return np.ascontiguousarray(a, dtype=dtype)


# ---- codecs --------------------------------------------------------------------------------------------------------
def f32_to_bf16(x) -> np.ndarray:
    x = _c(x, np.float32)
    y = np.empty(x.shape, np.uint16)
    lib().or_f32_to_bf16_array(_p(x), _p(y), x.size)
    return y


def bf16_to_f32(b) -> np.ndarray:
    return (np.asarray(b, np.uint16).astype(np.uint32) << 16).view(np.float32)


def f32_to_e4m3(x) -> np.ndarray:
    x = _c(x, np.float32)
    y = np.empty(x.shape, np.uint8)
    lib().or_f32_to_e4m3_array(_p(x), _p(y), x.size)
    return y


def e4m3_to_f32(c) -> np.ndarray:
    c = np.asarray(c, np.uint8)
    return np.array([lib().or_e4m3_to_f32(int(v)) for v in c.ravel()], np.float32).reshape(c.shape)


# ---- quantization ----------------------------------------------------------------------------------------------
def exp_f32(x) -> np.ndarray:
    """e^x as the library computes it (uh_oracle.cpp exp_f32), elementwise over fp32 values."""
    x = _c(x, np.float32)
    y = np.empty_like(x)
    lib().or_exp_f32_array(_p(x), _p(y), x.size)
    return y


def act_quant_fp8(x_bf16, block=128):
    x = _c(x_bf16, np.uint16)
    rows, cols = x.shape
    q = np.empty((rows, cols), np.uint8)
    s = np.empty((rows, cols // block), np.uint8)
    lib().or_act_quant_fp8(_p(x), cols, _p(q), _p(s), rows, cols, block)
    return q, s


def fake_quant_fp4(x_bf16, block=32):
    """bf16 [rows, cols] -> bf16 [rows, cols]: e2m1 fake quantization per block (ref_elem.hip:43-59)."""
    x = np.array(x_bf16, dtype=np.uint16, copy=True, order="C")
    rows, cols = x.shape
    lib().or_fake_quant_fp4(_p(x), cols, rows, cols, block)
    return x


def fake_quant_fp8(x_bf16, block=128):
    x = _c(x_bf16, np.uint16).copy()
    rows, cols = x.shape
    lib().or_fake_quant_fp8(_p(x), cols, rows, cols, block)
    return x


def act_quant_fp8_f32s(x_bf16, block=128):
    x = _c(x_bf16, np.uint16)
    rows, cols = x.shape
    q = np.empty((rows, cols), np.uint8)
    s = np.empty((rows, cols // block), np.float32)
    lib().or_act_quant_fp8_f32s(_p(x), cols, _p(q), _p(s), rows, cols, block)
    return q, s


# ---- layout ---------------------------------------------------------------------------------------------------------
def repack(w, s, N, K):
    w = _c(w, np.uint8)
    s = _c(s, np.uint8)
    tw = np.empty(N * K // 2, np.uint8)
    ts = np.empty(N * K // 32, np.uint8)
    lib().or_repack(_p(w), _p(s), _p(tw), _p(ts), N, K)
    return tw, ts


def unrepack(tw, ts, N, K):
    tw = _c(tw, np.uint8)
    ts = _c(ts, np.uint8)
    w = np.empty((N, K // 2), np.uint8)
    s = np.empty((N, K // 32), np.uint8)
    lib().or_unrepack(_p(tw), _p(ts), _p(w), _p(s), N, K)
    return w, s


def mx_dequant(w, s, N, K, tiled=False):
    w = _c(w, np.uint8)
    s = _c(s, np.uint8)
    out = np.empty((N, K), np.float32)
    lib().or_mx_dequant(_p(w), _p(s), _p(out), N, K, int(tiled))
    return out


# ---- GEMMs ----------------------------------------------------------------------------------------------------------
def gemm_a8w4(a, sa, w, sw, N, tiled=False, threads=8):
    """(bf16 [M,N], fp32 [M,N]) in the reference's operation order."""
    a = _c(a, np.uint8)
    sa = _c(sa, np.uint8)
    w = _c(w, np.uint8)
    sw = _c(sw, np.uint8)
    M, K = a.shape
    c16 = np.empty((M, N), np.uint16)
    c32 = np.empty((M, N), np.float32)
    lib().or_gemm_a8w4(_p(a), _p(sa), _p(w), _p(sw), _p(c16), _p(c32), N, M, N, K, int(tiled), threads)
    return c16, c32


def gemm_a8w4_f64(a, sa, w, sw, N, tiled=False, threads=8):
    a = _c(a, np.uint8)
    sa = _c(sa, np.uint8)
    w = _c(w, np.uint8)
    sw = _c(sw, np.uint8)
    M, K = a.shape
    c = np.empty((M, N), np.float64)
    lib().or_gemm_a8w4_f64(_p(a), _p(sa), _p(w), _p(sw), _p(c), N, M, N, K, int(tiled), threads)
    return c


def gemm_w8a8(a, sa, w, sw, threads=8):
    """Scales e8m0 (uint8) or fp32 (float32), chosen by dtype. Returns (bf16, fp32)."""
    a = _c(a, np.uint8)
    w = _c(w, np.uint8)
    M, K = a.shape
    N = w.shape[0]
    f32 = np.asarray(sa).dtype == np.float32
    sa = _c(sa, np.float32 if f32 else np.uint8)
    sw = _c(sw, np.float32 if f32 else np.uint8)
    c16 = np.empty((M, N), np.uint16)
    c32 = np.empty((M, N), np.float32)
    if f32:
        lib().or_gemm_w8a8(_p(a), None, _p(sa), _p(w), None, _p(sw), _p(c16), _p(c32), N, M, N, K, threads)
    else:
        lib().or_gemm_w8a8(_p(a), _p(sa), None, _p(w), _p(sw), None, _p(c16), _p(c32), N, M, N, K, threads)
    return c16, c32


def gemm_w8a8_f64(a, sa, w, sw, threads=8):
    a = _c(a, np.uint8)
    w = _c(w, np.uint8)
    M, K = a.shape
    N = w.shape[0]
    f32 = np.asarray(sa).dtype == np.float32
    sa = _c(sa, np.float32 if f32 else np.uint8)
    sw = _c(sw, np.float32 if f32 else np.uint8)
    c = np.empty((M, N), np.float64)
    if f32:
        lib().or_gemm_w8a8_f64(_p(a), None, _p(sa), _p(w), None, _p(sw), _p(c), N, M, N, K, threads)
    else:
        lib().or_gemm_w8a8_f64(_p(a), _p(sa), None, _p(w), _p(sw), None, _p(c), N, M, N, K, threads)
    return c


def gemm_grouped_fp8w(a, w, sw, G, R, threads=8):
    """a bf16 (uint16) [M, G, K]; w e4m3 [G R, K]; sw e8m0 [ceil(G R / 128), K / 128]. Returns (bf16, fp32) [M, G, R]."""
    a = _c(a, np.uint16)
    w = _c(w, np.uint8)
    sw = _c(sw, np.uint8)
    M, K = a.shape[0], w.shape[1]
    assert a.shape == (M, G, K) and w.shape[0] == G * R
    c16 = np.empty((M, G, R), np.uint16)
    c32 = np.empty((M, G, R), np.float32)
    lib().or_gemm_grouped_fp8w(_p(a), _p(w), _p(sw), _p(c16), _p(c32), M, G, R, K, threads)
    return c16, c32


def gemm_grouped_fp8w_f64(a, w, sw, G, R, threads=8):
    a = _c(a, np.uint16)
    w = _c(w, np.uint8)
    sw = _c(sw, np.uint8)
    M, K = a.shape[0], w.shape[1]
    c = np.empty((M, G, R), np.float64)
    lib().or_gemm_grouped_fp8w_f64(_p(a), _p(w), _p(sw), _p(c), M, G, R, K, threads)
    return c


def rmsnorm_quant(x, w, eps, quant=True):
    """rmsnorm of bf16 rows x [rows, dim] with bf16 weights w [dim] in the reference's order; with quant also
    act_quant_fp8 (block 128) of the output. Returns y (bf16) or (y, q, qs)."""
    x = _c(x, np.uint16)
    w = _c(w, np.uint16)
    rows, dim = x.shape
    y = np.empty((rows, dim), np.uint16)
    if not quant:
        lib().or_rmsnorm_quant(_p(x), dim, _p(w), _p(y), dim, None, None, rows, dim, eps)
        return y
    q = np.empty((rows, dim), np.uint8)
    qs = np.empty((rows, dim // 128), np.uint8)
    lib().or_rmsnorm_quant(_p(x), dim, _p(w), _p(y), dim, _p(q), _p(qs), rows, dim, eps)
    return y, q, qs


# ---- MoE pieces -------------------------------------------------------------------------------------------------------
def swiglu(g, u, w, limit):
    g = _c(g, np.uint16)
    u = _c(u, np.uint16)
    rows, dim = g.shape
    h = np.empty_like(g)
    wv = None if w is None else _c(w, np.float32)
    lib().or_swiglu(_p(g), _p(u), _p(wv), _p(h), rows, dim, limit)
    return h


def route_ds(logits, bias, K, route_scale=1.0, tid2eid=None, ids=None, bias_vl=None, vocab=0):
    logits = _c(logits, np.float32)
    T, E = logits.shape
    bias = _c(bias, np.float32)
    sel = np.empty((T, K), np.int32)
    wt = np.empty((T, K), np.float32)
    t2e = None if tid2eid is None else _c(tid2eid, np.int32)
    idv = None if ids is None else _c(ids, np.int32)
    bvl = None if bias_vl is None else _c(bias_vl, np.float32)
    lib().or_route_ds(_p(logits), _p(bias), _p(t2e), _p(idv), _p(sel), _p(wt), T, E, K, route_scale, _p(bvl), vocab)
    return sel, wt


def route_glm(logits, bias, K, route_scale=1.0):
    logits = _c(logits, np.float32)
    T, E = logits.shape
    bias = _c(bias, np.float32)
    sel = np.empty((T, K), np.int32)
    wt = np.empty((T, K), np.float32)
    lib().or_route_glm(_p(logits), _p(bias), _p(sel), _p(wt), T, E, K, route_scale)
    return sel, wt


def route_softmax(logits, K):
    logits = _c(logits, np.float32)
    T, E = logits.shape
    sel = np.empty((T, K), np.int32)
    wt = np.empty((T, K), np.float32)
    lib().or_route_softmax(_p(logits), _p(sel), _p(wt), T, E, K)
    return sel, wt


def dispatch(sel, wt, E, tile_rows=128, resident=None, max_tiles=None):
    """Host-order dispatch: dict of count, off, eidx, ewt, row_expert, pidx, tiles [n,3], plan [5]."""
    sel = _c(sel, np.int32)
    wt = _c(wt, np.float32)
    T, K = sel.shape
    P = T * K
    if max_tiles is None:
        max_tiles = P + E
    out = dict(
        count=np.empty(E, np.int32), off=np.empty(E, np.int32), eidx=np.empty(P, np.int32),
        ewt=np.empty(P, np.float32), row_expert=np.empty(P, np.int32), pidx=np.empty((T, K), np.int32),
        tiles=np.zeros((max_tiles, 3), np.int32), remote_tiles=np.zeros((max_tiles, 3), np.int32),
        plan=np.empty(5, np.int32))
    res = None if resident is None else _c(resident, np.uint8)
    n = lib().or_dispatch(_p(sel), _p(wt), T, K, E, _p(res), tile_rows, _p(out["count"]), _p(out["off"]),
                          _p(out["eidx"]), _p(out["ewt"]), _p(out["row_expert"]), _p(out["pidx"]), _p(out["tiles"]),
                          max_tiles, _p(out["remote_tiles"]), _p(out["plan"]))
    out["tiles"] = out["tiles"][: min(n, max_tiles)]
    out["remote_tiles"] = out["remote_tiles"][: out["plan"][3]]
    return out


def moe_combine(pair_out, pidx, shared=None):
    pair_out = _c(pair_out, np.uint16)
    pidx = _c(pidx, np.int32)
    T, K = pidx.shape
    dim = pair_out.shape[1]
    out = np.empty((T, dim), np.uint16)
    sh = None if shared is None else _c(shared, np.uint16)
    lib().or_moe_combine(_p(pair_out), _p(pidx), _p(sh), _p(out), T, K, dim)
    return out


def remote_tokens(pidx, eidx, remote0):
    """Compact remote tokens (moe_dispatch.hip:149-203): dict of U, tok2u [T], u2t [U], p2u [P] (rows < remote0
    left -1), u2p [U, K]."""
    pidx = _c(pidx, np.int32)
    eidx = _c(eidx, np.int32)
    T, K = pidx.shape
    P = eidx.size
    tok2u = np.empty(T, np.int32)
    u2t = np.empty(max(T, 1), np.int32)
    p2u = np.full(max(P, 1), -1, np.int32)
    u2p = np.empty((max(T, 1), K), np.int32)
    U = lib().or_remote_tokens(_p(pidx), _p(eidx), T, K, int(remote0), P, _p(tok2u), _p(u2t), _p(p2u), _p(u2p))
    return dict(U=U, tok2u=tok2u, u2t=u2t[:U], p2u=p2u[:P], u2p=u2p[:U])


def remote_combine(pair_out, u2p):
    pair_out = _c(pair_out, np.uint16)
    u2p = _c(u2p, np.int32)
    U, K = u2p.shape
    dim = pair_out.shape[1]
    dst = np.empty((U, dim), np.uint16)
    lib().or_remote_combine(_p(pair_out), _p(u2p), U, K, dim, _p(dst))
    return dst


def moe_combine_partial(pair_out, pidx, remote0, tok2u, remote, shared=None, hc_x=None, post=None, comb=None):
    """moe_combine_partial(_link) (moe_dispatch.hip:243-278): returns out, and the post-mixed streams when hc_x
    [T, hc, dim] is given (a copy; the input is not changed)."""
    pair_out = _c(pair_out, np.uint16)
    pidx = _c(pidx, np.int32)
    T, K = pidx.shape
    dim = pair_out.shape[1]
    out = np.empty((T, dim), np.uint16)
    rem = _c(remote, np.uint16) if remote is not None and remote.size else np.zeros((1, dim), np.uint16)
    sh = None if shared is None else _c(shared, np.uint16)
    hx = None if hc_x is None else np.array(hc_x, np.uint16, copy=True, order="C")
    po = None if post is None else _c(post, np.float32)
    co = None if comb is None else _c(comb, np.float32)
    hc = 0 if hx is None else hx.shape[1]
    lib().or_moe_combine_partial(_p(pair_out), _p(pidx), int(remote0), _p(_c(tok2u, np.int32)), _p(rem), _p(sh),
                                 _p(out), T, K, dim, _p(hx), _p(po), _p(co), hc)
    return out if hx is None else (out, hx)


def hc_post(x, res, post, comb):
    """The mHC post-mix (ref_elem.hip hc_post): x [T, dim], res [T, hc, dim] -> out [T, hc, dim]."""
    x, res = _c(x, np.uint16), _c(res, np.uint16)
    T, hc, dim = res.shape
    out = np.empty_like(res)
    lib().or_hc_post(_p(x), _p(res), _p(_c(post, np.float32)), _p(_c(comb, np.float32)), _p(out), T, hc, dim)
    return out


def moe_forward(x, sel, wt, experts, D, I, limit, tiled=True, threads=8, subset=None, with_h=False):
    """experts: list of E dicts with w1, s1, w3, s3, w2, s2 (uint8 arrays, tile-major when tiled) or None.
    Returns (out bf16 [T, D] or None when subset is given, pair_out bf16 [T*K, D]), and with with_h also the codes
    [T*K, I] and e8m0 scales [T*K, I/128] of h (act_quant of the SwiGLU output) per pair row."""
    x = _c(x, np.uint16)
    sel = _c(sel, np.int32)
    wt = _c(wt, np.float32)
    T, K = sel.shape
    E = len(experts)
    keep = []
    tabs = {k: (ctypes.c_void_p * E)() for k in ("w1", "s1", "w3", "s3", "w2", "s2")}
    for e, ex in enumerate(experts):
        for k in tabs:
            if ex is None:
                tabs[k][e] = None
            else:
                arr = _c(ex[k], np.uint8)
                keep.append(arr)
                tabs[k][e] = arr.ctypes.data
    pair_out = np.zeros((T * K, D), np.uint16)
    out = None if subset is not None else np.empty((T, D), np.uint16)
    sub = None if subset is None else _c(subset, np.int32)
    hq = np.zeros((T * K, I), np.uint8) if with_h else None
    hs = np.zeros((T * K, I // 128), np.uint8) if with_h else None
    lib().or_moe_forward(_p(x), _p(sel), _p(wt), T, K, E, D, I,
                         ctypes.cast(tabs["w1"], _P), ctypes.cast(tabs["s1"], _P), ctypes.cast(tabs["w3"], _P),
                         ctypes.cast(tabs["s3"], _P), ctypes.cast(tabs["w2"], _P), ctypes.cast(tabs["s2"], _P),
                         int(tiled), limit, _p(pair_out), _p(out), threads, _p(sub), 0 if sub is None else len(sub),
                         _p(hq), _p(hs))
    return (out, pair_out, hq, hs) if with_h else (out, pair_out)
