"""uh_mx_moe_forward_noalloc (the routed-expert FFN with its workspace in a fixed per-device array, for callers that
cannot allocate) against uh_mx_moe_forward with a caller-allocated workspace: bit-identical outputs and routing on
two calls in a row at the headline shape (D = 4096, I = 2048, E = 256, top-6), the second smaller (T = 64, then
T = 8, so stale scratch contents from the first call must not leak into the second), and a clear error for a shape
whose workspace exceeds the array."""
import numpy as np
import pytest

from tests.helpers import randn_bf16
from unholy_amd import call
from unholy_amd._lib import UhError
from unholy_amd.device import DeviceBuffer, fill_random_bytes, pointer_table, synchronize

pytestmark = pytest.mark.gpu

D, I, E, K = 4096, 2048, 256, 6
LIMIT = 10.0


def _weights(seed):
    shapes = [(I, D), (I, D), (D, I)]
    mat = [n * k // 2 + n * k // 32 for n, k in shapes]
    buf = DeviceBuffer(E * sum(mat))
    fill_random_bytes(buf, E * sum(mat), seed, 0, 255)
    tab = [[0] * E for _ in range(6)]
    for e in range(E):
        off = e * sum(mat)
        for m, (n, k) in enumerate(shapes):
            tab[2 * m][e] = buf.ptr + off
            tab[2 * m + 1][e] = buf.ptr + off + n * k // 2
            fill_random_bytes(tab[2 * m + 1][e], n * k // 32, seed + 1 + 3 * e + m, 119, 125)
            off += mat[m]
    return buf, pointer_table([p for row in tab for p in row])


def test_noalloc_forward_matches_allocating_forward():
    buf, table = _weights(99)
    rng = np.random.default_rng(8)
    assert call("uh_mx_moe_noalloc_max_bytes") >= call("uh_mx_moe_workspace_size", 64, K, E, D, I)
    for T in (64, 8):
        x = DeviceBuffer.from_array(randn_bf16(rng, (T, D)))
        lg = DeviceBuffer.from_array(rng.standard_normal((T, E), dtype=np.float32))
        ws_bytes = call("uh_mx_moe_workspace_size", T, K, E, D, I)
        ws = DeviceBuffer(ws_bytes)
        outs, sels, wts = [], [], []
        for noalloc in (False, True):
            out, sel, wt = DeviceBuffer(T * D * 2), DeviceBuffer(T * K * 4), DeviceBuffer(T * K * 4)
            if noalloc:
                call("uh_mx_moe_forward_noalloc", x, lg, T, K, E, D, I, table, LIMIT, out, sel, wt, None)
            else:
                call("uh_mx_moe_forward", x, lg, T, K, E, D, I, table, LIMIT, ws, ws_bytes, out, sel, wt, None)
            synchronize()
            outs.append(out.download((T, D), np.uint16))
            sels.append(sel.download((T, K), np.int32))
            wts.append(wt.download((T, K), np.float32))
        print(f"noalloc T={T}: bit-identical {np.mean(outs[0] == outs[1]):.6f}")
        assert np.array_equal(sels[0], sels[1]) and np.array_equal(wts[0], wts[1])
        assert np.array_equal(outs[0], outs[1])
    buf.free()


def test_noalloc_rejects_oversized_workspace():
    T = 4096
    assert call("uh_mx_moe_workspace_size", T, K, E, D, I) > call("uh_mx_moe_noalloc_max_bytes")
    with pytest.raises(UhError, match="above the fixed scratch"):
        call("uh_mx_moe_forward_noalloc", None, None, T, K, E, D, I, None, LIMIT, None, None, None, None)
