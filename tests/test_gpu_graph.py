"""HIP-graph replay of library launches: every replay (with eager work between replays) equals the eager result."""
import numpy as np
import pytest

import oracle
from tests.helpers import randn_bf16
from tests.test_gpu_moe import _moe_case
from unholy_amd import call
from unholy_amd.device import DeviceBuffer, Graph, Stream, synchronize

pytestmark = pytest.mark.gpu


def dev(a):
    return DeviceBuffer.from_array(np.ascontiguousarray(a))


# M = 4: the GEMV; 64 and 200: the row-tile kernel (asm-issued loads, counted waits).
@pytest.mark.parametrize("M", [4, 64, 200])
def test_graph_replays_fp8_dense_step(M):
    rng = np.random.default_rng(3 + M)
    N, K = 1024, 4096
    x = dev(randn_bf16(rng, (M, K)))
    wq = rng.integers(0, 256, (N, K), dtype=np.uint8)
    wq[(wq & 0x7F) == 0x7F] = 0
    w, sw = dev(wq), dev(rng.random(((N + 127) // 128, K // 128), dtype=np.float32) * np.float32(0.01))
    q, sa, c = DeviceBuffer(M * K), DeviceBuffer(M * (K // 128) * 4), DeviceBuffer(M * N * 2)
    st = Stream()

    def step():
        call("uh_act_quant_fp8_f32s", x, K, q, sa, M, K, 128, st.handle)
        call("uh_gemm_fp8_f32s", q, sa, w, sw, c, N, M, N, K, st.handle)

    step()
    st.synchronize()
    eager = c.download((M, N), np.uint16)
    g = Graph(st, step)
    for rep in range(3):
        c.zero()
        synchronize()
        g.launch()
        st.synchronize()
        assert np.array_equal(c.download((M, N), np.uint16), eager), rep
        step()  # eager work between replays
        st.synchronize()


@pytest.mark.parametrize("M", [1, 64])
def test_graph_replays_grouped_fp8w(M):
    """The grouped fp8-weight GEMM (M = 1: the GEMV; 64: the row-tile kernel) replayed: every replay equals eager."""
    rng = np.random.default_rng(11 + M)
    G, R, K = 4, 512, 4096
    a = dev(randn_bf16(rng, (M, G, K)))
    wq = rng.integers(0, 256, (G * R, K), dtype=np.uint8)
    wq[(wq & 0x7F) == 0x7F] = 0
    w, sw = dev(wq), dev(rng.integers(118, 126, (G * R // 128, K // 128), dtype=np.uint8))
    c = DeviceBuffer(M * G * R * 2)
    st = Stream()

    def step():
        call("uh_gemm_grouped_fp8w_wmma", a, w, sw, c, M, G, R, K, st.handle)

    step()
    st.synchronize()
    eager = c.download((M, G * R), np.uint16)
    g = Graph(st, step)
    for rep in range(3):
        c.zero()
        synchronize()
        g.launch()
        st.synchronize()
        assert np.array_equal(c.download((M, G * R), np.uint16), eager), rep
        step()
        st.synchronize()


@pytest.mark.parametrize("T", [8, 48, 80])
def test_graph_replays_decode_forward(T):
    """T = 8: single-block dispatch + GEMVs; 48: multi-kernel dispatch (its counters cleared by a kernel) + GEMVs;
    80: the prefill GEMM path."""
    rng = np.random.default_rng(9 + T)
    E, K, D, I, limit = 32, 6, 1024, 512, 10.0
    experts, bufs, tab, x, logits = _moe_case(rng, T, E, K, D, I)
    ws_bytes = call("uh_mx_moe_workspace_size", T, K, E, D, I)
    ws, out = DeviceBuffer(ws_bytes), DeviceBuffer(T * D * 2)
    dx, dl = dev(x), dev(logits)
    st = Stream()

    def step():
        call("uh_mx_moe_forward", dx, dl, T, K, E, D, I, tab.ptr, limit, ws.ptr, ws_bytes, out.ptr, None, None,
             st.handle)

    step()
    st.synchronize()
    eager = out.download((T, D), np.uint16)
    g = Graph(st, step)
    for rep in range(3):
        out.zero()
        synchronize()
        g.launch()
        st.synchronize()
        assert np.array_equal(out.download((T, D), np.uint16), eager), rep
        step()
        st.synchronize()
