"""GPU parity of the grouped fp8-weight GEMM ("mgk,grk->mgr", the reference's wo_a projection): the reference-order
entry bit-exact against the CPU oracle, the fast entries (GEMV, tiled MFMA GEMM, reference-order fallback for
untileable shapes) within the bf16 bar, and the GEMV's fused output quantization bit-exact."""
import numpy as np
import pytest

import oracle
from tests.helpers import from_bf16, max_rel, randn_bf16
from unholy_amd import call
from unholy_amd.device import DeviceBuffer

pytestmark = pytest.mark.gpu


def dev(a):
    return DeviceBuffer.from_array(np.ascontiguousarray(a))


def _case(rng, M, G, R, K):
    a = randn_bf16(rng, (M, G, K))
    w = rng.integers(0, 256, (G * R, K), dtype=np.uint8)
    w[(w & 0x7F) == 0x7F] = 0  # no NaN codes
    sw = rng.integers(118, 126, ((G * R + 127) // 128, K // 128), dtype=np.uint8)
    return a, w, sw


@pytest.mark.parametrize("M,G,R,K", [(3, 2, 256, 256), (1, 8, 1024, 512), (5, 3, 200, 384), (40, 2, 128, 128)])
def test_grouped_fp8w_reference_order_bit_exact(M, G, R, K):
    rng = np.random.default_rng(M * 31 + R)
    a, w, sw = _case(rng, M, G, R, K)
    ref16, _ = oracle.gemm_grouped_fp8w(a, w, sw, G, R)
    c = DeviceBuffer(M * G * R * 2)
    call("uh_gemm_grouped_fp8w", dev(a), dev(w), dev(sw), c, M, G, R, K, None)
    got = c.download((M, G, R), np.uint16)
    print(f"grouped fp8w ref order M={M} G={G} R={R} K={K}: bit-identical fraction {np.mean(got == ref16):.6f}")
    assert np.array_equal(got, ref16)


# M <= 16: the row-tile kernel's 32-column form (R % 32 == 0, K <= 8192: one to four 2,048-input chunks, ragged K);
# 16 < M <= 384: its 64-column form (R % 64 == 0, K <= 4096: one to four 1,024-input chunks, a ragged last chunk at
# K = 640 and 1,152, 1 to 12 row tiles, the DSV4 shape); other shapes up to M = 160 the GEMV in 32-row chunks (R = 200
# is the reference-order kernel; K = 9,216 the GEMV); larger M: the tiled GEMM (128-column tiles, M = 385, 400, 520;
# 256-column ones for R % 256 == 0 once they make more than 256 workgroups: M = 400, G R = 16,896).
@pytest.mark.parametrize("M,G,R,K", [(1, 8, 1024, 4096), (16, 2, 512, 1024), (32, 3, 256, 640), (7, 2, 200, 256),
                                     (33, 2, 256, 512), (100, 2, 256, 512), (200, 3, 128, 384), (300, 2, 384, 1024),
                                     (257, 2, 256, 512), (200, 3, 512, 384), (65, 2, 200, 256), (64, 8, 1024, 4096),
                                     (17, 2, 128, 768), (160, 2, 192, 3072), (48, 3, 64, 1152), (95, 1, 64, 9216),
                                     (4, 3, 96, 640), (16, 1, 32, 8192), (9, 2, 160, 5120), (1, 2, 64, 128),
                                     (384, 1, 64, 256), (385, 1, 128, 384), (400, 2, 256, 512), (520, 2, 384, 1024),
                                     (400, 1, 16896, 128)])
def test_grouped_fp8w_fast_path(M, G, R, K):
    rng = np.random.default_rng(M * 7 + G * R + K)
    a, w, sw = _case(rng, M, G, R, K)
    ref16, _ = oracle.gemm_grouped_fp8w(a, w, sw, G, R)
    ref64 = oracle.gemm_grouped_fp8w_f64(a, w, sw, G, R)
    c = DeviceBuffer(M * G * R * 2)
    call("uh_gemm_grouped_fp8w_wmma", dev(a), dev(w), dev(sw), c, M, G, R, K, None)
    got = from_bf16(c.download((M, G, R), np.uint16))
    mr = max_rel(got, from_bf16(ref16))
    print(f"grouped fp8w fast M={M} G={G} R={R} K={K}: max_rel {mr:.3e} vs f64 {max_rel(got, ref64):.3e} "
          f"bit-identical {np.mean(got == from_bf16(ref16)):.4f}")
    assert mr <= 1e-2
    assert max_rel(got, ref64) <= 1e-2


@pytest.mark.parametrize("M", [1, 8, 32])
def test_gemv_grouped_fp8w_fused_quant(M):
    """The GEMV entry with GemvQuant: its bf16 outputs as the fast path's, and q / qs exactly act_quant_fp8 (block 128)
    of those outputs; the counters are left zero."""
    G, R, K = 4, 256, 512
    rng = np.random.default_rng(M)
    a, w, sw = _case(rng, M, G, R, K)
    da, dw, dsw = dev(a), dev(w), dev(sw)
    c = DeviceBuffer(M * G * R * 2)
    q, qs = DeviceBuffer(M * G * R), DeviceBuffer(M * G * R // 128)
    counters = dev(np.zeros(G * R // 128, np.uint32))
    call("uh_gemv_grouped_fp8w", da, dw, dsw, c, M, G, R, K, q, qs, counters, None)
    c_fast = DeviceBuffer(M * G * R * 2)
    call("uh_gemm_grouped_fp8w_wmma", da, dw, dsw, c_fast, M, G, R, K, None)
    out = c.download((M, G * R), np.uint16)
    assert np.array_equal(out, c_fast.download((M, G * R), np.uint16))
    q_ref, qs_ref = oracle.act_quant_fp8(out)
    assert np.array_equal(q.download((M, G * R), np.uint8), q_ref)
    assert np.array_equal(qs.download((M, G * R // 128), np.uint8), qs_ref)
    assert not counters.download((G * R // 128,), np.uint32).any()


def test_grouped_fp8w_shape_errors():
    a, w, sw = _case(np.random.default_rng(0), 2, 2, 128, 256)
    da, dw, dsw = dev(a), dev(w), dev(sw)
    c = DeviceBuffer(2 * 2 * 128 * 2)
    with pytest.raises(Exception, match="K % 128"):
        call("uh_gemm_grouped_fp8w_wmma", da, dw, dsw, c, 2, 2, 128, 200, None)
    with pytest.raises(Exception, match="M > 32"):
        call("uh_gemv_grouped_fp8w", da, dw, dsw, c, 33, 2, 128, 256, None, None, None, None)
    call("uh_gemm_grouped_fp8w_wmma", da, dw, dsw, c, 0, 2, 128, 256, None)  # M = 0: nothing to do

