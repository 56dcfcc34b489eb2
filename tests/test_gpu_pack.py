"""The expert pack on the GPU: slots loaded into device memory are the file's bytes; the whole routed-expert forward
on the pack's expert table equals the forward on the same experts repacked on the device (uh_mx_repack_to), bit
for bit; checksum verification refuses a damaged or an absent slot."""
import ctypes

import numpy as np
import pytest

from tests.helpers import randn_bf16
from tests.test_pack import G2, G13, K2, K13, _experts, parse_header, write_pack
from unholy_amd import call
from unholy_amd._lib import UhError
from unholy_amd.device import DeviceBuffer, pointer_table, synchronize

pytestmark = pytest.mark.gpu

D, I = K13, G13  # w1 / w3 [I, D] = [256, 512], w2 [D, I] = [512, 256]


def _load(path, first, count, verify=1, direct=0, pad=0):
    hb = (ctypes.c_uint8 * 264)()
    call("uh_pack_read_header", str(path).encode(), hb)
    h = parse_header(hb)
    stride = h["slot_bytes"] + pad
    buf = DeviceBuffer(count * stride)
    call("uh_pack_load", str(path).encode(), first, count, buf.ptr, stride, verify, direct, None)
    return hb, h, buf, stride


def _forward(tab, x, logits, T, K, E):
    ws_bytes = call("uh_mx_moe_workspace_size", T, K, E, D, I)
    ws, out = DeviceBuffer(ws_bytes), DeviceBuffer(T * D * 2)
    dx, dl = DeviceBuffer.from_array(x), DeviceBuffer.from_array(logits)
    call("uh_mx_moe_forward", dx.ptr, dl.ptr, T, K, E, D, I, tab.ptr, 10.0, ws.ptr, ws_bytes, out.ptr, None, None,
         None)
    synchronize()
    return out.download((T, D), np.uint16)


@pytest.mark.parametrize("T,K", [(4, 2), (40, 4)])
def test_pack_load_and_forward(tmp_path, T, K):
    rng = np.random.default_rng(21 + T)
    E = 8
    experts = _experts(rng, E)
    path = tmp_path / "e.pack"
    write_pack(path, 1, 0, E, experts)
    hb, h, buf, stride = _load(path, 0, E)
    raw = path.read_bytes()
    assert buf.download((E * stride,), np.uint8).tobytes() == raw[h["slots_offset"]:h["slots_offset"] + E * stride]
    tab_host = (ctypes.c_uint64 * (6 * E))()
    call("uh_pack_expert_table", hb, buf.ptr, stride, E, tab_host)
    tab_pack = DeviceBuffer.from_array(np.array(tab_host, np.uint64))
    keep, flat = [], [None] * (6 * E)  # keep: every device buffer alive until the kernels have run
    for e in range(E):
        for m, (rows, cols) in enumerate(((G13, K13), (G13, K13), (G2, K2))):
            w, s = DeviceBuffer.from_array(experts[e][2 * m]), DeviceBuffer.from_array(experts[e][2 * m + 1])
            tw, ts = DeviceBuffer(rows * cols // 2), DeviceBuffer(rows * cols // 32)
            call("uh_mx_repack_to", w.ptr, s.ptr, tw.ptr, ts.ptr, rows, cols, None)
            keep += [w, s, tw, ts]
            flat[(2 * m) * E + e], flat[(2 * m + 1) * E + e] = tw, ts
    tab_dev = pointer_table(flat)
    x = randn_bf16(rng, (T, D))
    logits = rng.standard_normal((T, E), dtype=np.float32)
    a = _forward(tab_pack, x, logits, T, K, E)
    b = _forward(tab_dev, x, logits, T, K, E)
    print(f"pack forward T={T}: bit-identical {np.mean(a == b):.6f}")
    assert np.array_equal(a, b)


def test_pack_verify_refuses_damage_and_absence(tmp_path):
    rng = np.random.default_rng(4)
    experts = _experts(rng, 4)
    path = tmp_path / "d.pack"
    write_pack(path, 1, 0, 4, experts, absent={2})
    _load(path, 0, 2)  # slots 0 and 1 verify
    with pytest.raises(UhError, match="absent"):
        _load(path, 0, 4)
    raw = bytearray(path.read_bytes())
    h = parse_header(raw)
    raw[h["slots_offset"] + 3 * h["slot_bytes"] + 100] ^= 0x40
    path.write_bytes(bytes(raw))
    with pytest.raises(UhError, match="checksum"):
        _load(path, 3, 1)
    with pytest.raises(UhError, match="absent"):  # unverified loads refuse an absent slot too
        _load(path, 1, 2, verify=0)
    _, _, buf, _ = _load(path, 3, 1, verify=0)  # unverified: the damaged bytes as they are
    got = buf.download((h["slot_bytes"],), np.uint8).tobytes()
    assert got == bytes(raw[h["slots_offset"] + 3 * h["slot_bytes"]:h["slots_offset"] + 4 * h["slot_bytes"]])


def test_pack_load_o_direct(tmp_path):
    """O_DIRECT reads (4 KiB-aligned slots read into an aligned bounce buffer, then copied into the pinned staging:
    pread into pinned memory fails with EFAULT under O_DIRECT), in a directory of the repository's tree when its file
    system takes O_DIRECT (the temporary directory is often tmpfs, which does not), else tmp_path."""
    import pathlib
    import shutil
    import tempfile
    rng = np.random.default_rng(8)
    experts = _experts(rng, 3)
    dirs = [pathlib.Path(tempfile.mkdtemp(prefix="odirect_", dir=pathlib.Path(__file__).resolve().parent)), tmp_path]
    try:
        for dr in dirs:
            path = dr / "o.pack"
            write_pack(path, 1, 0, 3, experts)
            try:
                _, h, buf, stride = _load(path, 0, 3, direct=1)
            except UhError as err:  # a file system without O_DIRECT
                print(f"O_DIRECT refused in {dr}: {err}")
                continue
            raw = path.read_bytes()
            got = buf.download((3 * stride,), np.uint8).tobytes()
            assert got == raw[h["slots_offset"]:h["slots_offset"] + 3 * stride]
            print(f"O_DIRECT load verified in {dr}")
            return
        pytest.skip("O_DIRECT not available on these file systems")
    finally:
        shutil.rmtree(dirs[0], ignore_errors=True)


def _odirect_dir():
    """A directory of the repository's tree (its file system may take O_DIRECT; the temporary directory is often
    tmpfs, which does not)."""
    import pathlib
    import tempfile
    return pathlib.Path(tempfile.mkdtemp(prefix="odirect_", dir=pathlib.Path(__file__).resolve().parent))


@pytest.mark.parametrize("count", [2, 3, 5, 7])
@pytest.mark.parametrize("direct", [0, 1])
def test_pack_load_unverified_chunks(tmp_path, count, direct):
    """Unverified loads of fewer slots than reader threads read each slot as several 4 KiB-aligned chunks: every slot's
    bytes in device memory equal the file's, with a destination stride larger than the slot (slot_bytes + 4096) and
    with O_DIRECT (where the file system takes it)."""
    import shutil
    rng = np.random.default_rng(50 + count)
    n = 8
    experts = _experts(rng, n)
    dr = _odirect_dir() if direct else tmp_path
    try:
        path = dr / "c.pack"
        write_pack(path, 1, 0, n, experts)
        first = n - count
        try:
            _, h, buf, stride = _load(path, first, count, verify=0, direct=direct, pad=4096)
        except UhError as err:
            if direct:
                pytest.skip(f"O_DIRECT not available here: {err}")
            raise
        raw = path.read_bytes()
        sb = h["slot_bytes"]
        got = buf.download((count * stride,), np.uint8).tobytes()
        for i in range(count):
            want = raw[h["slots_offset"] + (first + i) * sb:h["slots_offset"] + (first + i + 1) * sb]
            assert got[i * stride:i * stride + sb] == want, (count, direct, i)
    finally:
        if direct:
            shutil.rmtree(dr, ignore_errors=True)
