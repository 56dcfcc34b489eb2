"""The expert pack's host side (no GPU): XXH64 against its published value and the reference's own implementation,
and a pack written by this library read back by the reference's own read_header, its slots the reference's
repack_matrix of the inputs and its checksum table the reference's xxh64 of them."""
import ctypes
import os
import struct

import numpy as np
import pytest

import oracle
from unholy_amd import call
from unholy_amd._lib import lib as uh_lib

HEADER_FMT = "<QII4I4Q6Q6Q4IQQ8QQ"  # the reference's Header (expert_pack.hpp:29-45), 264 bytes
FIELDS = ("magic version header_bytes n_layers n_mtp n_experts reserved0 n_slots slot_bytes slots_offset "
          "checksum_offset").split()


def parse_header(b):
    v = struct.unpack(HEADER_FMT, bytes(b[:264]))
    h = dict(zip(FIELDS, v[:11]))
    h["part_offset"], h["part_bytes"] = list(v[11:17]), list(v[17:23])
    h["w13_out"], h["w13_in"], h["w2_out"], h["w2_in"] = v[23:27]
    h["config_hash"], h["source_hash"], h["header_hash"] = v[27], v[28], v[37]
    return h


def xxh(data, seed=0):
    a = np.frombuffer(bytes(data), np.uint8)
    return uh_lib().uh_pack_xxh64(a.ctypes.data if a.size else None, a.size, seed)


def ref():
    r = oracle.ref_lib()
    if r is None:
        pytest.skip("oracle/_ref (the reference's host code) is not built here")
    return r


def test_xxh64_published_value_and_reference():
    assert struct.calcsize(HEADER_FMT) == 264
    assert xxh(b"") == 0xEF46DB3751D8E999  # XXH64 of the empty input, seed 0, as published with xxHash
    r = ref()
    rng = np.random.default_rng(3)
    for n in list(range(0, 80)) + [127, 128, 129, 1000, 4096, 1 << 20]:
        a = rng.integers(0, 256, n, dtype=np.uint8)
        for seed in (0, 1, 0xFFFFFFFFFFFFFFFF):
            got = uh_lib().uh_pack_xxh64(a.ctypes.data if n else None, n, seed)
            assert got == r.ref_xxh64(a.ctypes.data if n else None, n, seed), (n, seed)


# w1 / w3 [256, 512], w2 [512, 256]: a slot of 51 x 4096 bytes.
G13, K13, G2, K2 = 256, 512, 512, 256


def _experts(rng, n):
    ex = []
    for _ in range(n):
        parts = []
        for rows, cols in ((G13, K13), (G13, K13), (G2, K2)):
            parts.append(rng.integers(0, 256, rows * cols // 2, dtype=np.uint8))
            parts.append(rng.integers(118, 127, rows * cols // 32, dtype=np.uint8))
        ex.append(parts)
    return ex


def write_pack(path, n_layers, n_mtp, n_experts, experts, absent=(), cfg=0x1234, src=0x5678):
    n = (n_layers + n_mtp) * n_experts
    ptrs = (ctypes.c_void_p * (6 * n))()
    for i in range(n):
        for j in range(6):
            ptrs[6 * i + j] = None if i in absent else experts[i][j].ctypes.data
    call("uh_pack_write", str(path).encode(), n_layers, n_mtp, n_experts, G13, K13, G2, K2, ptrs, cfg, src)


def test_pack_written_here_reads_in_the_reference(tmp_path):
    r = ref()
    rng = np.random.default_rng(9)
    n_layers, n_mtp, E = 2, 1, 3
    n = (n_layers + n_mtp) * E
    experts = _experts(rng, n)
    path = tmp_path / "experts.pack"
    write_pack(path, n_layers, n_mtp, E, experts, absent={4})
    raw = path.read_bytes()
    hb = (ctypes.c_uint8 * 264)()
    assert r.ref_read_header(str(path).encode(), hb) == 0  # the reference accepts it (magic, version, header hash)
    ours = (ctypes.c_uint8 * 264)()
    call("uh_pack_read_header", str(path).encode(), ours)
    assert bytes(hb) == bytes(ours) == raw[:264]
    h = parse_header(raw)
    slot = 3 * (G13 * K13 // 2 + G13 * K13 // 32)
    assert (h["n_layers"], h["n_mtp"], h["n_experts"], h["n_slots"]) == (n_layers, n_mtp, E, n)
    assert (h["slot_bytes"], h["slots_offset"], h["checksum_offset"]) == (slot, 1 << 20, (1 << 20) + n * slot)
    assert h["part_bytes"] == [G13 * K13 // 2, G13 * K13 // 32] * 2 + [G2 * K2 // 2, G2 * K2 // 32]
    assert (h["w13_out"], h["w13_in"], h["w2_out"], h["w2_in"]) == (G13, K13, G2, K2)
    assert (h["config_hash"], h["source_hash"]) == (0x1234, 0x5678)
    assert not any(raw[264:1 << 20])  # the header page's rest and the gap to the first slot are zero
    table_bytes = -(-n * 16 // 4096) * 4096
    assert len(raw) == h["checksum_offset"] + table_bytes
    for i in range(n):
        s = np.frombuffer(raw, np.uint8, slot, h["slots_offset"] + i * slot)
        hash_, present = struct.unpack_from("<QQ", raw, h["checksum_offset"] + 16 * i)
        if i == 4:
            assert (hash_, present) == (0, 0) and not s.any()
            continue
        assert present == 1 and hash_ == r.ref_xxh64(s.ctypes.data, slot, 0)
        for m, (rows, cols) in enumerate(((G13, K13), (G13, K13), (G2, K2))):
            tw = np.empty(rows * cols // 2, np.uint8)
            ts = np.empty(rows * cols // 32, np.uint8)
            r.ref_repack_matrix(experts[i][2 * m].ctypes.data, experts[i][2 * m + 1].ctypes.data, tw.ctypes.data,
                                ts.ctypes.data, rows, cols)
            o_w, o_s = h["part_offset"][2 * m], h["part_offset"][2 * m + 1]
            assert np.array_equal(s[o_w:o_w + tw.size], tw) and np.array_equal(s[o_s:o_s + ts.size], ts)


def test_pack_header_damage_is_refused(tmp_path):
    rng = np.random.default_rng(1)
    path = tmp_path / "p.pack"
    write_pack(path, 1, 0, 1, _experts(rng, 1))
    raw = bytearray(path.read_bytes())
    raw[40] ^= 1  # slot_bytes: the header hash no longer matches
    path.write_bytes(bytes(raw))
    with pytest.raises(Exception, match="header hash"):
        call("uh_pack_read_header", str(path).encode(), (ctypes.c_uint8 * 264)())
    with pytest.raises(Exception, match="4096"):  # a slot that is not whole 4 KiB pages
        call("uh_pack_write", str(tmp_path / "q").encode(), 1, 0, 1, 256, 256, 256, 256,
             (ctypes.c_void_p * 6)(), 0, 0)
    assert not os.path.exists(tmp_path / "q.tmp")
