"""The KV snapshot file format (host logic only; the device export/import it
wraps is covered by the GPU tests)."""
import json
import struct

import numpy as np
import pytest

from qwfnfer_amd import snapshot as S

HDR = {"n_head_kv": 2, "head_dim": 128, "block_tokens": 64, "quant_variant": 0}


def _rows(rng, n, rb=272):
    return rng.integers(0, 256, (n, rb), dtype=np.uint8), rng.integers(0, 256, (n, rb), dtype=np.uint8)


@pytest.mark.parametrize("n", [0, 1, 63, 1000])
def test_round_trip(tmp_path, n):
    rng = np.random.default_rng(n)
    k, v = _rows(rng, n)
    p = str(tmp_path / "s.kv")
    h = S.write_snapshot_file(p, HDR, k, v)
    h2, k2, v2 = S.read_snapshot_file(p)
    assert h2 == h and h["n_tokens"] == n and h["row_bytes"] == 272
    np.testing.assert_array_equal(k2, k)
    np.testing.assert_array_equal(v2, v)


def test_layout_is_the_documented_one(tmp_path):
    rng = np.random.default_rng(7)
    k, v = _rows(rng, 5)
    p = str(tmp_path / "s.kv")
    S.write_snapshot_file(p, HDR, k, v)
    raw = open(p, "rb").read()
    assert raw[:8] == b"QWFNKV\x00\x01"
    (hl,) = struct.unpack("<I", raw[8:12])
    h = json.loads(raw[12:12 + hl])
    assert h["format"] == "ggml-q8_0-rows" and h["k_offset"] == 12 + hl
    assert raw[h["k_offset"]:h["k_offset"] + 5 * 272] == k.tobytes()
    assert raw[h["v_offset"]:] == v.tobytes()


def test_row_bytes_is_the_ggml_block_count():
    # head-major row of n_head_kv * head_dim elements in 32-element blocks of 34 bytes
    assert S.row_bytes(2, 128) == 8 * 34
    assert S.row_bytes(2, 256) == 16 * 34
    assert S.row_bytes(1, 64) == 2 * 34


def test_rejects_malformed(tmp_path):
    rng = np.random.default_rng(8)
    k, v = _rows(rng, 3)
    p = str(tmp_path / "s.kv")
    with pytest.raises(ValueError):
        S.write_snapshot_file(p, {"n_head_kv": 2}, k, v)                 # header incomplete
    with pytest.raises(ValueError):
        S.write_snapshot_file(p, HDR, k[:, :100], v[:, :100])          # wrong row size
    S.write_snapshot_file(p, HDR, k, v)
    raw = bytearray(open(p, "rb").read())
    open(p, "wb").write(raw[:-1])                                      # truncated
    with pytest.raises(ValueError):
        S.read_snapshot_file(p)
    bad = bytearray(raw)
    bad[0] ^= 0xff                                                      # wrong magic
    open(p, "wb").write(bad)
    with pytest.raises(ValueError):
        S.read_snapshot_file(p)
