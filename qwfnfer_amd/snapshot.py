"""KV cache snapshot files: one sequence of one layer's cache as the
reference's own cache rows.

The reference keeps no snapshot of its caches (its state lives only in the
backend buffers of ``state::init``, /root/reference src/qwfn_state.cpp:18-96).
A snapshot here is the token-major rows of that state -- row t = the token's
``n_head_kv * head_dim`` values, head-major (src/qwfn_state.cpp:40, 52-53), in
ggml's layout of the cache type: ``block_q8_0`` {fp16 d; int8 qs[32]},
``block_q4_0`` {fp16 d; uint8 qs[16]} or fp16 values -- for K and for V, behind
a small self-describing header, so a C++ engine can write or read the same
bytes with fread/fwrite and no other dependency.

File format, little-endian:

    offset 0   8 bytes   magic b"QWFNKV\\x00\\x01"
    offset 8   4 bytes   u32 H, the header length
    offset 12  H bytes   UTF-8 JSON object: format ("ggml-q8_0-rows",
                         "ggml-q4_0-rows" or "ggml-f16-rows"), n_head_kv,
                         head_dim, block_tokens, quant_variant, kv_type,
                         n_tokens, row_bytes, k_offset, v_offset
    k_offset             K rows, n_tokens * row_bytes bytes
    v_offset             V rows, n_tokens * row_bytes bytes

The pooled block keys are not stored: they are a function of K and are
rebuilt on load (:func:`load_snapshot` pools every whole block).
"""
from __future__ import annotations

import json
import struct
from typing import Optional, Tuple

import numpy as np

MAGIC = b"QWFNKV\x00\x01"
FORMATS = {0: "ggml-q8_0-rows", 1: "ggml-q4_0-rows", 2: "ggml-f16-rows"}   # by kv_type
FORMAT = FORMATS[0]
_FIELDS = ("n_head_kv", "head_dim", "block_tokens", "quant_variant")


def row_bytes(n_head_kv: int, head_dim: int, kv_type: int = 0) -> int:
    """One token's row of the reference's cache tensor of the type."""
    if kv_type == 2:
        return n_head_kv * head_dim * 2
    return n_head_kv * (head_dim // 32) * (18 if kv_type == 1 else 34)


def write_snapshot_file(path: str, header: dict, k_rows: np.ndarray, v_rows: np.ndarray) -> dict:
    """Write K and V rows (uint8 [n_tokens, row_bytes] each) under a header
    holding at least ``n_head_kv``, ``head_dim``, ``block_tokens`` and
    ``quant_variant``.  Returns the header as written."""
    k_rows = np.ascontiguousarray(k_rows, dtype=np.uint8)
    v_rows = np.ascontiguousarray(v_rows, dtype=np.uint8)
    missing = [f for f in _FIELDS if f not in header]
    if missing:
        raise ValueError(f"snapshot header lacks {missing}")
    kt = int(header.get("kv_type", 0))
    if kt not in FORMATS:
        raise ValueError(f"kv_type {kt} unknown")
    rb = row_bytes(int(header["n_head_kv"]), int(header["head_dim"]), kt)
    if k_rows.ndim != 2 or k_rows.shape[1] != rb or v_rows.shape != k_rows.shape:
        raise ValueError(f"rows must be uint8 [n_tokens, {rb}] for K and V alike, got "
                         f"{k_rows.shape} and {v_rows.shape}")
    n = int(k_rows.shape[0])
    h = {"format": FORMATS[kt], **{f: int(header[f]) for f in _FIELDS}, "kv_type": kt, "n_tokens": n,
         "row_bytes": rb, "k_offset": 0, "v_offset": 0}
    # the offsets depend on the header's own length: iterate to the fixed point
    # (the length only grows with the offsets' digits, so this settles at once)
    while True:
        blob = json.dumps(h, sort_keys=True).encode("utf-8")
        base = len(MAGIC) + 4 + len(blob)
        if h["k_offset"] == base:
            break
        h["k_offset"], h["v_offset"] = base, base + n * rb
    with open(path, "wb") as f:
        f.write(MAGIC)
        f.write(struct.pack("<I", len(blob)))
        f.write(blob)
        f.write(k_rows.tobytes())
        f.write(v_rows.tobytes())
    return h


def read_snapshot_file(path: str) -> Tuple[dict, np.ndarray, np.ndarray]:
    """Read a snapshot: (header, k_rows, v_rows), the rows memory-mapped
    read-only.  Raises ValueError on a file this format does not describe."""
    with open(path, "rb") as f:
        magic = f.read(len(MAGIC))
        if magic != MAGIC:
            raise ValueError(f"{path}: not a KV snapshot (magic {magic!r})")
        (hl,) = struct.unpack("<I", f.read(4))
        h = json.loads(f.read(hl).decode("utf-8"))
    kt = int(h.get("kv_type", 0))
    if kt not in FORMATS or h.get("format") != FORMATS[kt]:
        raise ValueError(f"{path}: unknown snapshot format {h.get('format')!r}")
    n, rb = int(h["n_tokens"]), int(h["row_bytes"])
    if rb != row_bytes(int(h["n_head_kv"]), int(h["head_dim"]), kt):
        raise ValueError(f"{path}: row_bytes {rb} does not match the head shape")
    mm = np.memmap(path, dtype=np.uint8, mode="r")
    k0, v0 = int(h["k_offset"]), int(h["v_offset"])
    if k0 != len(MAGIC) + 4 + hl or v0 != k0 + n * rb or mm.size != v0 + n * rb:
        raise ValueError(f"{path}: size or offsets inconsistent with {n} rows of {rb} bytes")
    return h, mm[k0:k0 + n * rb].reshape(n, rb), mm[v0:v0 + n * rb].reshape(n, rb)


def save_snapshot(cache, path: str, seq: int, n_tokens: int, stream=None) -> dict:
    """Positions [0, n_tokens) of sequence ``seq`` of a device cache
    (:class:`qwfnfer_amd.qsa.KvCache`) to a snapshot file.  Synchronises."""
    import torch
    from . import qsa
    kr, vr = qsa.export_rows_q8_0(cache, seq, 0, n_tokens, stream=stream)
    torch.cuda.synchronize()
    cfg = cache.cfg
    return write_snapshot_file(path, {"n_head_kv": cfg.n_head_kv, "head_dim": cfg.head_dim,
                                      "block_tokens": cfg.block_tokens, "quant_variant": cfg.quant_variant,
                                      "kv_type": cfg.kv_type},
                               kr.cpu().numpy(), vr.cpu().numpy())


def load_snapshot(cache, path: str, seq: int, stream=None) -> int:
    """Load a snapshot into positions [0, n_tokens) of sequence ``seq`` and pool
    its whole blocks.  The cache's head shape and block size must match the
    file's.  Returns n_tokens."""
    import torch
    from . import qsa
    h, kr, vr = read_snapshot_file(path)
    cfg = cache.cfg
    for f in ("n_head_kv", "head_dim", "block_tokens", "kv_type"):
        if int(h.get(f, 0)) != int(getattr(cfg, f)):
            raise ValueError(f"{path}: {f} {h[f]} does not match the cache's {getattr(cfg, f)}")
    n = int(h["n_tokens"])
    dev = cache.k_pages.device
    kd = torch.from_numpy(np.array(kr)).to(dev)
    vd = torch.from_numpy(np.array(vr)).to(dev)
    qsa.import_rows_q8_0(cache, seq, 0, kd, vd, stream=stream)
    qsa.pool_rebuild(cache, seq, n // cfg.block_tokens, stream=stream)
    torch.cuda.synchronize()
    return n
