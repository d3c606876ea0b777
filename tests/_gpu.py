"""Helpers of the GPU parity tests: a device cache and its host (oracle) twin
filled with the same seeded rows."""
from __future__ import annotations

import numpy as np
import torch

from oracle import oracle as O
from qwfnfer_amd import qsa


def cfg_of(c) -> qsa.QsaConfig:
    return qsa.QsaConfig(**{k: getattr(c, k) for k in qsa.QsaConfig.__dataclass_fields__})


def make_pair(cfg, n_seq: int, pages_per_seq: int, seed: int | None = None, spare: int = 0):
    """Device KvCache + HostCache with one page table (permuted when seed is
    given; `spare` extra physical pages stay unused)."""
    n_phys = n_seq * pages_per_seq + spare
    if seed is None:
        pt = np.arange(n_seq * pages_per_seq, dtype=np.int32).reshape(n_seq, pages_per_seq)
    else:
        pt = np.random.default_rng(seed).permutation(n_phys)[: n_seq * pages_per_seq]
        pt = pt.astype(np.int32).reshape(n_seq, pages_per_seq)
    dev = qsa.KvCache.allocate(cfg_of(cfg), n_seq, pages_per_seq, page_table=torch.from_numpy(pt),
                               n_phys_pages=n_phys)
    host = O.HostCache(cfg, n_seq, pages_per_seq, page_table=pt, n_phys_pages=n_phys)
    return dev, host


def kv_rows(rng, n: int, cfg, scaled: bool = True):
    """K, V ~ N(0,1) [n, Hkv, hd], each q8_0 block times a log-uniform [0.1, 10]
    scale when `scaled` (the configuration's scale draw)."""
    shp = (n, cfg.n_head_kv, cfg.head_dim)
    k = rng.standard_normal(shp, dtype=np.float32)
    v = rng.standard_normal(shp, dtype=np.float32)
    if scaled:
        nb = cfg.head_dim // 32
        for x in (k, v):
            s = np.exp(rng.uniform(np.log(0.1), np.log(10.0), (n, cfg.n_head_kv, nb))).astype(np.float32)
            x.reshape(n, cfg.n_head_kv, nb, 32)[...] *= s[..., None]
    return k, v


def fill(dev, host, rng, lengths, scaled: bool = True, pool: bool = True):
    """Append tokens [0, L_s) of every sequence s on both sides (one device call
    per sequence) and pool every whole block."""
    cfg = host.cfg
    for s, L in enumerate(lengths):
        if L <= 0:
            continue
        k, v = kv_rows(rng, L, cfg, scaled)
        pos = np.arange(L, dtype=np.int32)
        sid = np.full(L, s, dtype=np.int32)
        assert host.append(k, v, pos, sid) == 0
        qsa.append_q8_0(dev, torch.from_numpy(k).cuda(), torch.from_numpy(v).cuda(),
                        torch.from_numpy(pos).cuda(), torch.from_numpy(sid).cuda())
        if pool and L // cfg.block_tokens > 0:
            nw = L // cfg.block_tokens
            for b in range(nw):
                assert host.pool_block(s, b) == 0
            qsa.pool_rebuild(dev, s, nw)
    torch.cuda.synchronize()


def np_of(t: torch.Tensor) -> np.ndarray:
    return t.detach().cpu().numpy()


def assert_close_attn(got: np.ndarray, ref: np.ndarray, what: str = ""):
    """The acceptance bound: |o - o_ref| <= 2e-3 + 1e-3 |o_ref| elementwise."""
    err = np.abs(got.astype(np.float64) - ref)
    bound = 2e-3 + 1e-3 * np.abs(ref)
    bad = err > bound
    assert not bad.any(), (f"{what}: {bad.sum()} elements out of tolerance, max abs err "
                           f"{err.max():.3g}, max rel {np.max(err / np.maximum(np.abs(ref), 1e-30)):.3g}")
    return float(err.max())
