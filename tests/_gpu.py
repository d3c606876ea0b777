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


FILL_CHUNK = 65536


def fill(dev, host, rng, lengths, scaled: bool = True, pool: bool = True, rows=None):
    """Append tokens [0, L_s) of every sequence s on both sides and pool every
    whole block.  Up to FILL_CHUNK tokens a sequence take one device call;
    longer ones are drawn and appended FILL_CHUNK tokens at a time.  `rows`
    (rng, n, cfg) -> (k, v) replaces the default draw."""
    cfg = host.cfg
    for s, L in enumerate(lengths):
        if L <= 0:
            continue
        for t0 in range(0, L, FILL_CHUNK):
            n = min(FILL_CHUNK, L - t0)
            k, v = rows(rng, n, cfg) if rows else kv_rows(rng, n, cfg, scaled)
            pos = np.arange(t0, t0 + n, dtype=np.int32)
            sid = np.full(n, s, dtype=np.int32)
            assert host.append(k, v, pos, sid) == 0
            qsa.append_q8_0(dev, torch.from_numpy(k).cuda(), torch.from_numpy(v).cuda(),
                            torch.from_numpy(pos).cuda(), torch.from_numpy(sid).cuda())
            del k, v
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
    bad = ~(err <= bound)                     # a NaN or inf output (NaN error) fails too
    assert not bad.any(), (f"{what}: {bad.sum()} elements out of tolerance, max abs err "
                           f"{err.max():.3g}, max rel {np.max(err / np.maximum(np.abs(ref), 1e-30)):.3g}")
    return float(err.max())


def decode_steps(cfg, lengths, steps, seed, dtype=np.float32, zero_pooled=False, modes=None,
                 reattend=False, verbose=False):
    """Decode steps on a batch of sequences vs the oracle's append + pool on
    completion + indexer + fp64 attention.

    modes: one entry per step, "fused" (qwfn_sparse_attn_decode) or "two_call"
    (qwfn_decode_append_select, then qwfn_sparse_decode_attn over its
    selection); default all fused.  reattend: after every step also run
    qwfn_sparse_decode_attn over the step's selection and check its output.
    zero_pooled: every pooled key of the filled prefix set to 0 on both sides
    (all scores tie).  Every step checks the selection bit-exact and the
    attention within tolerance; the end checks cache bytes and pooled keys."""
    rng = np.random.default_rng(seed)
    n_seq = len(lengths)
    modes = list(modes) if modes is not None else ["fused"] * steps
    assert len(modes) == steps
    pps = (max(lengths) + steps) // cfg.page_tokens + 1
    dev, host = make_pair(cfg, n_seq, pps, seed=seed)
    fill(dev, host, rng, lengths)
    if zero_pooled:
        host.pooled[...] = 0
        dev.pooled.zero_()
    cur = np.array(lengths, np.int32)
    max_len = int(cur.max()) + steps
    c = cfg_of(cfg)
    ws = qsa.Workspace(c, n_seq, max_len)
    msel = c.max_selected(max_len)
    sel = torch.empty((n_seq, cfg.n_head_kv, msel), dtype=torch.int32, device="cuda")
    nsel = torch.empty((n_seq, cfg.n_head_kv), dtype=torch.int32, device="cuda")
    outs = []
    for step, mode in enumerate(modes):
        cur = cur + 1
        q = rng.standard_normal((n_seq, cfg.n_head, cfg.head_dim), dtype=np.float32)
        kn, vn = kv_rows(rng, n_seq, cfg)
        kn, vn = kn.astype(dtype), vn.astype(dtype)
        qd, knd, vnd = torch.from_numpy(q).cuda(), torch.from_numpy(kn).cuda(), torch.from_numpy(vn).cuda()
        curd = torch.from_numpy(cur).cuda()
        if verbose:
            print(f"  step {step} {mode} seq_len {cur.tolist()}", flush=True)
        if mode == "fused":
            out = qsa.sparse_attn_decode(dev, qd, knd, vnd, curd, max_len, ws, sel=sel, n_sel=nsel)
        elif mode == "two_call":
            qsa.decode_append_select(dev, qd, knd, vnd, curd, max_len, ws, sel, nsel)
            out = qsa.sparse_decode_attn(dev, qd, curd, max_len, ws, sel, nsel)
        else:
            raise ValueError(mode)
        out2 = qsa.sparse_decode_attn(dev, qd, curd, max_len, ws, sel, nsel) if reattend else None
        torch.cuda.synchronize()
        for s in range(n_seq):
            p = int(cur[s]) - 1
            assert host.append(kn[s:s + 1], vn[s:s + 1], [p], [s]) == 0
            if cur[s] % cfg.block_tokens == 0:
                host.pool_block(s, p // cfg.block_tokens)
        hs, hn = host.indexer_topk(q, cur, max_sel=msel)
        gs, gn = np_of(sel), np_of(nsel)
        np.testing.assert_array_equal(gn, hn, err_msg=f"step {step} ({mode})")
        for s in range(n_seq):
            for g in range(cfg.n_head_kv):
                np.testing.assert_array_equal(gs[s, g, :gn[s, g]], hs[s, g, :hn[s, g]],
                                              err_msg=f"step {step} ({mode}) seq {s} head {g}")
        ref = host.attention_f64(q, cur, hs, hn)
        assert_close_attn(np_of(out), ref, f"decode step {step} ({mode})")
        if out2 is not None:
            assert_close_attn(np_of(out2), ref, f"decode step {step}: attention over the step's selection")
        outs.append(np_of(out))
    assert qsa.read_status(dev) == 0
    np.testing.assert_array_equal(np_of(dev.k_pages), host.k_pages)
    np.testing.assert_array_equal(np_of(dev.v_pages), host.v_pages)
    for s in range(n_seq):
        nw = int(cur[s]) // cfg.block_tokens
        np.testing.assert_array_equal(np_of(dev.pooled)[s, :, :nw], host.pooled[s, :, :nw])
    return outs
