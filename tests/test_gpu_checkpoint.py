"""Parity of the checkpoint's own indexer (qwfn_idx_*) with the CPU oracle, at
the checkpoint's attention shape (24 query heads, 2 KV heads of 256, blocks of
4 tokens, 513 kept blocks, only a partial tail forced, one selection for both
KV heads).

Bit-exact: the raw fp16 keys, the pooled keys (same arithmetic order as the
oracle; the rotation's fp64 cos / sin are rounded to fp32, so a last-bit
difference between the device and host libm would surface here), the
selection.  Attention: |o - o_ref| <= 2e-3 + 1e-3 |o_ref| against the fp64
oracle over the same selection."""
import ctypes as C

import numpy as np
import pytest
import torch

from _ckpt import CKPT, ICfg, oracle_pool_all, oracle_select
from _gpu import assert_close_attn, cfg_of, kv_rows, make_pair, np_of
from qwfnfer_amd import _lib, qsa

pytestmark = pytest.mark.gpu

ICFG = ICfg()


def _pair(cfg, n_seq, pps, seed, spare=0):
    dev, host = make_pair(cfg, n_seq, pps, seed=seed, spare=spare)
    rng = np.random.default_rng(seed + 1)
    k_norm = rng.uniform(0.5, 1.5, ICFG.idx_dim).astype(np.float32)
    ic = qsa.IdxCache.allocate(qsa.IdxConfig(**ICFG.__dict__), dev, torch.from_numpy(k_norm))
    return dev, host, ic, k_norm


def _raw_rows(dev, ic, seq, n):
    """The device's raw keys of positions [0, n) of seq, in position order."""
    pt = np_of(dev.page_table)[seq]
    t = np.arange(n)
    return np_of(ic.raw)[pt[t // dev.cfg.page_tokens], t % dev.cfg.page_tokens]


def _ws(cfg, ic, n_seq, L):
    c = cfg_of(cfg)
    return qsa.Workspace(c, n_seq, L, nbytes=max(c.workspace_bytes(n_seq, L), ic.workspace_bytes(n_seq, L)))


@pytest.mark.parametrize("dtype", [np.float32, np.float16])
def test_idx_append_pool_matches_oracle(dtype):
    cfg = CKPT
    rng = np.random.default_rng(800)
    dev, host, ic, w = _pair(cfg, 2, 5, seed=801, spare=1)
    L = 1001
    kr = (rng.standard_normal((L, 128)) * 2).astype(dtype)
    qsa.idx_append_pool(ic, torch.from_numpy(kr).cuda(), torch.arange(L, dtype=torch.int32, device="cuda"))
    torch.cuda.synchronize()
    rows = _raw_rows(dev, ic, 0, L)
    np.testing.assert_array_equal(rows.view(np.uint16), kr.astype(np.float16).view(np.uint16))
    nb = (L + 3) // 4
    want = oracle_pool_all(cfg, ICFG, kr.astype(np.float16), w, nb)
    np.testing.assert_array_equal(np_of(ic.pooled)[0, :nb], want)
    # decode steps: one row at a time, each re-pooling its (partial or just
    # completed) block
    allr = kr.astype(np.float16)
    for step in range(7):
        p = L + step
        x = (rng.standard_normal((1, 128)) * 2).astype(dtype)
        qsa.idx_append_pool(ic, torch.from_numpy(x).cuda(), torch.tensor([p], dtype=torch.int32, device="cuda"))
        torch.cuda.synchronize()
        allr = np.concatenate([allr, x.astype(np.float16)])
        b = p // 4
        got = np_of(ic.pooled)[0, b]
        np.testing.assert_array_equal(got, oracle_pool_all(cfg, ICFG, allr, w, b + 1)[b], err_msg=f"step {step}")
    # rows of the other sequence through seq_ids, out of order
    pos = rng.permutation(64).astype(np.int32)
    x = (rng.standard_normal((64, 128))).astype(dtype)
    qsa.idx_append_pool(ic, torch.from_numpy(x).cuda(), torch.from_numpy(pos).cuda(),
                        seq_ids=torch.ones(64, dtype=torch.int32, device="cuda"))
    torch.cuda.synchronize()
    r1 = np.zeros((64, 128), np.float16)
    r1[pos] = x.astype(np.float16)
    np.testing.assert_array_equal(_raw_rows(dev, ic, 1, 64), r1)
    np.testing.assert_array_equal(np_of(ic.pooled)[1, :16], oracle_pool_all(cfg, ICFG, r1, w, 16))
    assert qsa.read_status(dev) == 0


def test_idx_append_pool_decode_call_rows():
    """A decode-sized call (one launch): rows of two sequences interleaved, a
    repeated (sequence, position) whose last row is kept, and a row past the
    view's sequences that only sets the status bit."""
    cfg = CKPT
    rng = np.random.default_rng(820)
    dev, host, ic, w = _pair(cfg, 2, 2, seed=821)
    L = 37
    base = rng.standard_normal((2, L, 128)).astype(np.float32)
    for s in range(2):
        qsa.idx_append_pool(ic, torch.from_numpy(base[s]).cuda(), torch.arange(L, dtype=torch.int32, device="cuda"),
                            seq_ids=torch.full((L,), s, dtype=torch.int32, device="cuda"))
    seqs = np.array([0, 1, 0, 1, 0, 7], np.int32)
    pos = np.array([37, 37, 38, 12, 37, 3], np.int32)
    x = rng.standard_normal((6, 128)).astype(np.float32)
    qsa.idx_append_pool(ic, torch.from_numpy(x).cuda(), torch.from_numpy(pos).cuda(),
                        seq_ids=torch.from_numpy(seqs).cuda())
    torch.cuda.synchronize()
    assert qsa.read_status(dev) == _lib.STATUS_SEQ_RANGE
    rows = [np.concatenate([base[0], np.zeros((2, 128), np.float32)]).astype(np.float16),
            np.concatenate([base[1], np.zeros((2, 128), np.float32)]).astype(np.float16)]
    rows[0][37] = x[4].astype(np.float16)              # the later of the two rows at (0, 37)
    rows[0][38] = x[2].astype(np.float16)
    rows[1][37] = x[1].astype(np.float16)
    rows[1][12] = x[3].astype(np.float16)
    for s in range(2):
        np.testing.assert_array_equal(_raw_rows(dev, ic, s, 39), rows[s], err_msg=f"seq {s}")
        nb = 10                                        # blocks 0 .. 9 hold positions 0 .. 39
        np.testing.assert_array_equal(np_of(ic.pooled)[s, :nb], oracle_pool_all(cfg, ICFG, rows[s], w, nb),
                                      err_msg=f"seq {s}")


def test_idx_rebuild_matches_oracle():
    cfg = CKPT
    rng = np.random.default_rng(810)
    dev, host, ic, w = _pair(cfg, 1, 12, seed=811)
    L = 3000
    kr = rng.standard_normal((L, 128)).astype(np.float32)
    qsa.idx_append_pool(ic, torch.from_numpy(kr).cuda(), torch.arange(L, dtype=torch.int32, device="cuda"))
    ic.pooled.zero_()
    qsa.idx_pool_rebuild(ic, 0, L // 4)
    torch.cuda.synchronize()
    want = oracle_pool_all(cfg, ICFG, kr.astype(np.float16), w, L // 4)
    np.testing.assert_array_equal(np_of(ic.pooled)[0, :L // 4], want)
    assert not np_of(ic.pooled)[0, L // 4:].any()


@pytest.mark.parametrize("lengths", [[1500], [6000], [6001, 2053], [6003, 4]])
def test_idx_select_matches_oracle(lengths):
    cfg = CKPT
    rng = np.random.default_rng(820 + sum(lengths))
    n = len(lengths)
    pps = max(lengths) // cfg.page_tokens + 1
    dev, host, ic, w = _pair(cfg, n, pps, seed=821)
    for s, L in enumerate(lengths):
        kr = rng.standard_normal((L, 128)).astype(np.float32)
        qsa.idx_append_pool(ic, torch.from_numpy(kr).cuda(), torch.arange(L, dtype=torch.int32, device="cuda"),
                            seq_ids=torch.full((L,), s, dtype=torch.int32, device="cuda"))
    q = rng.standard_normal((n, 4, 128)).astype(np.float32)
    Lmax = max(lengths)
    ws = _ws(cfg, ic, n, Lmax)
    sel, nsel = qsa.idx_select(ic, torch.from_numpy(q).cuda(), torch.tensor(lengths, dtype=torch.int32,
                                                                             device="cuda"), Lmax, ws)
    torch.cuda.synchronize()
    gs, gn, pooled = np_of(sel), np_of(nsel), np_of(ic.pooled)
    for s, L in enumerate(lengths):
        want = oracle_select(cfg, ICFG, pooled[s], q[s], L, sel.shape[-1])
        assert len(want) == min(513, (L + 3) // 4)
        for g in range(2):
            assert gn[s, g] == len(want)
            np.testing.assert_array_equal(gs[s, g, :gn[s, g]], want, err_msg=f"seq {s} head {g}")
    assert qsa.read_status(dev) == 0


def test_checkpoint_decode_steps():
    """Decode steps of the checkpoint layer: K/V and the raw indexer key
    appended, the indexer's block pooled, one selection for both KV heads, the
    attention over it -- each step against the oracle."""
    cfg = CKPT
    rng = np.random.default_rng(830)
    L0 = 5000
    pps = (L0 + 16) // cfg.page_tokens + 1
    dev, host, ic, w = _pair(cfg, 1, pps, seed=831)
    k, v = kv_rows(rng, L0, cfg)
    host.append(k, v, np.arange(L0, dtype=np.int32))
    qsa.append_q8_0(dev, torch.from_numpy(k).cuda(), torch.from_numpy(v).cuda(),
                    torch.arange(L0, dtype=torch.int32, device="cuda"))
    kr = rng.standard_normal((L0, 128)).astype(np.float32)
    qsa.idx_append_pool(ic, torch.from_numpy(kr).cuda(), torch.arange(L0, dtype=torch.int32, device="cuda"))
    c = cfg_of(cfg)
    Lmax = L0 + 6
    ws = _ws(cfg, ic, 1, Lmax)
    msel = c.max_selected(Lmax)
    for step in range(6):
        p = L0 + step
        kn, vn = kv_rows(rng, 1, cfg)
        xr = rng.standard_normal((1, 128)).astype(np.float32)
        q = rng.standard_normal((1, 24, 256)).astype(np.float32)
        qi = rng.standard_normal((1, 4, 128)).astype(np.float32)
        pos = torch.tensor([p], dtype=torch.int32, device="cuda")
        qsa.append_q8_0(dev, torch.from_numpy(kn).cuda(), torch.from_numpy(vn).cuda(), pos)
        qsa.idx_append_pool(ic, torch.from_numpy(xr).cuda(), pos)
        L = torch.tensor([p + 1], dtype=torch.int32, device="cuda")
        sel = torch.empty((1, 2, msel), dtype=torch.int32, device="cuda")
        nsel = torch.empty((1, 2), dtype=torch.int32, device="cuda")
        qsa.idx_select(ic, torch.from_numpy(qi).cuda(), L, Lmax, ws, sel=sel, n_sel=nsel)
        out = qsa.sparse_decode_attn(dev, torch.from_numpy(q).cuda(), L, Lmax, ws, sel=sel, n_sel=nsel)
        torch.cuda.synchronize()
        host.append(kn, vn, [p])
        kr = np.concatenate([kr, xr])
        want = oracle_select(cfg, ICFG, np_of(ic.pooled)[0], qi[0], p + 1, msel)
        np.testing.assert_array_equal(np_of(ic.pooled)[0, p // 4],
                                      oracle_pool_all(cfg, ICFG, kr.astype(np.float16), w, p // 4 + 1)[p // 4])
        gs, gn = np_of(sel), np_of(nsel)
        hs = np.full((1, 2, msel), -1, np.int32)
        for g in range(2):
            assert gn[0, g] == len(want)
            np.testing.assert_array_equal(gs[0, g, :gn[0, g]], want, err_msg=f"step {step} head {g}")
            hs[0, g, :len(want)] = want
        ref = host.attention_f64(q, [p + 1], hs, gn)
        assert_close_attn(np_of(out), ref, f"step {step}")
    assert qsa.read_status(dev) == 0


@pytest.mark.parametrize("dtype,L0", [(np.float32, [4998, 3001]), (np.float16, [4998, 3001]),
                                      (np.float32, [12002, 9001]), (np.float16, [31994, 16001])])
def test_checkpoint_fused_decode_steps(dtype, L0):
    """qwfn_idx_sparse_attn_decode (the K/V rows, the raw indexer key and its
    pooled block in one launch, then the indexer and the attention) for two
    sequences over steps that complete blocks in each: the cache bytes, raw and
    pooled keys and selections bit-exact against the oracle, the attention
    within the tolerance; a twin cache stepped through the four separate calls
    ends with the same bytes, selections and outputs bit for bit.  Up to 8,192
    blocks every attention workgroup selects from the indexer's row, with 8,
    16 and 32 keys a thread at these lengths."""
    cfg = CKPT
    rng = np.random.default_rng(850)            # block completions within the 7 steps in each sequence
    steps = 7
    pps = (max(L0) + steps + 8) // cfg.page_tokens + 1
    pairs = [_pair(cfg, 2, pps, seed=851), _pair(cfg, 2, pps, seed=851)]
    dev, host, ic, w = pairs[0]
    dev2, _, ic2, _ = pairs[1]
    kr = []
    for s in range(2):
        k, v = kv_rows(rng, L0[s], cfg)
        assert host.append(k, v, np.arange(L0[s], dtype=np.int32), np.full(L0[s], s, np.int32)) == 0
        x = rng.standard_normal((L0[s], 128)).astype(np.float32)
        kr.append(x)
        for d, c in ((dev, ic), (dev2, ic2)):
            qsa.append_q8_0(d, torch.from_numpy(k).cuda(), torch.from_numpy(v).cuda(),
                            torch.arange(L0[s], dtype=torch.int32, device="cuda"),
                            seq_ids=torch.full((L0[s],), s, dtype=torch.int32, device="cuda"))
            qsa.idx_append_pool(c, torch.from_numpy(x).cuda(), torch.arange(L0[s], dtype=torch.int32, device="cuda"),
                                seq_ids=torch.full((L0[s],), s, dtype=torch.int32, device="cuda"))
    c = cfg_of(cfg)
    Lmax = max(L0) + steps + 1
    ws, ws2 = _ws(cfg, ic, 2, Lmax), _ws(cfg, ic2, 2, Lmax)
    msel = c.max_selected(Lmax)
    tdt = torch.float16 if dtype == np.float16 else torch.float32
    for step in range(steps):
        lens = [L + step + 1 for L in L0]
        print(f"  fused idx decode step {step}, lengths {lens}, {np.dtype(dtype).name} rows", flush=True)
        kn, vn = kv_rows(rng, 2, cfg)
        kn, vn = kn.astype(dtype), vn.astype(dtype)
        xr = rng.standard_normal((2, 128)).astype(dtype)
        q = rng.standard_normal((2, 24, 256)).astype(np.float32)
        qi = rng.standard_normal((2, 4, 128)).astype(np.float32)
        L = torch.tensor(lens, dtype=torch.int32, device="cuda")
        sel = torch.full((2, 2, msel), -7, dtype=torch.int32, device="cuda")   # entries past n_sel stay as filled
        nsel = torch.empty((2, 2), dtype=torch.int32, device="cuda")
        qd, qid = torch.from_numpy(q).cuda(), torch.from_numpy(qi).cuda()
        knd, vnd, xrd = (torch.from_numpy(a).cuda() for a in (kn, vn, xr))
        out = qsa.idx_sparse_attn_decode(ic, qd, qid, knd, vnd, xrd, L, Lmax, ws, sel=sel, n_sel=nsel)
        # the twin: the four calls of the same step
        pos = L - 1
        qsa.append_q8_0(dev2, knd, vnd, pos, seq_ids=torch.arange(2, dtype=torch.int32, device="cuda"))
        qsa.idx_append_pool(ic2, xrd, pos, seq_ids=torch.arange(2, dtype=torch.int32, device="cuda"))
        sel2 = torch.full_like(sel, -7)
        nsel2 = torch.empty_like(nsel)
        qsa.idx_select(ic2, qid, L, Lmax, ws2, sel=sel2, n_sel=nsel2)
        out2 = qsa.sparse_decode_attn(dev2, qd, L, Lmax, ws2, sel=sel2, n_sel=nsel2)
        torch.cuda.synchronize()
        assert host.append(kn, vn, np.array([l - 1 for l in lens], np.int32), np.arange(2, dtype=np.int32)) == 0
        hs = np.full((2, 2, msel), -1, np.int32)
        gs, gn = np_of(sel), np_of(nsel)
        for s in range(2):
            p = lens[s] - 1
            kr[s] = np.concatenate([kr[s], xr[s:s + 1].astype(np.float32)])
            np.testing.assert_array_equal(np_of(ic.pooled)[s, p // 4],
                                          oracle_pool_all(cfg, ICFG, kr[s].astype(np.float16), w, p // 4 + 1)[p // 4],
                                          err_msg=f"step {step} seq {s} pooled key")
            want = oracle_select(cfg, ICFG, np_of(ic.pooled)[s], qi[s], lens[s], msel)
            for g in range(2):
                assert gn[s, g] == len(want)
                np.testing.assert_array_equal(gs[s, g, :gn[s, g]], want, err_msg=f"step {step} seq {s} head {g}")
                hs[s, g, :len(want)] = want
        ref = host.attention_f64(q, lens, hs, gn)
        assert_close_attn(np_of(out), ref, f"step {step}")
        assert torch.equal(out, out2) and torch.equal(sel, sel2) and torch.equal(nsel, nsel2), f"step {step}"
    np.testing.assert_array_equal(np_of(dev.k_pages), host.k_pages)
    np.testing.assert_array_equal(np_of(dev.v_pages), host.v_pages)
    for a, b in ((dev.k_pages, dev2.k_pages), (dev.v_pages, dev2.v_pages), (ic.raw, ic2.raw), (ic.pooled, ic2.pooled)):
        assert torch.equal(a, b)
    for s in range(2):
        np.testing.assert_array_equal(_raw_rows(dev, ic, s, L0[s] + steps), kr[s].astype(np.float16), err_msg=f"seq {s}")
    assert qsa.read_status(dev) == 0


@pytest.mark.parametrize("dtype", [np.float32, np.float16])
def test_checkpoint_prefill(dtype):
    """A prefill chunk with the checkpoint's indexer: K/V and raw keys appended,
    the touched blocks pooled, each query selected by its q_idx and attending
    causally -- selections for every query, outputs for a sample."""
    cfg = CKPT
    rng = np.random.default_rng(840)
    pre, n_q = 2600, 203
    end = pre + n_q
    pps = end // cfg.page_tokens + 1
    dev, host, ic, w = _pair(cfg, 1, pps, seed=841)
    k, v = kv_rows(rng, pre, cfg)
    host.append(k, v, np.arange(pre, dtype=np.int32))
    qsa.append_q8_0(dev, torch.from_numpy(k).cuda(), torch.from_numpy(v).cuda(),
                    torch.arange(pre, dtype=torch.int32, device="cuda"))
    kr0 = rng.standard_normal((pre, 128)).astype(np.float32)
    qsa.idx_append_pool(ic, torch.from_numpy(kr0).cuda(), torch.arange(pre, dtype=torch.int32, device="cuda"))
    kn, vn = kv_rows(rng, n_q, cfg)
    kn, vn = kn.astype(dtype), vn.astype(dtype)
    krn = rng.standard_normal((n_q, 128)).astype(dtype)
    q = rng.standard_normal((n_q, 24, 256)).astype(np.float32)
    qi = rng.standard_normal((n_q, 4, 128)).astype(np.float32)
    c = cfg_of(cfg)
    msel = c.max_selected(end)
    sel = torch.empty((n_q, 2, msel), dtype=torch.int32, device="cuda")
    nsel = torch.empty((n_q, 2), dtype=torch.int32, device="cuda")
    ws = qsa.Workspace.for_prefill(c, end, 64)
    out = qsa.idx_sparse_attn_prefill(ic, torch.from_numpy(q).cuda(), torch.from_numpy(qi).cuda(), 0, pre, ws,
                                      k_new=torch.from_numpy(kn).cuda(), v_new=torch.from_numpy(vn).cuda(),
                                      k_raw=torch.from_numpy(krn).cuda(), sel=sel, n_sel=nsel)
    torch.cuda.synchronize()
    assert qsa.read_status(dev) == 0
    host.append(kn, vn, np.arange(pre, end, dtype=np.int32))
    allr = np.concatenate([kr0.astype(np.float16), krn.astype(np.float16)])
    nb = (end + 3) // 4
    pooled = np_of(ic.pooled)[0]
    np.testing.assert_array_equal(pooled[:nb], oracle_pool_all(cfg, ICFG, allr, w, nb))
    np.testing.assert_array_equal(np_of(dev.k_pages), host.k_pages)
    gs, gn, o = np_of(sel), np_of(nsel), np_of(out)
    for i in range(n_q):
        want = oracle_select(cfg, ICFG, pooled, qi[i], pre + i + 1, msel)
        for g in range(2):
            assert gn[i, g] == len(want), f"query {i}"
            np.testing.assert_array_equal(gs[i, g, :gn[i, g]], want, err_msg=f"query {i} head {g}")
        if i % 29 == 0 or i == n_q - 1:
            ref = host.attention_f64(q[i:i + 1], [pre + i + 1], gs[i:i + 1], gn[i:i + 1])
            assert_close_attn(o[i:i + 1], ref, f"query {i}")


# ---- long contexts: more eligible blocks than the indexer workgroup's
# registers hold (8192), selected by the multi-workgroup k_select_cut ------------

@pytest.mark.parametrize("lengths,mode", [([40003], "random"), ([33000, 45001], "random"), ([36000], "tie"),
                                          ([40003], "cluster")])
def test_idx_select_long_context(lengths, mode):
    """The checkpoint selection over 8,250 .. 11,250 blocks.  random: the top
    blocks spread over the score row.  tie: all-zero raw keys, so every block
    scores the same and the index order decides (the threshold bin overflows
    the candidate list: the radix fallback).  cluster: 200 consecutive blocks
    whose unrotated dims align with the query heads, so the top blocks crowd
    into a few of the selection workgroups' regions."""
    cfg = CKPT
    tie = mode == "tie"
    rng = np.random.default_rng(850 + sum(lengths) + tie + 7 * (mode == "cluster"))
    n = len(lengths)
    pps = max(lengths) // cfg.page_tokens + 1
    dev, host, ic, w = _pair(cfg, n, pps, seed=851)
    q = rng.standard_normal((n, 4, 128)).astype(np.float32)
    for s, L in enumerate(lengths):
        kr = np.zeros((L, 128), np.float32) if tie else rng.standard_normal((L, 128)).astype(np.float32)
        if mode == "cluster":                      # blocks 2000 .. 2199: dims 64.. along the heads' sum
            kr[8000:8800, :64] *= 0.01
            kr[8000:8800, 64:] = 0.01 * kr[8000:8800, 64:] + q[s, :, 64:].sum(0)
        qsa.idx_append_pool(ic, torch.from_numpy(kr).cuda(), torch.arange(L, dtype=torch.int32, device="cuda"),
                            seq_ids=torch.full((L,), s, dtype=torch.int32, device="cuda"))
    Lmax = max(lengths)
    ws = _ws(cfg, ic, n, Lmax)
    sel, nsel = qsa.idx_select(ic, torch.from_numpy(q).cuda(),
                               torch.tensor(lengths, dtype=torch.int32, device="cuda"), Lmax, ws)
    torch.cuda.synchronize()
    gs, gn, pooled = np_of(sel), np_of(nsel), np_of(ic.pooled)
    for s, L in enumerate(lengths):
        want = oracle_select(cfg, ICFG, pooled[s], q[s], L, sel.shape[-1])
        assert len(want) == 513
        if tie:                                    # the lowest indices, and the partial tail
            nb = L // 4
            exp = list(range(513 - (1 if L % 4 else 0))) + ([nb] if L % 4 else [])
            np.testing.assert_array_equal(want, np.array(exp, np.int32))
        if mode == "cluster":                      # the whole cluster is selected
            assert set(range(2000, 2200)) <= set(want.tolist())
        for g in range(2):
            assert gn[s, g] == 513
            np.testing.assert_array_equal(gs[s, g, :513], want, err_msg=f"seq {s} head {g}")
    assert qsa.read_status(dev) == 0


def _set_cut_polls(n: int) -> int:
    prev = C.c_int32()
    _lib.call("qwfn_qsa_test_set_cut_polls", n, C.byref(prev))
    return prev.value


@pytest.mark.parametrize("mode", ["random", "cluster", "newest", "no_poll", "eight", "long_max"])
def test_checkpoint_fused_decode_long_context(mode, request):
    """qwfn_idx_sparse_attn_decode past 8192 eligible blocks, where the
    attention workgroups select from the indexer's score row themselves (no
    selection launch): two sequences over two steps, the selections bit for
    bit against the oracle's, the attention within the tolerance, and the
    outputs and selections bit for bit equal to the four separate calls
    (qwfn_idx_select's multi-workgroup selection, then the given-selection
    attention).  cluster: 200 consecutive blocks aligned with the query heads'
    sum, so the winners crowd into one run of the row.  newest: both tokens of
    step 0 complete a block whose rows (the new one too) are so aligned, so the
    block the indexer launch's append workgroup re-pools and scores must win.
    no_poll: the scoring workgroups' wait for the launch's sampled cut bounded
    at zero polls (qwfn_qsa_test_set_cut_polls), so every chunk leaves no
    candidates and the attention selects over the whole row; both tokens of
    step 0 complete a block.  eight: eight sequences, more indexer workgroups
    than the device holds at once, so later sequences' cut workgroups start
    only as earlier sequences' scoring workgroups finish.  long_max: a call bound
    (max_seq_len 120,001) far past the lengths, so most of the indexer's chunk
    workgroups lie past the eligible blocks and end without waiting."""
    cfg = CKPT
    rng = np.random.default_rng(880 + ("random", "cluster", "newest", "no_poll", "eight", "long_max").index(mode))
    L0 = ([40003, 45003] if mode in ("newest", "no_poll") else
          [33001 + 997 * i for i in range(8)] if mode == "eight" else [40003, 45001])
    ns = len(L0)
    if mode == "no_poll":
        prev = _set_cut_polls(0)
        request.addfinalizer(lambda: _set_cut_polls(prev))
    steps = 2
    Lmax = 120001 if mode == "long_max" else max(L0) + steps + 1
    pps = (Lmax + 8) // cfg.page_tokens + 1
    pairs = [_pair(cfg, ns, pps, seed=881), _pair(cfg, ns, pps, seed=881)]
    dev, host, ic, w = pairs[0]
    dev2, _, ic2, _ = pairs[1]
    qi_all = rng.standard_normal((steps, ns, 4, 128)).astype(np.float32)
    for s in range(ns):
        k, v = kv_rows(rng, L0[s], cfg)
        assert host.append(k, v, np.arange(L0[s], dtype=np.int32), np.full(L0[s], s, np.int32)) == 0
        x = rng.standard_normal((L0[s], 128)).astype(np.float32)
        if mode == "cluster":                      # blocks 2000 .. 2199 along the heads' sum of step 0
            x[8000:8800, :64] *= 0.01
            x[8000:8800, 64:] = 0.01 * x[8000:8800, 64:] + qi_all[0, s, :, 64:].sum(0)
        if mode == "newest":                       # the block step 0 completes, its first three rows
            x[-3:, :64] *= 0.01
            x[-3:, 64:] = 0.01 * x[-3:, 64:] + qi_all[0, s, :, 64:].sum(0)
        for d, c in ((dev, ic), (dev2, ic2)):
            qsa.append_q8_0(d, torch.from_numpy(k).cuda(), torch.from_numpy(v).cuda(),
                            torch.arange(L0[s], dtype=torch.int32, device="cuda"),
                            seq_ids=torch.full((L0[s],), s, dtype=torch.int32, device="cuda"))
            qsa.idx_append_pool(c, torch.from_numpy(x).cuda(), torch.arange(L0[s], dtype=torch.int32, device="cuda"),
                                seq_ids=torch.full((L0[s],), s, dtype=torch.int32, device="cuda"))
    c = cfg_of(cfg)
    ws, ws2 = _ws(cfg, ic, ns, Lmax), _ws(cfg, ic2, ns, Lmax)
    msel = c.max_selected(Lmax)
    for step in range(steps):
        lens = [L + step + 1 for L in L0]
        print(f"  fused idx decode, long context ({mode}), step {step}, lengths {lens}", flush=True)
        kn, vn = kv_rows(rng, ns, cfg)
        xr = rng.standard_normal((ns, 128)).astype(np.float32)
        q = rng.standard_normal((ns, 24, 256)).astype(np.float32)
        qi = qi_all[step]
        if mode == "newest" and step == 0:         # the completing row, aligned too
            xr[:, :64] *= 0.01
            xr[:, 64:] = 0.01 * xr[:, 64:] + qi[:, :, 64:].sum(1)
        L = torch.tensor(lens, dtype=torch.int32, device="cuda")
        sel = torch.full((ns, 2, msel), -7, dtype=torch.int32, device="cuda")
        nsel = torch.empty((ns, 2), dtype=torch.int32, device="cuda")
        qd, qid = torch.from_numpy(q).cuda(), torch.from_numpy(qi).cuda()
        knd, vnd, xrd = (torch.from_numpy(a).cuda() for a in (kn, vn, xr))
        out = qsa.idx_sparse_attn_decode(ic, qd, qid, knd, vnd, xrd, L, Lmax, ws, sel=sel, n_sel=nsel)
        pos = L - 1
        qsa.append_q8_0(dev2, knd, vnd, pos, seq_ids=torch.arange(ns, dtype=torch.int32, device="cuda"))
        qsa.idx_append_pool(ic2, xrd, pos, seq_ids=torch.arange(ns, dtype=torch.int32, device="cuda"))
        sel2 = torch.full_like(sel, -7)
        nsel2 = torch.empty_like(nsel)
        qsa.idx_select(ic2, qid, L, Lmax, ws2, sel=sel2, n_sel=nsel2)
        out2 = qsa.sparse_decode_attn(dev2, qd, L, Lmax, ws2, sel=sel2, n_sel=nsel2)
        torch.cuda.synchronize()
        assert host.append(kn, vn, np.array([l - 1 for l in lens], np.int32), np.arange(ns, dtype=np.int32)) == 0
        hs = np.full((ns, 2, msel), -1, np.int32)
        gs, gn = np_of(sel), np_of(nsel)
        pooled = np_of(ic.pooled)
        for s in range(ns):
            want = oracle_select(cfg, ICFG, pooled[s], qi[s], lens[s], msel)
            assert len(want) == 513
            if mode == "cluster" and step == 0:
                assert set(range(2000, 2200)) <= set(want.tolist())
            if mode == "newest" and step == 0:
                assert lens[s] % 4 == 0 and (lens[s] - 1) // 4 in want.tolist()
            for g in range(2):
                assert gn[s, g] == len(want)
                np.testing.assert_array_equal(gs[s, g, :gn[s, g]], want, err_msg=f"step {step} seq {s} head {g}")
                hs[s, g, :len(want)] = want
        ref = host.attention_f64(q, lens, hs, gn)
        assert_close_attn(np_of(out), ref, f"step {step}")
        assert torch.equal(sel, sel2) and torch.equal(nsel, nsel2), f"step {step}: selections differ"
        assert torch.equal(out, out2), f"step {step}: outputs differ from the four calls'"
    assert qsa.read_status(dev) == 0


def test_per_head_selection_long_context():
    """A per-KV-head selection (no shared selection) over 10,000 4-token blocks:
    k_select_big with one workgroup per (sequence, KV head)."""
    from _gpu import fill
    from _refs import Cfg
    cfg = Cfg(n_head=24, n_head_kv=2, head_dim=256, block_tokens=4, page_tokens=256, top_k_blocks=300,
              sink_blocks=1, local_tokens=16)
    rng = np.random.default_rng(860)
    L = 40004
    dev, host = make_pair(cfg, 1, L // 256 + 1, seed=861)
    fill(dev, host, rng, [L])
    q = rng.standard_normal((1, 24, 256)).astype(np.float32)
    c = cfg_of(cfg)
    ws = qsa.Workspace(c, 1, L)
    sel, nsel = qsa.indexer_topk(dev, torch.from_numpy(q).cuda(), torch.tensor([L], dtype=torch.int32,
                                                                                 device="cuda"), L, ws)
    torch.cuda.synchronize()
    hs, hn = host.indexer_topk(q, [L], max_sel=sel.shape[-1])
    gs, gn = np_of(sel), np_of(nsel)
    np.testing.assert_array_equal(gn, hn)
    for g in range(2):
        np.testing.assert_array_equal(gs[0, g, :gn[0, g]], hs[0, g, :hn[0, g]], err_msg=f"head {g}")
    assert qsa.read_status(dev) == 0


def _long_prefill(seed, raw_keys=None):
    """A 37-query chunk appended at 36,001 (over 9,000 eligible 4-token blocks
    a query): selections bit for bit against the oracle's on the pooled keys
    the device built, every ninth query's attention within tolerance.
    raw_keys(rng, n, t0) gives the indexer's raw keys of tokens t0 .. t0+n-1."""
    cfg = CKPT
    rng = np.random.default_rng(seed)
    pre, n_q = 36001, 37
    end = pre + n_q
    pps = end // cfg.page_tokens + 1
    dev, host, ic, w = _pair(cfg, 1, pps, seed=seed + 1)
    raw = raw_keys or (lambda r, n, t0: r.standard_normal((n, 128)).astype(np.float32))
    kr0 = raw(rng, pre, 0)
    qsa.idx_append_pool(ic, torch.from_numpy(kr0).cuda(), torch.arange(pre, dtype=torch.int32, device="cuda"))
    k, v = kv_rows(rng, pre, cfg)
    host.append(k, v, np.arange(pre, dtype=np.int32))
    qsa.append_q8_0(dev, torch.from_numpy(k).cuda(), torch.from_numpy(v).cuda(),
                    torch.arange(pre, dtype=torch.int32, device="cuda"))
    kn, vn = kv_rows(rng, n_q, cfg)
    krn = raw(rng, n_q, pre)
    q = rng.standard_normal((n_q, 24, 256)).astype(np.float32)
    qi = rng.standard_normal((n_q, 4, 128)).astype(np.float32)
    c = cfg_of(cfg)
    msel = c.max_selected(end)
    sel = torch.empty((n_q, 2, msel), dtype=torch.int32, device="cuda")
    nsel = torch.empty((n_q, 2), dtype=torch.int32, device="cuda")
    ws = qsa.Workspace.for_prefill(c, end, n_q)
    out = qsa.idx_sparse_attn_prefill(ic, torch.from_numpy(q).cuda(), torch.from_numpy(qi).cuda(), 0, pre, ws,
                                      k_new=torch.from_numpy(kn).cuda(), v_new=torch.from_numpy(vn).cuda(),
                                      k_raw=torch.from_numpy(krn).cuda(), sel=sel, n_sel=nsel)
    torch.cuda.synchronize()
    assert qsa.read_status(dev) == 0
    host.append(kn, vn, np.arange(pre, end, dtype=np.int32))
    pooled = np_of(ic.pooled)[0]
    gs, gn, o = np_of(sel), np_of(nsel), np_of(out)
    for i in range(n_q):
        want = oracle_select(cfg, ICFG, pooled, qi[i], pre + i + 1, msel)
        assert len(want) == 513
        for g in range(2):
            np.testing.assert_array_equal(gs[i, g, :gn[i, g]], want, err_msg=f"query {i} head {g}")
        if i % 9 == 0:
            ref = host.attention_f64(q[i:i + 1], [pre + i + 1], gs[i:i + 1], gn[i:i + 1])
            assert_close_attn(o[i:i + 1], ref, f"query {i}")
    return pooled


def test_checkpoint_prefill_long_context():
    """Prefill queries at positions past 32,768 (over 8192 eligible blocks
    each): the bounded scoring and the 1024-thread refinement of one shared row."""
    _long_prefill(870)


def _class_keys(classes):
    """Raw indexer keys whose pooled blocks take one of a few values: the
    rotated dims zero (so the position does not enter), the rest the block's
    class vector; classes[b] is block b's class (4-token blocks)."""
    vecs = np.random.default_rng(77).standard_normal((int(classes.max()) + 1, 128)).astype(np.float32)
    vecs[:, :64] = 0.0

    def raw(rng, n, t0):
        b = (np.arange(t0, t0 + n) // 4).clip(max=len(classes) - 1)
        return vecs[classes[b]].copy()
    return raw


def test_checkpoint_prefill_long_context_all_keys_equal():
    """Every pooled block the same: every score ties, far more candidates than
    the refinement holds, so it scores the whole row exactly and selects the
    lowest-indexed blocks."""
    pooled = _long_prefill(880, _class_keys(np.zeros(9100, dtype=np.int64)))
    assert (pooled[1:9000] == pooled[0]).all()


def test_checkpoint_prefill_long_context_three_key_values():
    """Pooled blocks of three values (300, 400 and the rest of the blocks):
    whole classes tie, so the selection's threshold falls inside a class of
    equal scores and its blocks are taken by index, with the refinement's own
    candidates where the two small classes lead, the exact row where not."""
    cls = np.full(9100, 2, dtype=np.int64)
    perm = np.random.default_rng(78).permutation(9000)
    cls[perm[:300]] = 0
    cls[perm[300:700]] = 1
    _long_prefill(890, _class_keys(cls))
