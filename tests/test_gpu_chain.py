"""qwfn_sparse_attn_decode_chain: n_pos chained decode positions in one call,
the multi-position decode of the reference's MTP verify step
(src/qwfn_engine.cpp:1892-1906: T sparse_attn_decode calls in one graph, each
reading through the writes of the ones before).

* Against the oracle: position k of every sequence appends its row at
  seq_len - 1 + k, pools the block it completes and selects and attends with
  length seq_len + k.  Selections, cache bytes and pooled keys bit-exact,
  attention within |o - o_ref| <= 2e-3 + 1e-3 |o_ref|.
* Against n_pos single qwfn_sparse_attn_decode calls on a copy of the same
  cache: outputs, selections and caches bit-identical.
* Captured in one hipGraph: every replay (with eager work between) equals the
  eager chain.
"""
import numpy as np
import pytest
import torch

from _gpu import assert_close_attn, cfg_of, fill, kv_rows, make_pair, np_of
from _refs import BASELINE, Cfg
from qwfnfer_amd import qsa

pytestmark = pytest.mark.gpu

# the checkpoint's bias rule at BASELINE head shapes: a block completed by a
# position is eligible at that position, so it is pooled before it is scored
CKPT_RULE = Cfg(sink_blocks=0, local_tokens=0, topk_counts_forced=1, relu_per_head=1)


def _chain_inputs(rng, cfg, n_pos, n_seq):
    q = rng.standard_normal((n_pos, n_seq, cfg.n_head, cfg.head_dim), dtype=np.float32)
    kn = np.empty((n_pos, n_seq, cfg.n_head_kv, cfg.head_dim), np.float32)
    vn = np.empty_like(kn)
    for k in range(n_pos):
        kn[k], vn[k] = kv_rows(rng, n_seq, cfg)
    return q, kn, vn


def _setup(cfg, lengths, n_pos, seed):
    rng = np.random.default_rng(seed)
    n_seq = len(lengths)
    pps = (max(lengths) + n_pos) // cfg.page_tokens + 1
    dev, host = make_pair(cfg, n_seq, pps, seed=seed)
    fill(dev, host, rng, lengths)
    q, kn, vn = _chain_inputs(rng, cfg, n_pos, n_seq)
    return rng, dev, host, q, kn, vn


@pytest.mark.parametrize("cfg,lengths,n_pos", [
    (BASELINE, [64 * 300 - 2, 5000], 3),            # sequence 0 completes block 299 at position 1
    (BASELINE, [163840 - 1], 2),                     # the headline context, completing block 2559
    (CKPT_RULE, [64 * 200 - 1, 64 * 90 - 2], 4),     # completed blocks eligible at once
])
def test_chain_matches_oracle(cfg, lengths, n_pos):
    print(f"chain vs oracle: lengths {lengths}, n_pos {n_pos}, local {cfg.local_tokens}", flush=True)
    rng, dev, host, q, kn, vn = _setup(cfg, lengths, n_pos, seed=911 + n_pos)
    n_seq = len(lengths)
    c = cfg_of(cfg)
    cur = np.array(lengths, np.int32) + 1                 # the first position's lengths
    max_len = int(cur.max()) + n_pos - 1
    ws = qsa.Workspace(c, n_seq, max_len)
    msel = c.max_selected(max_len)
    sel = torch.empty((n_pos, n_seq, cfg.n_head_kv, msel), dtype=torch.int32, device="cuda")
    nsel = torch.empty((n_pos, n_seq, cfg.n_head_kv), dtype=torch.int32, device="cuda")
    out = qsa.sparse_attn_decode_chain(dev, torch.from_numpy(q).cuda(), torch.from_numpy(kn).cuda(),
                                       torch.from_numpy(vn).cuda(), torch.from_numpy(cur).cuda(), max_len, ws,
                                       sel=sel, n_sel=nsel)
    torch.cuda.synchronize()
    gs, gn, go = np_of(sel), np_of(nsel), np_of(out)
    for k in range(n_pos):
        ck = cur + k
        for s in range(n_seq):
            p = int(ck[s]) - 1
            assert host.append(kn[k, s:s + 1], vn[k, s:s + 1], [p], [s]) == 0
            if ck[s] % cfg.block_tokens == 0:
                host.pool_block(s, p // cfg.block_tokens)
        hs, hn = host.indexer_topk(q[k], ck, max_sel=msel)
        np.testing.assert_array_equal(gn[k], hn, err_msg=f"position {k}")
        for s in range(n_seq):
            for g in range(cfg.n_head_kv):
                np.testing.assert_array_equal(gs[k, s, g, :gn[k, s, g]], hs[s, g, :hn[s, g]],
                                              err_msg=f"position {k} seq {s} head {g}")
        assert_close_attn(go[k], host.attention_f64(q[k], ck, hs, hn), f"chain position {k}")
    assert qsa.read_status(dev) == 0
    np.testing.assert_array_equal(np_of(dev.k_pages), host.k_pages)
    np.testing.assert_array_equal(np_of(dev.v_pages), host.v_pages)
    end = cur + n_pos - 1
    for s in range(n_seq):
        nw = int(end[s]) // cfg.block_tokens
        np.testing.assert_array_equal(np_of(dev.pooled)[s, :, :nw], host.pooled[s, :, :nw])


def _clone(dev):
    c = qsa.KvCache.allocate(dev.cfg, dev.n_seq, dev.pages_per_seq, page_table=dev.page_table.cpu(),
                             n_phys_pages=dev.n_phys_pages)
    for name in ("k_pages", "v_pages", "pooled"):
        getattr(c, name).copy_(getattr(dev, name))
    return c


def test_chain_equals_single_calls():
    cfg = BASELINE
    lengths = [64 * 700 - 3, 20000, 7000]
    n_pos = 4
    print(f"chain vs single calls: lengths {lengths}, n_pos {n_pos}", flush=True)
    _, dev, _, q, kn, vn = _setup(cfg, lengths, n_pos, seed=77)
    twin = _clone(dev)
    n_seq = len(lengths)
    c = cfg_of(cfg)
    cur = torch.tensor(lengths, dtype=torch.int32, device="cuda") + 1
    max_len = int(cur.max()) + n_pos - 1
    ws = qsa.Workspace(c, n_seq, max_len)
    msel = c.max_selected(max_len)
    qd, knd, vnd = torch.from_numpy(q).cuda(), torch.from_numpy(kn).cuda(), torch.from_numpy(vn).cuda()
    sel = torch.empty((n_pos, n_seq, cfg.n_head_kv, msel), dtype=torch.int32, device="cuda")
    nsel = torch.empty((n_pos, n_seq, cfg.n_head_kv), dtype=torch.int32, device="cuda")
    out = qsa.sparse_attn_decode_chain(dev, qd, knd, vnd, cur, max_len, ws, sel=sel, n_sel=nsel)
    ws1 = qsa.Workspace(c, n_seq, max_len)
    for k in range(n_pos):
        s1 = torch.empty((n_seq, cfg.n_head_kv, msel), dtype=torch.int32, device="cuda")
        n1 = torch.empty((n_seq, cfg.n_head_kv), dtype=torch.int32, device="cuda")
        o1 = qsa.sparse_attn_decode(twin, qd[k].contiguous(), knd[k].contiguous(), vnd[k].contiguous(),
                                    (cur + k).contiguous(), max_len, ws1, sel=s1, n_sel=n1)
        torch.cuda.synchronize()
        assert torch.equal(o1, out[k]), f"position {k}: outputs differ"
        assert torch.equal(n1, nsel[k]), f"position {k}: counts differ"
        for s in range(n_seq):
            for g in range(cfg.n_head_kv):
                m = int(n1[s, g])
                assert torch.equal(s1[s, g, :m], sel[k, s, g, :m]), f"position {k} seq {s} head {g}"
    for name in ("k_pages", "v_pages", "pooled"):
        assert torch.equal(getattr(dev, name), getattr(twin, name)), name


def test_chain_in_one_hipgraph():
    cfg = BASELINE
    lengths = [64 * 400 - 1, 12345]
    n_pos = 3
    print(f"chain in a hipGraph: lengths {lengths}, n_pos {n_pos}", flush=True)
    _, dev, _, q, kn, vn = _setup(cfg, lengths, n_pos, seed=5)
    n_seq = len(lengths)
    c = cfg_of(cfg)
    cur = torch.tensor(lengths, dtype=torch.int32, device="cuda") + 1
    max_len = int(cur.max()) + n_pos - 1
    ws = qsa.Workspace(c, n_seq, max_len)
    qd, knd, vnd = torch.from_numpy(q).cuda(), torch.from_numpy(kn).cuda(), torch.from_numpy(vn).cuda()
    out = torch.empty((n_pos, n_seq, cfg.n_head, cfg.head_dim), dtype=torch.float32, device="cuda")
    qsa.sparse_attn_decode_chain(dev, qd, knd, vnd, cur, max_len, ws, out=out)   # eager: writes the rows
    torch.cuda.synchronize()
    ref = out.clone()
    st = torch.cuda.Stream()
    st.wait_stream(torch.cuda.current_stream())
    g = torch.cuda.CUDAGraph()
    with torch.cuda.stream(st):
        with torch.cuda.graph(g, stream=st):
            qsa.sparse_attn_decode_chain(dev, qd, knd, vnd, cur, max_len, ws, out=out, stream=st)
    torch.cuda.current_stream().wait_stream(st)
    torch.cuda.synchronize()
    for rep in range(3):
        out.fill_(float("nan"))
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, ref), f"replay {rep} differs from the eager chain"
        # eager work between replays: the same chain again (it rewrites the same rows)
        o2 = qsa.sparse_attn_decode_chain(dev, qd, knd, vnd, cur, max_len, ws)
        torch.cuda.synchronize()
        assert torch.equal(o2, ref)
    assert qsa.read_status(dev) == 0
