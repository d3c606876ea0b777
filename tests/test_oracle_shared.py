"""Shared selection (one selection for every KV head): the oracle's indexer
against its definition -- each KV head's block score (pinned exactly by
block_score_exact), summed over the heads in head order in float32, then the
selection from its definition (select_ref), copied to every head."""
import numpy as np
import pytest

from oracle import oracle as O
from _refs import TINY, Cfg, block_score_exact, select_ref


def _host(cfg, L, seed):
    rng = np.random.default_rng(seed)
    pps = L // cfg.page_tokens + 1
    host = O.HostCache(cfg, 1, pps)
    k = rng.standard_normal((L, cfg.n_head_kv, cfg.head_dim), dtype=np.float32)
    assert host.append(k, k, np.arange(L, dtype=np.int32)) == 0
    for b in range(L // cfg.block_tokens):
        assert host.pool_block(0, b) == 0
    return host, rng


@pytest.mark.parametrize("relu", [0, 1])
@pytest.mark.parametrize("L", [37, 130, 200])
def test_shared_selection_sums_the_heads_in_order(relu, L):
    cfg = Cfg(**{**TINY.__dict__, "shared_selection": 1, "relu_per_head": relu})
    host, rng = _host(cfg, 200, seed=600 + L + relu)
    q = rng.standard_normal((1, cfg.n_head, cfg.head_dim), dtype=np.float32)
    sel, nsel = host.indexer_topk(q, np.array([L], np.int32))
    G = cfg.group
    nb = L // cfg.block_tokens
    total = np.zeros(nb, np.float32)
    for g in range(cfg.n_head_kv):
        s_g = np.array([block_score_exact(q[0, g * G:(g + 1) * G], host.pooled[0, g, b], bool(relu))
                        for b in range(nb)], np.float32)
        total = s_g if g == 0 else (total + s_g).astype(np.float32)
    want = select_ref(cfg, total, L)
    for g in range(cfg.n_head_kv):
        assert nsel[0, g] == len(want)
        np.testing.assert_array_equal(sel[0, g, :nsel[0, g]], want)


def test_one_kv_head_shared_is_the_plain_selection():
    base = Cfg(n_head=4, n_head_kv=1, head_dim=64, block_tokens=4, page_tokens=64, top_k_blocks=3,
               sink_blocks=1, local_tokens=9)
    shared = Cfg(**{**base.__dict__, "shared_selection": 1})
    ha, rng = _host(base, 150, seed=610)
    hb, _ = _host(shared, 150, seed=610)
    q = rng.standard_normal((1, 4, 64), dtype=np.float32)
    for L in (50, 150):
        sa, na = ha.indexer_topk(q, np.array([L], np.int32))
        sb, nb = hb.indexer_topk(q, np.array([L], np.int32))
        assert na[0, 0] == nb[0, 0]
        np.testing.assert_array_equal(sa[0, 0, :na[0, 0]], sb[0, 0, :nb[0, 0]])
