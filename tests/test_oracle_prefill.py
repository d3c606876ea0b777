"""The oracle's prefill (per-query selection and fp64 attention) against a
brute-force restatement of the per-query causal rule: scores of every whole
block by the (separately pinned) block score, the selection from its
definition, and textbook softmax over the selected cells at or before the
query's position."""
import numpy as np
import pytest

from oracle import oracle as O
from _refs import BASELINE, TINY, Cfg, attention_ref, select_ref


def _filled(cfg, lengths, seed, seq_perm=True):
    rng = np.random.default_rng(seed)
    pps = max(lengths) // cfg.page_tokens + 1
    n_phys = len(lengths) * pps
    pt = np.random.default_rng(seed).permutation(n_phys).astype(np.int32).reshape(len(lengths), pps)
    host = O.HostCache(cfg, len(lengths), pps, page_table=pt, n_phys_pages=n_phys)
    for s, L in enumerate(lengths):
        k = rng.standard_normal((L, cfg.n_head_kv, cfg.head_dim), dtype=np.float32)
        v = rng.standard_normal((L, cfg.n_head_kv, cfg.head_dim), dtype=np.float32)
        assert host.append(k, v, np.arange(L, dtype=np.int32), np.full(L, s, np.int32)) == 0
        for b in range(L // cfg.block_tokens):
            assert host.pool_block(s, b) == 0
    return host, rng


@pytest.mark.parametrize("cfg,lengths,seq,pos0,n_q", [
    (TINY, [40, 150], 1, 112, 38),        # crosses blocks, window and eligible set grow
    (TINY, [90, 30], 0, 0, 40),           # from the first token: sink and window overlap
    (Cfg(n_head=8, n_head_kv=1, head_dim=64, block_tokens=8, page_tokens=64, top_k_blocks=3,
         sink_blocks=2, local_tokens=20), [300], 0, 230, 40),
])
def test_prefill_oracle_matches_brute_force(cfg, lengths, seq, pos0, n_q):
    host, rng = _filled(cfg, lengths, seed=500 + pos0)
    q = rng.standard_normal((n_q, cfg.n_head, cfg.head_dim), dtype=np.float32)
    sel, nsel, out = host.prefill_f64(q, seq, pos0)
    G = cfg.n_head // cfg.n_head_kv
    bt = cfg.block_tokens
    for i in range(n_q):
        p = pos0 + i
        L = p + 1
        for g in range(cfg.n_head_kv):
            scores = np.full(L // bt + 1, np.nan, dtype=np.float32)
            for b in range(L // bt):
                scores[b] = O.block_score(cfg, q[i, g * G:(g + 1) * G], host.pooled[seq, g, b])
            want = select_ref(cfg, scores, L)
            got = sel[i, g, :nsel[i, g]]
            np.testing.assert_array_equal(got, want, err_msg=f"query {i} head {g}")
            cells = [t for b in want for t in range(b * bt, min((b + 1) * bt, L))]
            K = np.stack([host.dequant_row("k", seq, t, g) for t in cells])
            V = np.stack([host.dequant_row("v", seq, t, g) for t in cells])
            for h in range(g * G, (g + 1) * G):
                ref = attention_ref(q[i, h], K, V)
                np.testing.assert_allclose(out[i, h], ref, rtol=1e-9, atol=1e-12,
                                           err_msg=f"query {i} head {h}")


def test_prefill_oracle_is_the_decode_rule_per_query():
    # one query of a prefill = a decode indexer + attention at seq_len = p + 1
    cfg = BASELINE
    host, rng = _filled(cfg, [7000], seed=520)
    q = rng.standard_normal((5, cfg.n_head, cfg.head_dim), dtype=np.float32)
    sel, nsel, out = host.prefill_f64(q, 0, 6900)
    for i in range(5):
        L = np.array([6900 + i + 1], np.int32)
        hs, hn = host.indexer_topk(q[i:i + 1], L, max_sel=sel.shape[-1])
        np.testing.assert_array_equal(hs[0], sel[i])
        np.testing.assert_array_equal(hn[0], nsel[i])
        np.testing.assert_array_equal(host.attention_f64(q[i:i + 1], L, hs, hn)[0], out[i])
