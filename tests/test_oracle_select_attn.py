"""The oracle's block score (exact rational fmaf), selection (brute-force sort
and special cases) and fp64 attention (numpy textbook softmax, closed forms)."""
import numpy as np
import pytest

from _refs import BASELINE, TINY, Cfg, attention_ref, block_score_exact, select_ref


@pytest.mark.parametrize("cfg,relu", [(TINY, 0), (TINY, 1), (BASELINE, 0)])
def test_block_score_exact_order(oracle, cfg, relu):
    cfg = Cfg(**{**cfg.__dict__, "relu_per_head": relu})
    rng = np.random.default_rng(20 + relu)
    for trial in range(6 if cfg is not TINY else 20):
        qg = rng.standard_normal((cfg.group, cfg.head_dim)).astype(np.float32)
        p = (rng.standard_normal(cfg.head_dim) * 0.125).astype(np.float32)
        got = oracle.block_score(cfg, qg, p)
        ref = block_score_exact(qg, p, bool(relu))
        assert np.float32(got).view(np.uint32) == np.float32(ref).view(np.uint32), (trial, got, ref)


def test_block_score_order_is_observable(oracle):
    """A plain sequential dot gives different bits on some inputs, so the exact
    check above would catch an order mistake."""
    cfg = BASELINE
    rng = np.random.default_rng(22)
    differ = 0
    for _ in range(20):
        qg = rng.standard_normal((cfg.group, cfg.head_dim)).astype(np.float32)
        p = rng.standard_normal(cfg.head_dim).astype(np.float32)
        seq = np.float32(0)
        for h in range(cfg.group):
            acc = np.float32(0)
            for d in range(cfg.head_dim):
                acc = np.float32(acc + np.float32(qg[h, d] * p[d]))
            seq = np.float32(seq + acc)
        differ += np.float32(oracle.block_score(cfg, qg, p)) != seq
    assert differ > 0


@pytest.mark.parametrize("cfg", [BASELINE, TINY, Cfg(top_k_blocks=3, sink_blocks=2, local_tokens=100)])
def test_select_matches_bruteforce(oracle, cfg):
    rng = np.random.default_rng(23)
    bt = cfg.block_tokens
    for seq_len in list(range(1, 3 * bt + 3)) + list(rng.integers(1, 200 * bt, 300)):
        seq_len = int(seq_len)
        nb = seq_len // bt + 1
        scores = rng.standard_normal(nb).astype(np.float32)
        scores[rng.random(nb) < 0.2] = 0.5          # ties
        got = oracle.select(cfg, scores, seq_len)
        np.testing.assert_array_equal(got, select_ref(cfg, scores, seq_len), err_msg=f"L={seq_len}")
        assert len(got) <= oracle.max_selected(cfg, seq_len)


def test_select_special_cases(oracle):
    cfg = BASELINE
    # config 2: ctx 32768 -> 73 blocks, forced {0} U 504..511
    L = 32768
    sc = np.random.default_rng(24).standard_normal(L // 64).astype(np.float32)
    s = oracle.select(cfg, sc, L)
    assert len(s) == 73 and s[0] == 0 and list(s[-8:]) == list(range(504, 512))
    # 4096: every block (|E| = 55 <= 64), dense-equivalent
    assert list(oracle.select(cfg, sc, 4096)) == list(range(64))
    # all-equal scores: the lowest eligible indices win
    eq = np.zeros(L // 64, np.float32)
    assert list(oracle.select(cfg, eq, L)) == [0] + list(range(1, 65)) + list(range(504, 512))
    # -inf / NaN blocks never beat finite ones
    bad = sc.copy()
    bad[1:200] = -np.inf
    bad[200:300] = np.nan
    s = oracle.select(cfg, bad, L)
    assert not set(range(1, 300)) & set(s)
    # dense mode
    assert list(oracle.select(cfg.__class__(**{**cfg.__dict__, "top_k_blocks": 0}), sc, 1000)) == list(range(16))


def test_indexer_topk_end_to_end_small(oracle):
    cfg = TINY
    rng = np.random.default_rng(25)
    c = oracle.HostCache(cfg, 2, 4)
    n = c.capacity
    k = rng.standard_normal((n, cfg.n_head_kv, cfg.head_dim)).astype(np.float32)
    for s in range(2):
        c.append(k, k, np.arange(n, dtype=np.int32), np.full(n, s, np.int32))
        for b in range(n // cfg.block_tokens):
            c.pool_block(s, b)
    q = rng.standard_normal((2, cfg.n_head, cfg.head_dim)).astype(np.float32)
    seq_len = np.array([n, 101], np.int32)
    sel, nsel = c.indexer_topk(q, seq_len)
    for s in range(2):
        for g in range(cfg.n_head_kv):
            nb = seq_len[s] // cfg.block_tokens
            scores = np.zeros(nb + 1, np.float32)
            for b in range(nb):
                scores[b] = block_score_exact(q[s, g * cfg.group:(g + 1) * cfg.group], c.pooled[s, g, b], False)
            ref = select_ref(cfg, scores, int(seq_len[s]))
            np.testing.assert_array_equal(sel[s, g, :nsel[s, g]], ref)


def test_attention_f64_matches_textbook(oracle):
    cfg = TINY
    rng = np.random.default_rng(26)
    c = oracle.HostCache(cfg, 1, 2)
    n = 100
    k = rng.standard_normal((n, 2, cfg.head_dim)).astype(np.float32)
    v = rng.standard_normal((n, 2, cfg.head_dim)).astype(np.float32)
    c.append(k, v, np.arange(n, dtype=np.int32))
    q = rng.standard_normal((1, cfg.n_head, cfg.head_dim)).astype(np.float32)
    sel = np.array([[[0, 3, 7, 24, -1], [1, 2, 23, 24, -1]]], np.int32)
    nsel = np.array([[4, 4]], np.int32)
    L = 98                                             # block 24 is partial: cells 96, 97
    out = c.attention_f64(q, [L], sel, nsel)
    for h in range(cfg.n_head):
        g = h // cfg.group
        cells = [t for b in sel[0, g, :4] for t in range(4 * b, 4 * b + 4) if t < L]
        K = np.stack([c.dequant_row("k", 0, t, g) for t in cells])
        V = np.stack([c.dequant_row("v", 0, t, g) for t in cells])
        np.testing.assert_allclose(out[0, h], attention_ref(q[0, h], K, V), rtol=1e-12, atol=1e-13)


def test_attention_f64_kv_round_f16(oracle):
    """kv_round_f16: the oracle's attention runs on every dequantized K and V
    value rounded to fp16 (numpy's float16 conversion, round to nearest even,
    as the reference's F16 cast of its gathered rows); the prefill oracle
    ignores the flag."""
    base = Cfg(**{**TINY.__dict__, "kv_round_f16": 0})
    cfg = Cfg(**{**TINY.__dict__, "kv_round_f16": 1})
    rng = np.random.default_rng(29)
    n = 100
    k = (rng.standard_normal((n, 2, cfg.head_dim)) * 3.7).astype(np.float32)
    v = (rng.standard_normal((n, 2, cfg.head_dim)) * 3.7).astype(np.float32)
    caches = []
    for c_ in (base, cfg):
        c = oracle.HostCache(c_, 1, 2)
        c.append(k, v, np.arange(n, dtype=np.int32))
        caches.append(c)
    q = rng.standard_normal((1, cfg.n_head, cfg.head_dim)).astype(np.float32)
    L = 99
    exact = caches[0].attention_f64(q, [L])
    out = caches[1].attention_f64(q, [L])
    c = caches[1]
    for h in range(cfg.n_head):
        g = h // cfg.group
        K = np.stack([c.dequant_row("k", 0, t, g) for t in range(L)]).astype(np.float16).astype(np.float32)
        V = np.stack([c.dequant_row("v", 0, t, g) for t in range(L)]).astype(np.float16).astype(np.float32)
        np.testing.assert_allclose(out[0, h], attention_ref(q[0, h], K, V), rtol=1e-12, atol=1e-13)
    assert np.abs(out - exact).max() > 0                 # the rounding is visible at these values
    pf = [c_.prefill_f64(q, 0, L - 1)[-1] for c_ in caches]
    np.testing.assert_array_equal(pf[0], pf[1])


def test_attention_closed_forms(oracle):
    cfg = TINY
    c = oracle.HostCache(cfg, 1, 1)
    rng = np.random.default_rng(27)
    v = rng.standard_normal((8, 2, cfg.head_dim)).astype(np.float32)
    k = np.zeros((8, 2, cfg.head_dim), np.float32)   # identical keys -> mean of V
    c.append(k, v, np.arange(8, dtype=np.int32))
    q = rng.standard_normal((1, cfg.n_head, cfg.head_dim)).astype(np.float32)
    out = c.attention_f64(q, [8])
    for h in range(cfg.n_head):
        V = np.stack([c.dequant_row("v", 0, t, h // cfg.group) for t in range(8)])
        np.testing.assert_allclose(out[0, h], V.mean(0), rtol=1e-12, atol=1e-14)
    # one key -> its V row
    out1 = c.attention_f64(q, [1])
    np.testing.assert_allclose(out1[0, 0], c.dequant_row("v", 0, 0, 0), rtol=0, atol=0)
    # a dominant logit -> that V row
    k2 = np.zeros((8, 2, cfg.head_dim), np.float32)
    k2[5] = 100.0 * np.sign(q[0, 0])[None, :]
    c.append(k2, v, np.arange(8, dtype=np.int32))
    out2 = c.attention_f64(q, [8])
    np.testing.assert_allclose(out2[0, 0], c.dequant_row("v", 0, 5, 0), rtol=1e-9, atol=1e-9)
