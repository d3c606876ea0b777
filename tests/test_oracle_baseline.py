"""The CPU baseline bench.py times (qwfn_oracle_decode_step_f32) against the
checkers.  The step appends the decode token and pools the block it
completes.  On the cache it leaves, its selection equals
qwfn_oracle_indexer_topk's bit for bit, and its output is within the attention
tolerance of qwfn_oracle_attention_f64 over that selection.  Its K/V are cast
to fp16 like the reference's decode; the fp64 checker dequantizes exactly."""
import numpy as np
import pytest

from _refs import BASELINE, TINY, Cfg

ATOL, RTOL = 2e-3, 1e-3


def _filled(oracle, cfg, lengths, pages, rng):
    c = oracle.HostCache(cfg, len(lengths), pages)
    for s, L in enumerate(lengths):
        k = rng.standard_normal((L, cfg.n_head_kv, cfg.head_dim)).astype(np.float32)
        v = rng.standard_normal((L, cfg.n_head_kv, cfg.head_dim)).astype(np.float32)
        c.append(k, v, np.arange(L, dtype=np.int32), np.full(L, s, np.int32))
        for b in range(L // cfg.block_tokens):
            c.pool_block(s, b)
    return c


@pytest.mark.parametrize("cfg,lengths,pages", [
    # a top-64 selection; the step that completes block 63 (4095 -> 4096); every block
    (BASELINE, [20031, 4095, 2600], 80),
    (TINY, [57, 200, 3], 4),
    (Cfg(top_k_blocks=0), [1500, 64], 8),           # dense
])
def test_baseline_step_matches_the_checkers(oracle, cfg, lengths, pages):
    rng = np.random.default_rng(31)
    c = _filled(oracle, cfg, lengths, pages, rng)
    n = len(lengths)
    q = rng.standard_normal((n, cfg.n_head, cfg.head_dim)).astype(np.float32)
    kn = rng.standard_normal((n, cfg.n_head_kv, cfg.head_dim)).astype(np.float32)
    vn = rng.standard_normal((n, cfg.n_head_kv, cfg.head_dim)).astype(np.float32)
    seq_len = np.array([L + 1 for L in lengths], np.int32)
    out, sel, nsel, threads = c.decode_step_f32(q, kn, vn, seq_len)
    assert threads >= 1
    # the decode token is in the cache, and a block it completes is pooled
    for s in range(n):
        for g in range(cfg.n_head_kv):
            assert np.allclose(c.dequant_row("k", s, lengths[s], g), kn[s, g], rtol=0.02, atol=0.02)
    sel_ref, nsel_ref = c.indexer_topk(q, seq_len, max_sel=sel.shape[-1])
    np.testing.assert_array_equal(nsel, nsel_ref)
    for s in range(n):
        for g in range(cfg.n_head_kv):
            np.testing.assert_array_equal(sel[s, g, :nsel[s, g]], sel_ref[s, g, :nsel_ref[s, g]])
    ref = c.attention_f64(q, seq_len, sel_ref, nsel_ref)
    np.testing.assert_allclose(out, ref, atol=ATOL, rtol=RTOL)


def test_baseline_step_sees_a_planted_key(oracle):
    """One key row made to dominate its block's pooled key and the query: the
    baseline must select that block and put nearly all the weight on its V
    row (a dropped head, a wrong group or a transposed operand would not)."""
    cfg = BASELINE
    rng = np.random.default_rng(32)
    L = 9000
    c = _filled(oracle, cfg, [L], 40, rng)
    q = np.zeros((1, cfg.n_head, cfg.head_dim), np.float32)
    q[0, 8:16, :] = 0.3                              # KV head 1's query heads
    t = 64 * 40 + 5                                  # block 40, far from the forced blocks
    k = np.zeros((1, cfg.n_head_kv, cfg.head_dim), np.float32)
    v = np.zeros((1, cfg.n_head_kv, cfg.head_dim), np.float32)
    k[0, 1, :] = 8.0
    v[0, 1, :] = np.linspace(-1, 1, cfg.head_dim)
    c.append(k, v, np.array([t], np.int32), np.array([0], np.int32))
    c.pool_block(0, 40)
    kn = rng.standard_normal((1, cfg.n_head_kv, cfg.head_dim)).astype(np.float32) * 0.01
    out, sel, nsel, _ = c.decode_step_f32(q, kn, kn, np.array([L + 1], np.int32))
    assert 40 in sel[0, 1, :nsel[0, 1]]
    np.testing.assert_allclose(out[0, 8:16], np.tile(v[0, 1], (8, 1)), atol=0.02)
