"""The checkpoint's selection rule (local_tokens = 0, topk_counts_forced = 1)
against the reference's own formulation of it: a bias vector over the blocks --
0 for every whole block, 1e9 for an incomplete tail block, -inf past it
(src/qwfn_engine.cpp:748-753; prefill rows :936-950) -- added to the scores,
then the top k_blocks entries of the biased vector (ggml_top_k,
src/qwfn_graph.cpp:493), ties to the lower block index; entries that are -inf
select cells the causal mask removes, so they are dropped here.  This is a
different algorithm from the forced-set + count form the oracle uses, so a
wrong count (the tail counted twice or not at all) or a whole tail block forced
fails it."""
import numpy as np
import pytest

from oracle import oracle as O
from _refs import Cfg, select_ref

CKPT = Cfg(n_head=4, n_head_kv=1, head_dim=128, block_tokens=4, page_tokens=64, top_k_blocks=7,
           sink_blocks=0, local_tokens=0, relu_per_head=1, shared_selection=1, topk_counts_forced=1)


def bias_topk(scores: np.ndarray, seq_len: int, r: int, kb: int) -> np.ndarray:
    n_past = seq_len - 1
    b_last, n_bid = n_past // r, (n_past + 1) // r
    nb = b_last + 1
    bias = np.full(nb, -np.inf, np.float32)
    bias[:n_bid] = 0.0
    if b_last >= n_bid:
        bias[b_last] = 1e9
    v = (scores[:nb].astype(np.float32) + bias).astype(np.float32)
    order = sorted(range(nb), key=lambda b: (-float(v[b]), b))[:kb]
    return np.array(sorted(b for b in order if v[b] != -np.inf), dtype=np.int32)


@pytest.mark.parametrize("seed", [0, 1, 2])
def test_checkpoint_rule_is_the_biased_top_k(seed):
    rng = np.random.default_rng(700 + seed)
    for L in range(1, 90):
        nb = (L + 3) // 4
        # coarse scores: many exact ties, so the index order is exercised
        scores = np.round(rng.standard_normal(nb + 4) * 2).astype(np.float32)
        want = bias_topk(scores, L, 4, CKPT.top_k_blocks)
        got = O.select(CKPT, scores, L)
        np.testing.assert_array_equal(got, want, err_msg=f"L={L}")
        np.testing.assert_array_equal(select_ref(CKPT, scores, L), want, err_msg=f"L={L}")
        assert len(got) <= CKPT.top_k_blocks


def test_whole_tail_block_is_not_forced():
    # L = 40: blocks 0..9 all whole; the tail block 9 scores lowest, so the
    # reference drops it (bias 0, like any whole block), though it holds the
    # token being decoded
    scores = np.arange(10, 0, -1).astype(np.float32)
    got = O.select(CKPT, scores, 40)
    np.testing.assert_array_equal(got, np.arange(7, dtype=np.int32))
    # L = 41: block 10 is partial and forced; six more by score
    scores = np.concatenate([scores, [-5.0]]).astype(np.float32)
    np.testing.assert_array_equal(O.select(CKPT, scores, 41), np.array([0, 1, 2, 3, 4, 5, 10], np.int32))
