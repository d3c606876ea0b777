"""The attention's own selection over long score rows (the checkpoint layer's
decode past 8192 eligible blocks), run alone through
qwfn_qsa_test_select_rows on score rows planted on the host, against the
oracle's selection (qwfn_oracle_select) on the same rows: counts and blocks
bit-exact, ties to the lower block.

The hook restates on the row what the product takes from the append and
indexer launches: a cut from 1,024 evenly spaced scores (block e_lo + j *
n_eligible // 1024; the hook keeps the smallest key of the sample's top rank,
the product the mean of 16 part keys), every eligible score at or above it as
a candidate in block order.  The attention's selection ranks the candidates
exactly; too few or too many candidates, or an overfull threshold bin, fall
back to three radix passes over the row.  Any cut leaves the result exact, so
the test pins the ranking and the fallbacks; scores planted at 4,096 evenly
spaced blocks (a superset of the 1,024 samples) steer each branch.  The
product's own cut is covered end to end by tests/test_gpu_checkpoint.py's
long-context fused decode."""
import ctypes as C

import numpy as np
import pytest
import torch

from _ckpt import CKPT
from _gpu import cfg_of, np_of
from _refs import Cfg
from oracle import oracle as O
from qwfnfer_amd import _lib

pytestmark = pytest.mark.gpu

# the checkpoint's rule (513 kept blocks counting a partial tail, no sink or
# window), and a rule with a sink block, a window and 600 scored blocks
RULES = {
    "ckpt": CKPT,
    "window": Cfg(n_head=24, n_head_kv=2, head_dim=256, block_tokens=4, page_tokens=256, top_k_blocks=600,
                  sink_blocks=1, local_tokens=37),
}


def _select(cfg, rows, lengths, max_seq_len):
    """Run the device selection on rows [n][nb_cap]; returns (sel, n_sel)."""
    c = cfg_of(cfg)
    n, nb_cap = rows.shape
    msel = c.max_selected(max_seq_len)
    sc = torch.from_numpy(np.ascontiguousarray(rows, np.float32)).cuda()
    L = torch.tensor(lengths, dtype=torch.int32, device="cuda")
    sel = torch.full((n, msel), -7, dtype=torch.int32, device="cuda")
    nsel = torch.full((n,), -7, dtype=torch.int32, device="cuda")
    s = c.shape()
    print(f"\n  select rows: lengths {lengths}, max_seq_len {max_seq_len}", flush=True)
    _lib.call("qwfn_qsa_test_select_rows", C.byref(s), sc.data_ptr(), nb_cap, L.data_ptr(), n, max_seq_len,
              sel.data_ptr(), nsel.data_ptr(), msel, torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    return np_of(sel), np_of(nsel), msel


def _case(rule, lengths, seed, plant=None, max_seq_len=None):
    cfg = RULES[rule]
    rng = np.random.default_rng(seed)
    max_seq_len = max_seq_len or max(lengths)
    nb_cap = (max_seq_len // cfg.block_tokens + 4 + 63) // 64 * 64
    rows = rng.standard_normal((len(lengths), nb_cap)).astype(np.float32)
    if plant is not None:
        for i, L in enumerate(lengths):
            plant(rows[i], _eligible(cfg, L), rng)
    gs, gn, msel = _select(cfg, rows, lengths, max_seq_len)
    for i, L in enumerate(lengths):
        want = O.select(cfg, rows[i], L, msel)
        assert gn[i] == len(want), f"row {i} (L {L}): {gn[i]} selected, oracle {len(want)}"
        np.testing.assert_array_equal(gs[i, :gn[i]], want, err_msg=f"row {i} (L {L})")
    return rows, gs, gn


def _eligible(cfg, L):
    last = L - 1
    w0 = last - cfg.local_tokens + 1
    fw = w0 // cfg.block_tokens if w0 > 0 else 0
    e_lo = cfg.sink_blocks
    return e_lo, max(e_lo, min(L // cfg.block_tokens, fw))


def _samples(e):                                      # 4,096 positions: the 1,024 samples among them
    e_lo, e_hi = e
    ne = e_hi - e_lo
    return e_lo + np.arange(4096) * ne // 4096


def _sample_high(row, e, rng):                        # the sampled blocks hold the top scores:
    row[_samples(e)] = np.float32(100) + np.arange(4096, dtype=np.float32) * np.float32(0.01)   # too few candidates


def _sample_low(row, e, rng):                         # the sampled blocks hold the lowest scores:
    row[_samples(e)] = np.float32(-100) - np.arange(4096, dtype=np.float32) * np.float32(0.01)  # too many


def _wide_tie(row, e, rng):                           # 700 equal top scores: the threshold bin
    e_lo, e_hi = e                                    # overflows the ranked list
    row[rng.choice(np.arange(e_lo, e_hi), 700, replace=False)] = np.float32(10)


def _near_tie(row, e, rng):                           # 40 equal scores straddling the top-k edge
    e_lo, e_hi = e
    top = np.argsort(-row[e_lo:e_hi], kind="stable")[:560] + e_lo
    row[top[480:520]] = row[top[500]]


def _relu_zeros(row, e, rng):                         # most scores exactly 0, as relu'd sums give
    row[rng.random(row.shape) < 0.9] = np.float32(0)


def _cluster(row, e, rng):                            # the top scores in one run of blocks
    e_lo, e_hi = e
    row[e_lo + 3000:e_lo + 3600] += np.float32(8)


def _inf_nan(row, e, rng):                            # +inf, -inf and NaN among finite scores
    e_lo, e_hi = e
    row[e_lo + 5:e_hi:997] = np.inf
    row[e_lo + 9:e_hi:1201] = -np.inf
    row[e_lo + 13:e_hi:89] = np.nan


def _all_equal(row, e, rng):                          # one value: the lowest blocks win
    row[...] = np.float32(0.25)


def _small_spread(row, e, rng):                       # scores a few ulps apart
    row[...] = np.float32(1) + rng.standard_normal(row.shape).astype(np.float32) * np.float32(1e-6)


@pytest.mark.parametrize("rule", ["ckpt", "window"])
@pytest.mark.parametrize("lengths", [[40003], [33000, 45001, 163841], [65537, 196000]])
def test_select_rows_random(rule, lengths):
    """Random rows at 8,250 .. 49,151 eligible blocks: each round count of the
    selection (16, 32, 48 rounds of 4-block groups a thread)."""
    _case(rule, lengths, seed=900 + len(lengths) + (rule == "window"))


@pytest.mark.parametrize("plant", [_sample_high, _sample_low, _wide_tie, _near_tie, _relu_zeros, _cluster, _inf_nan,
                                   _all_equal, _small_spread])
def test_select_rows_steered(plant):
    _case("ckpt", [163841, 40003], seed=910, plant=plant)
    _case("window", [163841], seed=911, plant=plant)


def test_select_rows_shorter_than_max():
    """Lengths well below max_seq_len (the rows' unused tails hold other
    scores), and one short enough for every block to be kept."""
    _case("ckpt", [40003, 9000, 2000], seed=920, max_seq_len=163841)


def test_select_rows_rejects_longer_rows():
    cfg = RULES["ckpt"]
    c = cfg_of(cfg)
    L = 4 * 49152 + 4 * 256 * 4
    nb_cap = (L // 4 + 4 + 63) // 64 * 64
    sc = torch.zeros(nb_cap, device="cuda")
    Lt = torch.tensor([L], dtype=torch.int32, device="cuda")
    msel = c.max_selected(L)
    sel = torch.empty(msel, dtype=torch.int32, device="cuda")
    nsel = torch.empty(1, dtype=torch.int32, device="cuda")
    s = c.shape()
    rc = _lib.load().qwfn_qsa_test_select_rows(C.byref(s), sc.data_ptr(), nb_cap, Lt.data_ptr(), 1, L, sel.data_ptr(),
                                              nsel.data_ptr(), msel, None)
    assert rc == _lib.QWFN_ERANGE
