"""Parity of the HIP path with the CPU oracle at the workloads bench.py times.

* Config 3 at 65,536 and 163,840 tokens (the headline), BASELINE shapes with a
  log-uniform [0.1, 10] scale per q8_0 block: fused decode steps that cross a
  block completion, then steps through the two-call path, with the attention
  also re-run over each step's selection.
* Longer contexts that reach every register path of the two selections: the
  indexer's 256-thread selection (two-call path) holds 4 .. 32 keys a thread,
  chosen by the eligible span, and the attention's own selection (k_dec, fused
  path) 4 .. 32 keys over its 256 threads, chosen by the span of max_seq_len.
* Configs 1 and 2: the bench's dense 4,096-token step and its 32,768-token
  sparse step through the fused call.
* Config 5: the bench's eight log-uniform lengths on a permuted page table,
  through the fused call (the attention selects for itself) and
  qwfn_sparse_decode_attn (k_dec over a given selection, several tiles a
  workgroup when one tile each would not fit the device at once).
* Config 4: one 8,192-query chunk of fp16 rows appended at 155,648: cache
  bytes and pooled keys bit-exact, every query's selection bit-exact,
  attention of every query within the tolerance.
* The checkpoint's bias rule (local_tokens 0, topk_counts_forced 1) through
  both decode paths across block completions: a completed block is eligible
  at the same step, so it must be pooled before it is scored.

Selections, cache bytes and pooled keys are bit-exact; attention is within
|o - o_ref| <= 2e-3 + 1e-3 |o_ref| of the fp64 oracle.
"""
import math
import time

import numpy as np
import pytest
import torch

from _gpu import assert_close_attn, cfg_of, decode_steps, fill, kv_rows, make_pair, np_of
from _refs import BASELINE, Cfg
from qwfnfer_amd import qsa

pytestmark = pytest.mark.gpu

# bench.py's config-5 lengths: floor(exp(U(ln 4096, ln 262144))) from numpy's
# default_rng(3), eight draws
CONFIG5_LENGTHS = [5848, 10966, 114711, 46115, 6058, 24812, 30033, 7959]


def test_config5_lengths_are_the_bench_draws():
    rng = np.random.default_rng(3)
    assert [int(math.exp(rng.uniform(math.log(4096), math.log(262144)))) for _ in range(8)] == CONFIG5_LENGTHS


def _span(cfg, L):
    """Eligible span the register selections size their keys-per-thread by."""
    last = L - 1
    fw = max(0, last - cfg.local_tokens + 1) // cfg.block_tokens
    e_hi = max(min(L // cfg.block_tokens, fw), cfg.sink_blocks)
    return e_hi - (cfg.sink_blocks & ~3)


# Config 3's contexts, then one length for each keys-per-thread tier past
# them: (indexer KPT, k_dec KPT) = (4, 4) at 65,536; (12, 16) at 163,840;
# (16, 16) at 230,400; (24, 32) at 320,000; (32, 32) at 480,000.  Config 5
# runs k_dec's KPT 8.
@pytest.mark.parametrize("L0,kpt_idx,kpt_dec", [(65536, 4, 4), (163840, 12, 16), (230400, 16, 16),
                                                (320000, 24, 32), (480000, 32, 32)])
def test_config3_long_context_decode(L0, kpt_idx, kpt_dec):
    span = _span(BASELINE, L0)
    assert min(t for t in [4, 8, 12, 16, 24, 32] if span <= t * 256) == kpt_idx
    max_len = L0 - 2 + 5                          # decode_steps' max_seq_len: the fill plus the steps
    assert min(t for t in [4, 8, 16, 32] if max_len // BASELINE.block_tokens <= t * 256) == kpt_dec
    # fill L0 - 2 tokens: the second fused step completes block L0/64 - 1 and
    # pools it; two two-call steps follow
    decode_steps(BASELINE, [L0 - 2], steps=5, seed=700 + L0 % 997,
                 modes=["fused", "fused", "fused", "two_call", "two_call"], reattend=True, verbose=True)


def test_config1_dense_and_config2_sparse_steps():
    # config 1: dense attention over every key, the fused call at 4,096 tokens
    # (the indexer selects every block); config 2: 32,768 tokens, top-64
    decode_steps(Cfg(top_k_blocks=0), [4096 - 2], steps=3, seed=740, verbose=True)
    decode_steps(BASELINE, [32768 - 2], steps=3, seed=741, modes=["fused", "fused", "two_call"], reattend=True,
                 verbose=True)


@pytest.mark.parametrize("shift", [False, True])
def test_config5_batched_decode(shift):
    # shift: every length moved to 62 mod 64, so the second step completes a
    # block in all eight sequences at once
    lengths = [L - (L % 64) + 62 for L in CONFIG5_LENGTHS] if shift else CONFIG5_LENGTHS
    decode_steps(BASELINE, lengths, steps=3, seed=720 + shift, modes=["fused", "fused", "two_call"],
                 reattend=True, verbose=True)


@pytest.mark.parametrize("stride", [1])
def test_config4_prefill_chunk(stride):
    # stride 1: the attention of every one of the 8192 queries is checked
    cfg = BASELINE
    pre, n_q = 155648, 8192
    seq = 0
    rng = np.random.default_rng(740)
    max_len = pre + n_q
    pps = max_len // cfg.page_tokens + 1
    dev, host = make_pair(cfg, 1, pps, seed=740)
    fill(dev, host, rng, [pre])
    kn, vn = kv_rows(rng, n_q, cfg)
    kn, vn = kn.astype(np.float16), vn.astype(np.float16)
    q = rng.standard_normal((n_q, cfg.n_head, cfg.head_dim), dtype=np.float32)
    bt = cfg.block_tokens
    assert host.append(kn, vn, np.arange(pre, max_len, dtype=np.int32), np.full(n_q, seq, np.int32)) == 0
    for b in range(pre // bt, max_len // bt):
        assert host.pool_block(seq, b) == 0
    c = cfg_of(cfg)
    msel = c.max_selected(max_len)
    sel = torch.empty((n_q, cfg.n_head_kv, msel), dtype=torch.int32, device="cuda")
    nsel = torch.empty((n_q, cfg.n_head_kv), dtype=torch.int32, device="cuda")
    ws = qsa.Workspace.for_prefill(c, max_len, n_q)          # the bench's one batch of 8192
    print(f"  prefill {n_q} queries at {pre}", flush=True)
    out = qsa.sparse_attn_prefill(dev, torch.from_numpy(q).cuda(), seq, pre, ws, torch.from_numpy(kn).cuda(),
                                  torch.from_numpy(vn).cuda(), sel=sel, n_sel=nsel)
    torch.cuda.synchronize()
    assert qsa.read_status(dev) == 0
    np.testing.assert_array_equal(np_of(dev.k_pages), host.k_pages)
    np.testing.assert_array_equal(np_of(dev.v_pages), host.v_pages)
    nw = max_len // bt
    np.testing.assert_array_equal(np_of(dev.pooled)[:, :, :nw], host.pooled[:, :, :nw])
    t0 = time.perf_counter()
    hs, hn, ref = host.prefill_f64(q, seq, pre, max_sel=msel, attn_stride=stride)
    print(f"  oracle prefill (attention stride {stride}): {time.perf_counter() - t0:.1f} s", flush=True)
    gs, gn = np_of(sel), np_of(nsel)
    np.testing.assert_array_equal(gn, hn)
    bad = [(i, g) for i in range(n_q) for g in range(cfg.n_head_kv)
           if not np.array_equal(gs[i, g, :gn[i, g]], hs[i, g, :hn[i, g]])]
    assert not bad, f"{len(bad)} (query, head) selections differ, first {bad[:4]}"
    idx = sorted(set(range(0, n_q, stride)) | {n_q - 1})
    assert_close_attn(np_of(out)[idx], ref[idx], f"prefill chunk, {len(idx)} sampled queries")


# The checkpoint's bias rule at BASELINE head shapes: no sink, no window, the
# kept count includes the forced partial tail block, relu per head.
CKPT_RULE = Cfg(sink_blocks=0, local_tokens=0, topk_counts_forced=1, relu_per_head=1)


@pytest.mark.parametrize("mode", ["fused", "two_call"])
def test_checkpoint_rule_decode_pools_before_scoring(mode):
    # 19197 + 3 = 64 * 300: sequence 0 completes block 299 at step 3;
    # 9598 + 2 = 64 * 150: sequence 1 completes block 149 at step 2.  Each
    # completed block is whole, hence eligible, at the step that completes it.
    decode_steps(CKPT_RULE, [64 * 300 - 3, 64 * 150 - 2], steps=4, seed=760, modes=[mode] * 4, reattend=True)
