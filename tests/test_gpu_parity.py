"""Parity of the HIP path (through the C ABI) with the CPU oracle.

Bit-exact: q8_0 bytes, pooled keys of whole blocks, selected block ids,
gathered cells.  Attention: |o - o_ref| <= 2e-3 + 1e-3 |o_ref| against the fp64
oracle on the same dequantized cache.
"""
import numpy as np
import pytest
import torch

from _gpu import assert_close_attn, cfg_of, decode_steps, fill, kv_rows, make_pair, np_of
from _refs import BASELINE, TINY, Cfg
from qwfnfer_amd import _lib, qsa

pytestmark = pytest.mark.gpu

G12 = Cfg(n_head=24, n_head_kv=2, head_dim=256, block_tokens=4, page_tokens=128, top_k_blocks=40,
          sink_blocks=1, local_tokens=16)          # the checkpoint's head shapes, small selection


@pytest.mark.parametrize("variant", [0, 1])
@pytest.mark.parametrize("dtype", [np.float32, np.float16])
def test_append_bytes_match_oracle(variant, dtype):
    cfg = Cfg(quant_variant=variant)
    rng = np.random.default_rng(100 + variant)
    dev, host = make_pair(cfg, 2, 3, seed=7, spare=2)
    n = 300
    seq = rng.integers(0, 2, n).astype(np.int32)
    pos = rng.permutation(2 * 3 * 256)[:n].astype(np.int32) % (3 * 256)
    key = seq.astype(np.int64) * 10**6 + pos
    _, keep = np.unique(key, return_index=True)
    seq, pos = seq[keep], pos[keep]
    k, v = kv_rows(rng, len(pos), cfg)
    k, v = k.astype(dtype), v.astype(dtype)
    assert host.append(k, v, pos, seq) == 0
    for _ in range(2):                                   # idempotent overwrite
        qsa.append_q8_0(dev, torch.from_numpy(k).cuda(), torch.from_numpy(v).cuda(),
                        torch.from_numpy(pos).cuda(), torch.from_numpy(seq).cuda())
        torch.cuda.synchronize()
        np.testing.assert_array_equal(np_of(dev.k_pages), host.k_pages)
        np.testing.assert_array_equal(np_of(dev.v_pages), host.v_pages)
    assert qsa.read_status(dev) == 0


def test_append_edge_values():
    cfg = BASELINE
    dev, host = make_pair(cfg, 1, 1)
    rows = np.zeros((8, 2, 128), np.float32)
    rows[1] = 1e-3                                      # constant block
    rows[2, :, ::7] = -5.0                              # sparse spikes
    rows[3] = np.ldexp(1.0, -20)                        # fp16-subnormal scale
    rows[4] = 3e4                                       # large scale
    rows[5, :, :32] = np.arange(32) - 15.5              # exact half-ties under id = 127/amax? (not exact)
    rows[6] = (np.arange(256).reshape(2, 128) % 17 - 8) * 0.25
    rows[7] = np.float32(1e-40)                         # fp32 subnormal inputs
    pos = np.arange(8, dtype=np.int32)
    host.append(rows, rows, pos)
    qsa.append_q8_0(dev, torch.from_numpy(rows).cuda(), torch.from_numpy(rows).cuda(),
                    torch.from_numpy(pos).cuda())
    torch.cuda.synchronize()
    np.testing.assert_array_equal(np_of(dev.k_pages), host.k_pages)


def test_append_reports_out_of_range_rows():
    cfg = BASELINE
    dev, host = make_pair(cfg, 1, 2)
    k = np.ones((2, 2, 128), np.float32)
    before = np_of(dev.k_pages).copy()
    qsa.append_q8_0(dev, torch.from_numpy(k).cuda(), torch.from_numpy(k).cuda(),
                    torch.tensor([512, -1], dtype=torch.int32, device="cuda"))
    assert qsa.read_status(dev) == _lib.STATUS_POS_RANGE
    qsa.append_q8_0(dev, torch.from_numpy(k).cuda(), torch.from_numpy(k).cuda(),
                    torch.tensor([0, 1], dtype=torch.int32, device="cuda"),
                    torch.tensor([1, 5], dtype=torch.int32, device="cuda"))
    assert qsa.read_status(dev) == _lib.STATUS_SEQ_RANGE
    np.testing.assert_array_equal(np_of(dev.k_pages), before)


@pytest.mark.parametrize("cfg", [BASELINE, TINY, G12])
def test_pool_matches_oracle(cfg):
    rng = np.random.default_rng(110)
    dev, host = make_pair(cfg, 2, 3, seed=3)
    lengths = [3 * cfg.page_tokens, 2 * cfg.page_tokens + 5]
    fill(dev, host, rng, lengths)
    for s, L in enumerate(lengths):
        nw = L // cfg.block_tokens
        np.testing.assert_array_equal(np_of(dev.pooled)[s, :, :nw], host.pooled[s, :, :nw])
    # pool_update of a listed subset recomputes the same values
    dev.pooled.zero_()
    ids = torch.tensor([0, 5, 7], dtype=torch.int32, device="cuda")
    sids = torch.tensor([1, 1, 0], dtype=torch.int32, device="cuda")
    qsa.pool_update(dev, ids, sids)
    torch.cuda.synchronize()
    got = np_of(dev.pooled)
    for b, s in ((0, 1), (5, 1), (7, 0)):
        np.testing.assert_array_equal(got[s, :, b], host.pooled[s, :, b])


def _indexer_case(cfg, lengths, seed, equal_scores=False, mutate=None):
    rng = np.random.default_rng(seed)
    pps = max(lengths) // cfg.page_tokens + 1
    dev, host = make_pair(cfg, len(lengths), pps, seed=seed)
    fill(dev, host, rng, lengths)
    q = rng.standard_normal((len(lengths), cfg.n_head, cfg.head_dim), dtype=np.float32)
    if equal_scores:                                   # every pooled key identical -> all ties
        host.pooled[...] = host.pooled[:, :, :1]
    if mutate is not None:                             # edit the pooled keys and queries on the host
        mutate(host.pooled, q, rng)
    if equal_scores or mutate is not None:
        dev.pooled.copy_(torch.from_numpy(host.pooled))
    L = np.array(lengths, np.int32)
    max_len = int(L.max())
    ws = qsa.Workspace(cfg_of(cfg), len(lengths), max_len)
    sel, nsel = qsa.indexer_topk(dev, torch.from_numpy(q).cuda(), torch.from_numpy(L).cuda(), max_len, ws)
    torch.cuda.synchronize()
    hs, hn = host.indexer_topk(q, L, max_sel=sel.shape[-1])
    sel, nsel = np_of(sel), np_of(nsel)
    np.testing.assert_array_equal(nsel, hn)
    for s in range(len(lengths)):
        for g in range(cfg.n_head_kv):
            np.testing.assert_array_equal(sel[s, g, :nsel[s, g]], hs[s, g, :hn[s, g]],
                                          err_msg=f"seq {s} len {lengths[s]} head {g}")
    return dev, host, q, L, sel, nsel, ws


@pytest.mark.parametrize("lengths", [[1], [63, 64, 65], [511, 512, 513], [4096], [4097, 4160],
                                     [32768], [20000, 100, 9000, 64 * 70]])
def test_indexer_matches_oracle(lengths):
    _indexer_case(BASELINE, lengths, seed=200 + len(lengths))


def test_indexer_ties_resolve_to_lower_index():
    _, _, _, _, sel, nsel, _ = _indexer_case(BASELINE, [32768], seed=210, equal_scores=True)
    assert list(sel[0, 0, :nsel[0, 0]]) == [0] + list(range(1, 65)) + list(range(504, 512))


def _inf_nan(p, q, rng):                               # +inf, -inf and NaN scores among finite ones
    q[..., 0] = np.abs(q[..., 0]) + np.float32(0.5)
    p[:, :, 5:40:7, 0] = np.inf
    p[:, :, 9:60:11, 0] = -np.inf
    p[:, :, 13:300:17, 3] = np.nan


def _outlier(p, q, rng):                               # one huge score squeezes the linear bins
    p[:, :, 77] *= np.float32(1e30)


def _half_ties(p, q, rng):                             # 200 equal scores among distinct ones
    p[:, :, 1:400:2] = p[:, :, 1:2]


def _small_spread(p, q, rng):                          # scores a few ulps apart
    p[...] = p[:, :, :1] + rng.standard_normal(p.shape).astype(np.float32) * np.float32(1e-6)


@pytest.mark.parametrize("mutate", [_inf_nan, _outlier, _half_ties, _small_spread])
def test_indexer_extreme_scores(mutate):
    _indexer_case(BASELINE, [32768, 20000], seed=230, mutate=mutate)


def test_indexer_more_blocks_than_lds_keys():
    # more than 8192 eligible blocks: the selection reads its keys from memory
    cfg = Cfg(n_head=8, n_head_kv=1, head_dim=64, block_tokens=2, page_tokens=64, top_k_blocks=40,
              sink_blocks=1, local_tokens=5)
    _indexer_case(cfg, [16600], seed=240)
    _indexer_case(cfg, [16600], seed=241, equal_scores=True)


# The 1024-thread selection first tries a cut placed from 4096 evenly spaced
# scores (block e_lo + j * n_eligible // 4096), then falls back to three passes
# over the keys.  With top_k 600 over 8,296 eligible blocks the cut keeps about
# 370 sample keys, so scores planted at exactly those blocks steer each branch;
# every case must select what the oracle selects.
BIG = Cfg(n_head=8, n_head_kv=1, head_dim=64, block_tokens=2, page_tokens=64, top_k_blocks=600,
          sink_blocks=1, local_tokens=5)
BIG_L = 16600


def _big_sample_blocks():
    last = BIG_L - 1
    w0 = last - BIG.local_tokens + 1
    e_lo, e_hi = BIG.sink_blocks, min(BIG_L // BIG.block_tokens, w0 // BIG.block_tokens)
    ne = e_hi - e_lo
    assert ne == 8296
    return e_lo + np.arange(4096) * ne // 4096


def _score_is_dim0(p, q, rng):                        # every query head reads dim 0 only
    q[...] = 0.0
    q[..., 0] = 1.0
    p[..., 0] = rng.standard_normal(p.shape[:-1]).astype(np.float32)


def _sample_high(p, q, rng):                           # the sampled blocks hold the top scores:
    _score_is_dim0(p, q, rng)                          # fewer candidates than top_k
    p[:, :, _big_sample_blocks(), 0] = np.float32(100) + np.arange(4096, dtype=np.float32) * np.float32(0.01)


def _sample_low(p, q, rng):                            # the sampled blocks hold the lowest scores:
    _score_is_dim0(p, q, rng)                          # more candidates than the LDS list holds
    p[:, :, _big_sample_blocks(), 0] = np.float32(-100) - np.arange(4096, dtype=np.float32) * np.float32(0.01)


def _wide_tie(p, q, rng):                              # 700 equal top scores: the candidates'
    _score_is_dim0(p, q, rng)                          # threshold bin overflows the rank list
    p[:, :, rng.choice(np.arange(1, 8297), 700, replace=False), 0] = np.float32(10)


def _sample_near_tie(p, q, rng):                       # 40 equal scores straddling the top-k edge
    _score_is_dim0(p, q, rng)
    top = np.argsort(-p[0, 0, 1:8297, 0], kind="stable")[:620] + 1
    p[:, :, top[580:620], 0] = p[0, 0, top[590], 0]


@pytest.mark.parametrize("mutate", [None, _sample_high, _sample_low, _wide_tie, _sample_near_tie, _inf_nan, _outlier,
                                    _small_spread])
def test_select_big_sampled_cut(mutate):
    _indexer_case(BIG, [BIG_L], seed=245, mutate=mutate)


def test_select_big_per_head_and_shared():
    """Two KV heads past 8192 eligible blocks: per-head selections (one
    multi-workgroup selection per head, three sequences), and one shared
    selection on the summed rows (the one-workgroup selection)."""
    two = Cfg(**{**BIG.__dict__, "n_head": 16, "n_head_kv": 2})
    _indexer_case(two, [BIG_L, 9000, BIG_L - 3], seed=246)
    _indexer_case(Cfg(**{**two.__dict__, "shared_selection": 1}), [BIG_L, BIG_L - 3], seed=247)


@pytest.mark.parametrize("cfg", [TINY, G12, Cfg(relu_per_head=1), Cfg(top_k_blocks=3, sink_blocks=2, local_tokens=100)])
def test_indexer_other_shapes(cfg):
    _indexer_case(cfg, [3 * cfg.page_tokens - 1, cfg.page_tokens + 7], seed=220)


def test_gather_matches_oracle():
    cfg = BASELINE
    dev, host, q, L, sel, nsel, ws = _indexer_case(cfg, [20000, 4500], seed=230)
    seq_len = torch.from_numpy(L).cuda()
    k, v, cells = qsa.gather_dequant(dev, seq_len, torch.from_numpy(sel).cuda(),
                                     torch.from_numpy(nsel).cuda(), sel.shape[-1])
    torch.cuda.synchronize()
    k, v, cells = np_of(k), np_of(v), np_of(cells)
    for s in range(2):
        for g in range(2):
            ids = [t for b in sel[s, g, :nsel[s, g]] for t in range(64 * b, 64 * b + 64) if t < L[s]]
            assert list(cells[s, g, :len(ids)]) == ids and (cells[s, g, len(ids):] == -1).all()
            for i in (0, 1, len(ids) // 2, len(ids) - 1):
                np.testing.assert_array_equal(k[s, g, i], host.dequant_row("k", s, ids[i], g))
                np.testing.assert_array_equal(v[s, g, i], host.dequant_row("v", s, ids[i], g))


@pytest.mark.parametrize("cfg,lengths", [(BASELINE, [32768]), (BASELINE, [700, 4096, 9000]),
                                         (TINY, [250, 77]), (G12, [300])])
def test_sparse_attention_matches_f64(cfg, lengths):
    dev, host, q, L, sel, nsel, ws = _indexer_case(cfg, lengths, seed=240)
    out = qsa.sparse_decode_attn(dev, torch.from_numpy(q).cuda(), torch.from_numpy(L).cuda(), int(L.max()), ws,
                                 torch.from_numpy(sel).cuda(), torch.from_numpy(nsel).cuda())
    torch.cuda.synchronize()
    ref = host.attention_f64(q, L, sel, nsel)
    assert_close_attn(np_of(out), ref, "sparse attention")


@pytest.mark.parametrize("L", [1, 64, 1000, 4096])
def test_dense_attention_matches_f64(L):
    cfg = Cfg(top_k_blocks=0)                          # config 1: dense GQA over every key
    rng = np.random.default_rng(250)
    dev, host = make_pair(cfg, 1, L // 256 + 1)
    fill(dev, host, rng, [L], scaled=False, pool=False)
    q = rng.standard_normal((1, 16, 128), dtype=np.float32)
    ws = qsa.Workspace(cfg_of(cfg), 1, L)
    Lt = torch.tensor([L], dtype=torch.int32, device="cuda")
    out = qsa.sparse_decode_attn(dev, torch.from_numpy(q).cuda(), Lt, L, ws)
    torch.cuda.synchronize()
    assert_close_attn(np_of(out), host.attention_f64(q, [L]), "dense attention")


# blocks shorter than a 64-cell tile (the attention gathers 64 / block_tokens
# blocks a tile): dense calls over every block, at lengths that end inside a
# block and inside a tile, for the checkpoint's heads, the tiny shape and the
# BASELINE heads at 2-, 4-, 16- and 32-token blocks (permuted pages)
GATH_DENSE = [(G12, [1, 5, 67, 2053]), (TINY, [3, 64, 301]),
              (Cfg(block_tokens=16, top_k_blocks=0), [17, 1000]), (Cfg(block_tokens=32, top_k_blocks=0), [95]),
              (Cfg(block_tokens=2, top_k_blocks=0), [129])]


@pytest.mark.parametrize("cfg,lengths", GATH_DENSE)
def test_dense_attention_gathered_tiles(cfg, lengths):
    cfg = Cfg(**{**cfg.__dict__, "top_k_blocks": 0})
    rng = np.random.default_rng(255)
    n = len(lengths)
    pps = max(lengths) // cfg.page_tokens + 2
    dev, host = make_pair(cfg, n, pps, seed=256)        # permuted pages
    fill(dev, host, rng, lengths, pool=False)
    q = rng.standard_normal((n, cfg.n_head, cfg.head_dim), dtype=np.float32)
    L = np.array(lengths, np.int32)
    ws = qsa.Workspace(cfg_of(cfg), n, int(L.max()))
    out = qsa.sparse_decode_attn(dev, torch.from_numpy(q).cuda(), torch.from_numpy(L).cuda(), int(L.max()), ws)
    torch.cuda.synchronize()
    assert qsa.read_status(dev) == 0
    assert_close_attn(np_of(out), host.attention_f64(q, L), "dense attention, gathered tiles")


def test_sparse_attention_gathered_unsorted_selection():
    """A given selection in no particular order, with a block past the length
    in the middle: gathered tiles mask per cell, not per prefix."""
    cfg = TINY
    dev, host, q, L, sel, nsel, ws = _indexer_case(cfg, [250, 77], seed=241)
    rng = np.random.default_rng(242)
    for s in range(len(L)):
        for g in range(cfg.n_head_kv):
            k = nsel[s, g]
            row = sel[s, g, :k].copy()
            rng.shuffle(row)
            row[k // 2] = (L[s] - 1) // cfg.block_tokens + 1      # the block after the last: masked
            sel[s, g, :k] = row
    out = qsa.sparse_decode_attn(dev, torch.from_numpy(q).cuda(), torch.from_numpy(L).cuda(), int(L.max()), ws,
                                 torch.from_numpy(sel).cuda(), torch.from_numpy(nsel).cuda())
    torch.cuda.synchronize()
    assert_close_attn(np_of(out), host.attention_f64(q, L, sel, nsel), "gathered attention, shuffled selection")


def _decode_steps(cfg, lengths, steps, seed, dtype=np.float32, zero_pooled=False):
    """Fused decode steps on a batch of sequences vs the oracle."""
    return decode_steps(cfg, lengths, steps, seed, dtype=dtype, zero_pooled=zero_pooled)


def test_decode_steps_cross_block_boundaries():
    _decode_steps(BASELINE, [4096 - 3], steps=70, seed=300)


def test_decode_steps_batched_paged():
    # config 5 in miniature: several sequences, permuted pages, different lengths
    _decode_steps(BASELINE, [5000, 700, 12345, 64 * 9 - 1], steps=6, seed=310, dtype=np.float16)


@pytest.mark.parametrize("relu", [0, 1])
def test_decode_steps_shared_selection(relu):
    # one selection for both KV heads on the heads' summed scores (the
    # checkpoint's selection rule); the oracle copies it to every head
    cfg = Cfg(shared_selection=1, relu_per_head=relu)
    _decode_steps(cfg, [5000, 64 * 40 - 2], steps=4, seed=340 + relu)
    _decode_steps(Cfg(**{**TINY.__dict__, "shared_selection": 1, "relu_per_head": relu}), [130], steps=5,
                  seed=342 + relu)


def test_decode_steps_tiny_and_checkpoint_shapes():
    _decode_steps(TINY, [61, 130], steps=10, seed=320)
    _decode_steps(G12, [250], steps=6, seed=321)


# One to three sequences of a matrix-core shape: the attention workgroups make
# the selection themselves from a scores-only indexer launch (and write it out).
@pytest.mark.parametrize("cfg", [
    BASELINE,
    Cfg(n_head=8, n_head_kv=2),                                     # group 4
    Cfg(n_head=4, n_head_kv=2),                                     # group 2
    Cfg(n_head=16, n_head_kv=2, head_dim=64),                       # 256-thread workgroups
    Cfg(n_head=24, n_head_kv=2, head_dim=256),                      # group 12, head_dim 256
])
def test_decode_steps_attention_selects(cfg):
    _decode_steps(cfg, [3000, 64 * 70 + 5, 100], steps=3, seed=350)


def test_decode_steps_attention_selects_ties():
    # every pooled key 0: ties everywhere, the radix path of the in-kernel selection
    _decode_steps(BASELINE, [20000], steps=2, seed=355, zero_pooled=True)


@pytest.mark.parametrize("cfg", [BASELINE, Cfg(kv_type=1), Cfg(kv_type=2), Cfg(kv_round_f16=1),
                                 Cfg(block_tokens=16), Cfg(kv_type=1, block_tokens=16)])
def test_decode_is_deterministic(cfg):
    # two fresh caches of the same rows: the fused step's bytes, pooled keys
    # and outputs are bit-identical; then the same step again on the first
    # cache (its token rewritten with the same values) gives the same outputs
    rng = np.random.default_rng(330)
    res = []
    for rep in range(2):
        dev, host = make_pair(cfg, 2, 40, seed=5)
        fill(dev, host, np.random.default_rng(331), [9000, 6000])
        ws = qsa.Workspace(cfg_of(cfg), 2, 10000)
        q = torch.from_numpy(np.random.default_rng(332).standard_normal((2, 16, 128), dtype=np.float32)).cuda()
        kn = torch.from_numpy(np.random.default_rng(333).standard_normal((2, 2, 128), dtype=np.float32)).cuda()
        L = torch.tensor([9001, 6001], dtype=torch.int32, device="cuda")
        out = qsa.sparse_attn_decode(dev, q, kn, kn, L, 10000, ws)
        torch.cuda.synchronize()
        res.append((np_of(out).tobytes(), np_of(dev.k_pages).tobytes(), np_of(dev.pooled).tobytes()))
        for again in range(3):
            out2 = qsa.sparse_attn_decode(dev, q, kn, kn, L, 10000, ws)
            torch.cuda.synchronize()
            assert np_of(out2).tobytes() == res[-1][0], f"repeat {again} differs"
    assert res[0] == res[1]


# ---- prefill ------------------------------------------------------------------------

def _prefill_case(cfg, pre, n_q, seed, q_batch=None, rows=True, dtype=np.float32, seq=1, kv=None):
    """A prefill chunk of sequence `seq` at positions pre .. pre+n_q-1 (the rows
    appended and the completed blocks pooled by the call when `rows`) against
    the oracle: cache bytes and pooled keys bit-exact, every query's selection
    bit-exact, outputs within the attention tolerance.  `kv` (rng, n, cfg) ->
    (k, v) draws the cache's and the chunk's rows instead of kv_rows."""
    rng = np.random.default_rng(seed)
    max_len = pre + n_q
    pps = max_len // cfg.page_tokens + 1
    dev, host = make_pair(cfg, 2, pps, seed=seed)
    fill(dev, host, rng, [pre // 2, pre] if seq == 1 else [pre, pre // 2], rows=kv)
    kn, vn = kv(rng, n_q, cfg) if kv else kv_rows(rng, n_q, cfg)
    kn, vn = kn.astype(dtype), vn.astype(dtype)
    q = rng.standard_normal((n_q, cfg.n_head, cfg.head_dim), dtype=np.float32)
    bt = cfg.block_tokens
    assert host.append(kn, vn, np.arange(pre, max_len, dtype=np.int32), np.full(n_q, seq, np.int32)) == 0
    for b in range(pre // bt, max_len // bt):
        assert host.pool_block(seq, b) == 0
    c = cfg_of(cfg)
    msel = c.max_selected(max_len)
    sel = torch.empty((n_q, cfg.n_head_kv, msel), dtype=torch.int32, device="cuda")
    nsel = torch.empty((n_q, cfg.n_head_kv), dtype=torch.int32, device="cuda")
    ws = qsa.Workspace.for_prefill(c, max_len, q_batch or n_q)
    qd = torch.from_numpy(q).cuda()
    if rows:
        out = qsa.sparse_attn_prefill(dev, qd, seq, pre, ws, torch.from_numpy(kn).cuda(), torch.from_numpy(vn).cuda(),
                                      sel=sel, n_sel=nsel)
    else:
        qsa.append_q8_0(dev, torch.from_numpy(kn).cuda(), torch.from_numpy(vn).cuda(),
                        torch.arange(pre, max_len, dtype=torch.int32, device="cuda"),
                        torch.full((n_q,), seq, dtype=torch.int32, device="cuda"))
        qsa.pool_rebuild(dev, seq, max_len // bt)
        out = qsa.sparse_attn_prefill(dev, qd, seq, pre, ws, sel=sel, n_sel=nsel)
    torch.cuda.synchronize()
    assert qsa.read_status(dev) == 0
    np.testing.assert_array_equal(np_of(dev.k_pages), host.k_pages)
    np.testing.assert_array_equal(np_of(dev.v_pages), host.v_pages)
    np.testing.assert_array_equal(np_of(dev.pooled)[:, :, :max_len // bt], host.pooled[:, :, :max_len // bt])
    hs, hn, ref = host.prefill_f64(q, seq, pre, max_sel=msel)
    gs, gn = np_of(sel), np_of(nsel)
    np.testing.assert_array_equal(gn, hn)
    for i in range(n_q):
        for g in range(cfg.n_head_kv):
            np.testing.assert_array_equal(gs[i, g, :gn[i, g]], hs[i, g, :hn[i, g]],
                                          err_msg=f"query {i} (pos {pre + i}) head {g}")
    assert_close_attn(np_of(out), ref, f"prefill pre={pre} n_q={n_q}")
    return np_of(out), gs, gn


def test_prefill_matches_oracle():
    # 6000..6159: eligible sets beyond top-64, chunk crosses blocks; config 4 in miniature
    _prefill_case(BASELINE, 6000, 160, seed=600)


def test_prefill_batches_are_invisible():
    # a workspace of 24 queries per launch pair gives the same bytes as one batch
    a = _prefill_case(BASELINE, 5000, 100, seed=610)
    b = _prefill_case(BASELINE, 5000, 100, seed=610, q_batch=24)
    for x, y in zip(a, b):
        np.testing.assert_array_equal(x, y)


def test_prefill_from_the_first_token_and_f16_rows():
    _prefill_case(BASELINE, 0, 700, seed=620, dtype=np.float16, seq=0)


def test_prefill_rows_already_in_place():
    _prefill_case(BASELINE, 4200, 64, seed=630, rows=False)


def test_prefill_other_shapes():
    _prefill_case(TINY, 90, 70, seed=640)            # 4-token blocks: the general attention kernel
    _prefill_case(G12, 200, 40, seed=641)


def _tied_keys(rng, n, cfg):
    """Every key row the same vector (so every pooled key, and every block
    score of a query, is the same); V ~ N(0,1)."""
    k = np.broadcast_to(np.linspace(-1.0, 1.0, cfg.head_dim, dtype=np.float32),
                        (n, cfg.n_head_kv, cfg.head_dim)).copy()
    v = rng.standard_normal((n, cfg.n_head_kv, cfg.head_dim), dtype=np.float32)
    return k, v


def test_prefill_tied_scores_rank_by_index():
    """All block scores equal: every eligible block is a candidate of the
    bounded scoring, and the exact ranking takes the lowest indices -- below
    the candidate cap (90 eligible blocks) and, past it (about 600), through
    the exact-row fallback."""
    _prefill_case(BASELINE, 6200, 24, seed=670, kv=_tied_keys)
    _prefill_case(BASELINE, 39000, 12, seed=671, kv=_tied_keys)


def _near_tied_keys(rng, n, cfg):
    """Key rows one vector times (1 + 1e-4 noise): block scores differ in their
    last few bits, so the bounded scoring rules out almost nothing."""
    base = np.linspace(-1.0, 1.0, cfg.head_dim, dtype=np.float32)
    k = base * (1.0 + 1e-4 * rng.standard_normal((n, cfg.n_head_kv, cfg.head_dim), dtype=np.float32))
    v = rng.standard_normal((n, cfg.n_head_kv, cfg.head_dim), dtype=np.float32)
    return k.astype(np.float32), v


def _wide_range_keys(rng, n, cfg):
    """K, V ~ N(0,1), each q8_0 block times a log-uniform scale in [1e-3, 1e3]."""
    k = rng.standard_normal((n, cfg.n_head_kv, cfg.head_dim), dtype=np.float32)
    v = rng.standard_normal((n, cfg.n_head_kv, cfg.head_dim), dtype=np.float32)
    nb = cfg.head_dim // 32
    for x in (k, v):
        sc = np.exp(rng.uniform(np.log(1e-3), np.log(1e3), (n, cfg.n_head_kv, nb))).astype(np.float32)
        x.reshape(n, cfg.n_head_kv, nb, 32)[...] *= sc[..., None]
    return k, v


def test_prefill_near_tied_scores():
    """Block scores equal but for their last bits: every eligible block is a
    candidate (below and past the candidate cap) and the exact scores decide."""
    _prefill_case(BASELINE, 6200, 24, seed=674, kv=_near_tied_keys)
    _prefill_case(BASELINE, 39000, 12, seed=675, kv=_near_tied_keys)


def test_prefill_wide_dynamic_range():
    """Keys over six decades of block scale: the bound's relative terms span the
    same range and every selection stays exact."""
    _prefill_case(BASELINE, 9000, 40, seed=676, kv=_wide_range_keys)


def test_prefill_head_dim_256_group_8():
    """head_dim 256 with 8 query heads a KV head: the prefill attention's
    paired-block QK with two scale words a cell (and the exact scoring path,
    whose query fragments the matrix-core scoring cannot hold)."""
    _prefill_case(Cfg(head_dim=256), 5000, 40, seed=673)


def test_prefill_relu_per_head_selection():
    """relu'd head dots with per-KV-head selections (the matrix-core scoring's
    relu path), at a context where most blocks are eligible."""
    _prefill_case(Cfg(relu_per_head=1), 9000, 48, seed=672)


def test_prefill_shared_selection():
    _prefill_case(Cfg(shared_selection=1), 6000, 96, seed=650)
    _prefill_case(Cfg(**{**TINY.__dict__, "shared_selection": 1, "relu_per_head": 1}), 90, 70, seed=651)


def test_prefill_odd_chunks_and_batches():
    # an odd chunk in odd batches (5 queries per launch pair) gives the same
    # bytes as one batch; a group of 4 heads on the matrix cores
    a = _prefill_case(BASELINE, 5003, 37, seed=660)
    b = _prefill_case(BASELINE, 5003, 37, seed=660, q_batch=5)
    for x, y in zip(a, b):
        np.testing.assert_array_equal(x, y)
    _prefill_case(Cfg(n_head=8, n_head_kv=2, top_k_blocks=8, local_tokens=100), 3000, 41, seed=661)   # G = 4
