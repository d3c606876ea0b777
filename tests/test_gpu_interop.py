"""The reference's cache rows <-> the paged layout, through the C ABI.

The reference's cache tensor row of a token is its n_head_kv * head_dim
elements, head-major, as ggml block_q8_0 {fp16 d; int8 qs[32]}
(src/qwfn_state.cpp:40, 52-53).  Exported rows must equal the oracle's q8_0
quantization of the appended values in that order, byte for byte; imported
rows must leave the bytes an append would; a snapshot must reproduce the
selections and attention of the cache it came from, bit for bit.
"""
import numpy as np
import pytest
import torch

from _gpu import cfg_of, fill, kv_rows, make_pair, np_of
from _refs import BASELINE, TINY, Cfg
from oracle import oracle as O
from qwfnfer_amd import _lib, qsa, snapshot

pytestmark = pytest.mark.gpu

G12 = Cfg(n_head=24, n_head_kv=2, head_dim=256, block_tokens=4, page_tokens=128, top_k_blocks=40,
          sink_blocks=1, local_tokens=16)


def _appended(cfg, seed, lengths, pps):
    rng = np.random.default_rng(seed)
    dev, host = make_pair(cfg, len(lengths), pps, seed=seed, spare=3)
    rows = []
    for s, L in enumerate(lengths):
        k, v = kv_rows(rng, L, cfg)
        pos = np.arange(L, dtype=np.int32)
        sid = np.full(L, s, dtype=np.int32)
        assert host.append(k, v, pos, sid) == 0
        qsa.append_q8_0(dev, torch.from_numpy(k).cuda(), torch.from_numpy(v).cuda(),
                        torch.from_numpy(pos).cuda(), torch.from_numpy(sid).cuda())
        rows.append((k, v))
    torch.cuda.synchronize()
    return dev, host, rows


def _ggml_rows(x, variant):
    """The reference's cache rows of f32 rows [n, Hkv, hd]: one ggml q8_0 row per token."""
    return np.stack([O.quantize_row_ggml(x[t].ravel(), variant) for t in range(x.shape[0])])


@pytest.mark.parametrize("cfg,lengths,pps", [
    (Cfg(quant_variant=0), [700, 300], 3),
    (Cfg(quant_variant=1), [513], 3),
    (TINY, [61, 130], 3),                  # V in the K layout (4-token blocks)
    (G12, [250], 2),                       # head_dim 256
])
def test_export_is_the_reference_row_format(cfg, lengths, pps):
    dev, host, rows = _appended(cfg, 900, lengths, pps)
    rb = cfg_of(cfg).row_bytes()
    assert rb == cfg.n_head_kv * cfg.head_dim // 32 * 34
    for s, (k, v) in enumerate(rows):
        L = k.shape[0]
        for pos0, n in ((0, L), (L // 3, L - L // 3), (L - 1, 1)):
            kr, vr = qsa.export_rows_q8_0(dev, s, pos0, n)
            torch.cuda.synchronize()
            np.testing.assert_array_equal(np_of(kr), _ggml_rows(k[pos0:pos0 + n], cfg.quant_variant),
                                          err_msg=f"K seq {s} [{pos0}, {pos0 + n})")
            np.testing.assert_array_equal(np_of(vr), _ggml_rows(v[pos0:pos0 + n], cfg.quant_variant),
                                          err_msg=f"V seq {s} [{pos0}, {pos0 + n})")
    kr, vr = qsa.export_rows_q8_0(dev, 0, 5, 7, v=False)
    assert vr is None and kr.shape == (7, rb)
    assert qsa.read_status(dev) == 0


@pytest.mark.parametrize("cfg", [BASELINE, TINY, G12])
def test_import_leaves_the_bytes_an_append_leaves(cfg):
    L = 300
    rng = np.random.default_rng(901)
    k, v = kv_rows(rng, L, cfg)
    pps = L // cfg.page_tokens + 2
    dev, host = make_pair(cfg, 2, pps, seed=17, spare=1)          # a different page permutation
    pos = np.arange(L, dtype=np.int32)
    assert host.append(k, v, pos, np.full(L, 1, np.int32)) == 0
    kr = torch.from_numpy(_ggml_rows(k, cfg.quant_variant)).cuda()
    vr = torch.from_numpy(_ggml_rows(v, cfg.quant_variant)).cuda()
    for _ in range(2):                                            # idempotent
        qsa.import_rows_q8_0(dev, 1, 0, kr, vr)
        torch.cuda.synchronize()
        np.testing.assert_array_equal(np_of(dev.k_pages), host.k_pages)
        np.testing.assert_array_equal(np_of(dev.v_pages), host.v_pages)


def test_any_bytes_round_trip():
    cfg = BASELINE
    dev, _ = make_pair(cfg, 1, 2, seed=3)
    rb = cfg_of(cfg).row_bytes()
    rng = np.random.default_rng(902)
    for pos0, n in ((0, 512), (37, 100), (511, 1)):
        kr = torch.from_numpy(rng.integers(0, 256, (n, rb), dtype=np.uint8)).cuda()
        vr = torch.from_numpy(rng.integers(0, 256, (n, rb), dtype=np.uint8)).cuda()
        qsa.import_rows_q8_0(dev, 0, pos0, kr, vr)
        k2, v2 = qsa.export_rows_q8_0(dev, 0, pos0, n)
        torch.cuda.synchronize()
        assert torch.equal(k2, kr) and torch.equal(v2, vr)


def test_bad_page_entries_set_the_status_bit():
    cfg = BASELINE
    pt = torch.tensor([[0, 7, 1]], dtype=torch.int32)               # page 7 outside a pool of 2
    dev = qsa.KvCache.allocate(cfg_of(cfg), 1, 3, page_table=pt, n_phys_pages=2)
    kr, vr = qsa.export_rows_q8_0(dev, 0, 200, 100)                  # rows 256.. hit the bad page
    torch.cuda.synchronize()
    assert qsa.read_status(dev) & _lib.STATUS_PAGE_RANGE
    qsa.import_rows_q8_0(dev, 0, 200, kr, vr)
    torch.cuda.synchronize()
    assert qsa.read_status(dev) & _lib.STATUS_PAGE_RANGE


def test_snapshot_reproduces_selection_and_attention(tmp_path):
    cfg = BASELINE
    L = 9000
    rng = np.random.default_rng(903)
    pps = L // 256 + 2
    a, host = make_pair(cfg, 1, pps, seed=21)
    fill(a, host, rng, [L])
    path = str(tmp_path / "layer.kv")
    h = snapshot.save_snapshot(a, path, 0, L)
    assert h["n_tokens"] == L and h["row_bytes"] == 272
    b, _ = make_pair(cfg, 2, pps, seed=22)                           # other pages, load into sequence 1
    assert snapshot.load_snapshot(b, path, 1) == L
    nw = L // cfg.block_tokens
    np.testing.assert_array_equal(np_of(b.pooled)[1, :, :nw], np_of(a.pooled)[0, :, :nw])
    q = torch.from_numpy(rng.standard_normal((1, 16, 128), dtype=np.float32)).cuda()
    outs = []
    for cache, s in ((a, 0), (b, 1)):
        n_seq = cache.n_seq
        qq = q.repeat(n_seq, 1, 1).contiguous()
        lens = torch.full((n_seq,), L, dtype=torch.int32, device="cuda")
        if n_seq == 2:
            lens[0] = 1                                                  # sequence 0 of b is empty but valid
        ws = qsa.Workspace(cfg_of(cfg), n_seq, L)
        sel, nsel = qsa.indexer_topk(cache, qq, lens, L, ws)
        out = qsa.sparse_decode_attn(cache, qq, lens, L, ws, sel=sel, n_sel=nsel)
        torch.cuda.synchronize()
        outs.append((np_of(sel)[s], np_of(nsel)[s], np_of(out)[s]))
    np.testing.assert_array_equal(outs[0][1], outs[1][1])
    for g in range(cfg.n_head_kv):
        np.testing.assert_array_equal(outs[0][0][g, :outs[0][1][g]], outs[1][0][g, :outs[1][1][g]])
    assert outs[0][2].tobytes() == outs[1][2].tobytes()
