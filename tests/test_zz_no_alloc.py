"""qwfn_sparse_attn_decode_noalloc (the library's per-device scratch array as
the workspace) against qwfn_sparse_attn_decode with a caller workspace: two
calls in a row on each of two identical caches, the second call smaller
(fewer sequences, a shorter max_seq_len, so the array is laid out anew);
outputs, selections, cache bytes and pooled keys must be identical."""
import numpy as np
import pytest
import torch

from _gpu import cfg_of, fill, kv_rows, make_pair, np_of
from _refs import BASELINE
from qwfnfer_amd import _lib, qsa

pytestmark = pytest.mark.gpu


def _twin(dev):
    """A second device cache holding the same bytes under the same page table."""
    c = qsa.KvCache.allocate(dev.cfg, dev.n_seq, dev.pages_per_seq, page_table=dev.page_table.cpu(),
                             n_phys_pages=dev.n_phys_pages)
    c.k_pages.copy_(dev.k_pages)
    c.v_pages.copy_(dev.v_pages)
    c.pooled.copy_(dev.pooled)
    return c


def test_noalloc_matches_workspace_call():
    cfg = BASELINE
    c = cfg_of(cfg)
    rng = np.random.default_rng(900)
    lengths = [20000, 7000, 3000]
    dev, host = make_pair(cfg, 3, 160, seed=900)          # 40,960 tokens a sequence
    fill(dev, host, rng, lengths)
    twin = _twin(dev)
    torch.cuda.synchronize()
    calls = [(3, [20001, 7001, 3001], 40000),          # the first call, then a smaller one
             (1, [20002], 20002)]
    inputs = []
    for n_seq, lens, max_len in calls:
        q = torch.from_numpy(rng.standard_normal((n_seq, cfg.n_head, cfg.head_dim), dtype=np.float32)).cuda()
        kn, vn = kv_rows(rng, n_seq, cfg)
        seq_len = torch.tensor(lens, dtype=torch.int32, device="cuda")
        msel = c.max_selected(max_len)
        bufs = [dict(out=torch.empty((n_seq, cfg.n_head, cfg.head_dim), device="cuda"),
                     sel=torch.full((n_seq, cfg.n_head_kv, msel), -1, dtype=torch.int32, device="cuda"),
                     nsel=torch.zeros((n_seq, cfg.n_head_kv), dtype=torch.int32, device="cuda"))
                for _ in range(2)]
        inputs.append((q, torch.from_numpy(kn).cuda(), torch.from_numpy(vn).cuda(), seq_len, max_len, bufs))
    # the caller-workspace entry point on one cache ...
    for q, kn, vn, seq_len, max_len, bufs in inputs:
        ws = qsa.Workspace(c, seq_len.numel(), max_len)
        b = bufs[0]
        qsa.sparse_attn_decode(dev, q, kn, vn, seq_len, max_len, ws, out=b["out"], sel=b["sel"], n_sel=b["nsel"])
    # ... and the no-alloc one, two calls in a row, on its twin
    torch.cuda.synchronize()
    for q, kn, vn, seq_len, max_len, bufs in inputs:
        b = bufs[1]
        qsa.sparse_attn_decode_noalloc(twin, q, kn, vn, seq_len, max_len, b["out"], sel=b["sel"], n_sel=b["nsel"])
    torch.cuda.synchronize()
    for i, (_, _, _, seq_len, _, bufs) in enumerate(inputs):
        a, b = bufs
        assert torch.equal(a["nsel"], b["nsel"]), f"call {i}: selection counts differ"
        assert torch.equal(a["sel"], b["sel"]), f"call {i}: selections differ"
        assert torch.equal(a["out"], b["out"]), f"call {i}: outputs differ"
        assert int(a["nsel"].min()) > 0
    assert torch.equal(dev.k_pages, twin.k_pages) and torch.equal(dev.v_pages, twin.v_pages)
    assert torch.equal(dev.pooled, twin.pooled)
    assert qsa.read_status(dev) == 0 and qsa.read_status(twin) == 0


def test_noalloc_rejects_what_the_array_cannot_hold():
    cfg = BASELINE
    dev, _ = make_pair(cfg, 16, 1)
    n_seq, max_len = 16, 1 << 20                        # 15.4 MiB of workspace
    q = torch.zeros((n_seq, cfg.n_head, cfg.head_dim), device="cuda")
    kn = torch.zeros((n_seq, cfg.n_head_kv, cfg.head_dim), device="cuda")
    out = torch.empty_like(q)
    seq_len = torch.ones(n_seq, dtype=torch.int32, device="cuda")
    with pytest.raises(_lib.QsaError) as ei:
        qsa.sparse_attn_decode_noalloc(dev, q, kn, kn, seq_len, max_len, out)
    assert ei.value.code == _lib.QWFN_ERANGE
