"""qwfn_qsa_time_next_call: a fused decode call with its three launches timed
(hipExtLaunchKernel with the armed events) gives the same outputs,
selections, cache bytes and pooled keys as the same call unarmed, on two
identical caches, and every armed pair of events holds a kernel's duration.
The two-call path is armed the same way, per call."""
import numpy as np
import pytest
import torch

from _gpu import fill, make_pair
from _refs import BASELINE
from qwfnfer_amd import qsa

pytestmark = pytest.mark.gpu


def _twin(dev):
    c = qsa.KvCache.allocate(dev.cfg, dev.n_seq, dev.pages_per_seq, page_table=dev.page_table.cpu(),
                             n_phys_pages=dev.n_phys_pages)
    c.k_pages.copy_(dev.k_pages)
    c.v_pages.copy_(dev.v_pages)
    c.pooled.copy_(dev.pooled)
    return c


def _events():
    ev = {k: (torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
          for k in qsa.TIMED_KERNELS}
    for a, b in ev.values():           # torch creates the handles at the first record
        a.record()
        b.record()
    return ev


@pytest.mark.parametrize("fused", [True, False])
def test_timed_call_matches_untimed_call(fused):
    cfg = BASELINE
    rng = np.random.default_rng(910)
    lengths = [12000, 3000]
    dev, host = make_pair(cfg, 2, 64, seed=910)
    fill(dev, host, rng, lengths)
    twin = _twin(dev)
    q = torch.from_numpy(rng.standard_normal((2, cfg.n_head, cfg.head_dim), dtype=np.float32)).cuda()
    kn = torch.from_numpy(rng.standard_normal((2, cfg.n_head_kv, cfg.head_dim), dtype=np.float32)).cuda()
    vn = torch.from_numpy(rng.standard_normal((2, cfg.n_head_kv, cfg.head_dim), dtype=np.float32)).cuda()
    sl = torch.tensor([L + 1 for L in lengths], dtype=torch.int32, device="cuda")
    max_len = 16000
    msel = dev.cfg.max_selected(max_len)
    outs = []
    ev = _events()
    torch.cuda.synchronize()
    for c, timed in ((dev, False), (twin, True)):
        ws = qsa.Workspace(dev.cfg, 2, max_len)
        out = torch.full((2, cfg.n_head, cfg.head_dim), float("nan"), device="cuda")
        sel = torch.full((2, cfg.n_head_kv, msel), -7, dtype=torch.int32, device="cuda")
        nsel = torch.full((2, cfg.n_head_kv), -7, dtype=torch.int32, device="cuda")
        if fused:
            if timed:
                qsa.time_next_call(ev)
            qsa.sparse_attn_decode(c, q, kn, vn, sl, max_len, ws, out=out, sel=sel, n_sel=nsel)
        else:
            if timed:
                qsa.time_next_call({"indexer": ev["indexer"]})
            qsa.decode_append_select(c, q, kn, vn, sl, max_len, ws, sel, nsel)
            if timed:
                qsa.time_next_call({k: ev[k] for k in ("attention", "merge")})
            qsa.sparse_decode_attn(c, q, sl, max_len, ws, sel, nsel, out=out)
        torch.cuda.synchronize()
        assert qsa.read_status(c) == 0
        outs.append((out.cpu(), sel.cpu(), nsel.cpu(), c.k_pages.cpu(), c.v_pages.cpu(), c.pooled.cpu()))
    for a, b in zip(*outs):
        assert torch.equal(a, b)
    for k, (a, b) in ev.items():
        ms = a.elapsed_time(b)
        print(f"{k}: {ms * 1e3:.2f} us", flush=True)
        assert 0.0 < ms < 50.0, (k, ms)
