"""The prefill scoring bound checked on the hardware: the approximate
matrix-core scores of k_pf_approx (qwfn_qsa_test_prefill_scores, through the C
ABI) against float64 dot products, on the adversarial cases of
tests/test_prefill_bound.py -- six decades of element scale, cancelling dots,
one-hot heads, heads of very different magnitude -- for the BASELINE shape
(8 heads a KV head, summed) and a relu'd 4-head group (the checkpoint
indexer's rule).  The prefill selection is exact because

    |approx - exact_fp32| <= kPaRel * sum_h |q_h| * |p| + kPaAbs,

and exact_fp32 (the indexer's fmaf chains) is within 80 * 2^-24 * sum_h |q_h|
|p| of the float64 dot, so the test asks the approximate scores to lie within
(kPaRel - 80 * 2^-24) * sum_h |q_h| * |p| + kPaAbs of the float64 dot: what the
kernel's bound needs, measured instead of modelled."""
import ctypes as C

import numpy as np
import pytest

from test_prefill_bound import KPA_ABS, KPA_REL

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")


def _blocks(rng, n_blk, hd):
    p = rng.standard_normal((n_blk, hd))
    kind = np.arange(n_blk) % 5
    wide = kind == 1                               # six decades of element scale
    p[wide] *= np.exp(rng.uniform(np.log(1e-3), np.log(1e3), (wide.sum(), hd)))
    spike = kind == 3                              # one element dominating
    p[spike] *= 1e-4
    p[np.where(spike)[0], rng.integers(0, hd, spike.sum())] = rng.choice([-1e3, 1e3], spike.sum())
    scaled = kind == 4                             # whole rows of very different magnitude
    p[scaled] *= 10.0 ** rng.integers(-6, 6, (scaled.sum(), 1))
    return p, kind


def _queries(rng, n_q, n_head, hd):
    q = rng.standard_normal((n_q, n_head, hd))
    kind = np.arange(n_q) % 4
    q[kind == 1] *= np.exp(rng.uniform(np.log(1e-3), np.log(1e3), ((kind == 1).sum(), n_head, hd)))
    one = np.where(kind == 2)[0]                   # one large element a head, the rest tiny
    q[one] *= 1e-4
    for i in one:
        q[i, np.arange(n_head), rng.integers(0, hd, n_head)] = rng.choice([-1e3, 1e3], n_head)
    q[kind == 3] *= 10.0 ** rng.integers(-6, 6, ((kind == 3).sum(), n_head, 1))
    return q


@pytest.mark.parametrize("n_head,relu", [(16, 0), (8, 1)])
def test_prefill_approx_scores_within_bound_on_gpu(n_head, relu):
    from qwfnfer_amd import _lib, qsa

    cfg = qsa.QsaConfig(n_head=n_head, relu_per_head=relu)
    G, hd, hkv = cfg.group, cfg.head_dim, cfg.n_head_kv
    rng = np.random.default_rng(77 + relu)
    n_blk, n_q = 1024, 128
    pps = n_blk * cfg.block_tokens // cfg.page_tokens
    cache = qsa.KvCache.allocate(cfg, 1, pps)
    p, kind = _blocks(rng, n_blk, hd)
    p = np.stack([p, _blocks(rng, n_blk, hd)[0]])                    # [hkv][n_blk][hd]
    q = _queries(rng, n_q, n_head, hd)
    # cancelling dots: every fifth block (kind 2) nearly orthogonal to the
    # group sum of one query, so that pair's score cancels to a few ulps
    for gh in range(hkv):
        for b in np.where(kind == 2)[0]:
            s = q[b % n_q, gh * G:(gh + 1) * G].sum(0)
            p[gh, b] -= (s @ p[gh, b]) / (s @ s) * s
    p32 = p.astype(np.float32)
    q32 = q.astype(np.float32)
    cache.pooled[0].copy_(torch.from_numpy(p32))
    nb_cap = n_blk + 64
    scores = torch.full((n_q, hkv, nb_cap), float("nan"), device="cuda")
    pnorm = torch.full((hkv, nb_cap), float("nan"), device="cuda")
    qd = torch.from_numpy(q32).cuda()
    s = cfg.shape()
    print(f"\n  prefill bound: n_head {n_head} relu {relu}, {n_q} queries x {n_blk} blocks", flush=True)
    _lib.call("qwfn_qsa_test_prefill_scores", C.byref(s), C.byref(cache.view()), qd.data_ptr(), n_q, 0, n_blk,
              scores.data_ptr(), pnorm.data_ptr(), nb_cap, torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    got = scores.cpu().numpy().astype(np.float64)
    pn = pnorm.cpu().numpy().astype(np.float64)
    sink = cfg.sink_blocks
    pd = p32.astype(np.float64)
    qd64 = q32.astype(np.float64)
    norm_p = np.linalg.norm(pd, axis=2)                              # [hkv][n_blk]
    worst = 0.0
    for gh in range(hkv):
        qg = qd64[:, gh * G:(gh + 1) * G]                            # [n_q][G][hd]
        dots = np.einsum("qgd,bd->qgb", qg, pd[gh])                  # float64
        exact = np.maximum(dots, 0).sum(1) if relu else dots.sum(1)  # [n_q][n_blk]
        qn = np.linalg.norm(qg, axis=2).sum(1)                       # [n_q]
        tol = (KPA_REL - 80 * 2.0 ** -24) * qn[:, None] * norm_p[gh][None, :] + KPA_ABS
        a = got[:, gh, sink:n_blk]
        err = np.abs(a - exact[:, sink:n_blk])
        assert np.isfinite(a).all(), "a score was not written"
        bad = err > tol[:, sink:n_blk]
        assert not bad.any(), (f"KV head {gh}: {int(bad.sum())} scores outside the bound, worst "
                               f"{float((err / tol[:, sink:n_blk]).max()):.3f} of it")
        worst = max(worst, float((err / tol[:, sink:n_blk]).max()))
        # the key norms the refinement uses: rounded up, by at most 2^-13
        nr = pn[gh, sink:n_blk]
        assert (nr >= norm_p[gh, sink:n_blk]).all(), "a key norm was rounded down"
        assert (nr <= norm_p[gh, sink:n_blk] * (1 + 2.0 ** -12)).all(), "a key norm is too large"
    print(f"  worst |approx - exact| / bound = {worst:.3f}", flush=True)
    assert worst > 1e-3                     # the cases reach the bound's scale, not only exact zeros
