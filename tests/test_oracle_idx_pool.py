"""The checkpoint indexer's pooled keys in the oracle (qwfn_oracle_idx_pool_block)
against what the mathematics fixes, independently of its loop:
  - block 0 sits at position 0, where the rotation is the identity: the key is
    RMSNorm(mean of the members) * k_norm, checked against numpy float64;
  - a block whose members are one basis vector e_i is rotated by the closed
    form: after RMSNorm it is sqrt(D) * w_i e_i, and the pair (i, i + nd/2)
    turns by ggml's fp32 angle -- pos times theta_scale = base^(-2/nd) (the
    float64 power rounded to float32), i times over, each product rounded to
    float32 by numpy -- (dims >= nd stay), so a wrong pairing (adjacent
    instead of split halves), a sign, the exponent, the position (b instead
    of b * block_tokens) or the exact float64 angle in place of the fp32 one
    fails;
  - the rotation keeps every pair's length and leaves dims >= nd alone;
  - the shared selection over the indexer scores is the definition's.
Each comparison allows one fp16 ulp: the stored key is fp16-rounded."""
import numpy as np
import pytest

from oracle import oracle as O
from _ckpt import CKPT, ICfg, oracle_select, scoring_cfg
from _refs import block_score_exact, select_ref


def f16_close(got, want):
    want = np.asarray(want, np.float64)
    tol = np.maximum(np.abs(want) * 2.0 ** -10, 2.0 ** -24) + 1e-6 * np.abs(want)
    err = np.abs(np.asarray(got, np.float64) - want)
    assert (err <= tol).all(), f"max err {err.max():.3g} (tol at worst {tol[np.argmax(err - tol)]:.3g})"


@pytest.mark.parametrize("D,nd,bt", [(128, 64, 4), (64, 64, 2), (256, 32, 8)])
def test_block0_is_the_float64_rmsnorm_of_the_mean(D, nd, bt):
    rng = np.random.default_rng(D + nd + bt)
    icfg = ICfg(idx_dim=D, rope_dim=nd, rms_eps=1e-6)
    cfg = CKPT.__class__(**{**CKPT.__dict__, "block_tokens": bt})
    m = (rng.standard_normal((bt, D)) * 3).astype(np.float16)
    w = rng.uniform(0.5, 1.5, D).astype(np.float32)
    got = O.idx_pool_block(cfg, icfg, m, w, 0)
    x = m.astype(np.float64).mean(0)
    want = x / np.sqrt(np.mean(x * x) + 1e-6) * w
    f16_close(got, want)


@pytest.mark.parametrize("b", [0, 1, 7, 1000, 40959])
@pytest.mark.parametrize("i", [0, 5, 31, 32, 40, 63, 64, 127])
def test_basis_vector_rotates_by_the_closed_form(b, i):
    D, nd, base, bt = 128, 64, 10000000.0, 4
    icfg = ICfg(idx_dim=D, rope_dim=nd, rope_freq_base=base, rms_eps=0.0)
    m = np.zeros((bt, D), np.float16)
    m[:, i] = 1.0
    w = np.ones(D, np.float32)
    got = O.idx_pool_block(CKPT, icfg, m, w, b)
    want = np.zeros(D)
    amp = np.sqrt(D)
    pos = b * bt
    h = nd // 2
    if i >= nd:
        want[i] = amp
    else:
        pair = i % h
        th = ggml_theta(pos, pair, base, nd)
        if i < h:        # (x0, x1) = (amp, 0)
            want[i], want[i + h] = amp * np.cos(th), amp * np.sin(th)
        else:            # (x0, x1) = (0, amp)
            want[i - h], want[i] = -amp * np.sin(th), amp * np.cos(th)
    f16_close(got, want)


def ggml_theta(pos, pair, base, nd):
    """ggml's rope angle of pair `pair`: float32(pos) times float32(base **
    (-2 / nd)), `pair` times over, each product rounded to float32."""
    scale = np.float32(base ** (-2.0 / nd))
    th = np.float32(pos)
    for _ in range(pair):
        th = np.float32(th * scale)
    return float(th)


def test_fp32_angle_is_observable():
    """At long positions the fp32 angle and the exact float64 one put the
    stored key more than the comparison's tolerance apart, so the closed-form
    test above tells them apart."""
    D, nd, base, bt, b = 128, 64, 10000000.0, 4, 40959
    icfg = ICfg(idx_dim=D, rope_dim=nd, rope_freq_base=base, rms_eps=0.0)
    amp, pos = np.sqrt(D), b * bt
    apart = 0
    for i in range(1, nd // 2):
        m = np.zeros((bt, D), np.float16)
        m[:, i] = 1.0
        got = O.idx_pool_block(CKPT, icfg, m, np.ones(D, np.float32), b)
        th = pos * base ** (-2.0 * i / nd)
        exact = np.zeros(D)
        exact[i], exact[i + nd // 2] = amp * np.cos(th), amp * np.sin(th)
        try:
            f16_close(got, exact)
        except AssertionError:
            apart += 1
    assert apart > 0


def test_rotation_keeps_pair_lengths_and_tail_dims():
    rng = np.random.default_rng(5)
    icfg = ICfg()
    m = rng.standard_normal((4, 128)).astype(np.float16)
    w = rng.uniform(0.5, 1.5, 128).astype(np.float32)
    y0 = O.idx_pool_block(CKPT, icfg, m, w, 0).astype(np.float64)
    for b in (3, 999, 30000):
        y = O.idx_pool_block(CKPT, icfg, m, w, b).astype(np.float64)
        np.testing.assert_array_equal(y[64:], y0[64:])
        r0 = y0[:32] ** 2 + y0[32:64] ** 2
        r = y[:32] ** 2 + y[32:64] ** 2
        np.testing.assert_allclose(r, r0, rtol=4e-3, atol=1e-6)


@pytest.mark.parametrize("L", [9, 40, 41, 43, 200])
def test_indexer_selection_over_pooled_keys_is_the_definition(L):
    rng = np.random.default_rng(L)
    cfg = CKPT.__class__(**{**CKPT.__dict__, "top_k_blocks": 7, "page_tokens": 64})
    icfg = ICfg()
    nb = (L + 3) // 4
    pooled = np.zeros((64, 128), np.float32)
    pooled[:nb] = rng.standard_normal((nb, 128)).astype(np.float16).astype(np.float32)
    q = rng.standard_normal((4, 128)).astype(np.float32)
    got = oracle_select(cfg, icfg, pooled, q, L, max_sel=16)
    scores = np.array([block_score_exact(q, pooled[b], True) for b in range(nb)], np.float32)
    np.testing.assert_array_equal(got, select_ref(scoring_cfg(cfg, icfg), scores, L))
