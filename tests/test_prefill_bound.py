"""The error bound of the prefill's matrix-core scoring (k_pf_approx /
k_pf_refine in qwfnfer_amd/csrc/qsa_kernels.hip), checked on a numpy model of
both arithmetics: the approximate score -- query and key each scaled by a power
of two into [2^14, 2^15), rounded to fp16, products summed in fp32, relu'd
heads summed, scaled back -- and the exact score in the decode indexer's order
(four fmaf chains over the dims with (d/4)%4 == j, (c0+c1)+(c2+c3), heads in
order; src/qwfn_graph.cpp:282-305 restated by oracle/qsa_oracle.c).  The
selection's exactness rests on |approx - exact| <= kPaRel * sum_h |q_h| * |p| +
kPaAbs; these cases aim at it: wide dynamic ranges, cancelling sums, relu, and
the fp32 accumulation order taken both ways.  CPU only."""
import os
import re

import numpy as np
import pytest

SRC = os.path.join(os.path.dirname(__file__), os.pardir, "qwfnfer_amd", "csrc", "qsa_kernels.hip")


def _constant(name):
    text = open(SRC).read()
    m = re.search(r"constexpr float %s = ([0-9.eE+-]+)f;" % name, text)
    assert m, name
    return float(m.group(1))


KPA_REL = _constant("kPaRel")
KPA_ABS = _constant("kPaAbs")


def _shift(m):
    """15 - e for m = f 2^e, f in [0.5, 1) (0 for m = 0)."""
    return np.where(m > 0, 15 - np.frexp(m)[1], 0)


def _fp32_chain_sum(terms, reverse=False):
    acc = np.float32(0.0)
    for t in (terms[::-1] if reverse else terms):
        acc = np.float32(acc + np.float32(t))
    return acc


def chain_heads(hd, g, relu):
    """Heads whose products share one fp32 accumulator (pa_chain in the
    kernel): one with relu, else as many as keep a chain at 256 products."""
    return 1 if relu or hd >= 256 else min(g, 256 // hd)


def approx_score(q, p, relu, reverse=False):
    """q [G, HD] fp32, p [HD] fp32 -> the approximate score (fp32)."""
    G, HD = q.shape
    ch = chain_heads(HD, G, relu)
    qe = int(_shift(np.abs(q).max()))
    pe = int(_shift(np.abs(p).max()))
    qh = np.ldexp(q, qe).astype(np.float16).astype(np.float32)
    ph = np.ldexp(p, pe).astype(np.float16).astype(np.float32)
    tot = np.float32(0.0)
    for h0 in range(0, G, ch):
        prods = (qh[h0:h0 + ch].astype(np.float64) * ph.astype(np.float64)).astype(np.float32).ravel()  # exact
        d = _fp32_chain_sum(prods, reverse)
        if relu:
            d = max(d, np.float32(0.0))
        tot = np.float32(tot + d)
    return np.float32(np.ldexp(np.float64(tot), -(qe + pe)))


def exact_score(q, p, relu):
    """The decode indexer's order, fmaf emulated by an exact product and one
    fp32 rounding of each sum."""
    G, HD = q.shape
    score = np.float32(0.0)
    for h in range(G):
        c = [np.float32(0.0)] * 4
        for d16 in range(HD // 16):
            for j in range(4):
                for e in range(4):
                    d = 16 * d16 + 4 * j + e
                    c[j] = np.float32(np.float64(c[j]) + np.float64(q[h, d]) * np.float64(p[d]))
        dot = np.float32(np.float32(c[0] + c[1]) + np.float32(c[2] + c[3]))
        if relu:
            dot = max(dot, np.float32(0.0))
        score = dot if h == 0 else np.float32(score + dot)
    return score


def bound(q, p):
    qn = sum(float(np.linalg.norm(q[h].astype(np.float64))) for h in range(q.shape[0]))
    return KPA_REL * qn * float(np.linalg.norm(p.astype(np.float64))) + KPA_ABS


def _cases(rng, n):
    G, HD = 8, 128
    for i in range(n):
        kind = i % 5
        q = rng.standard_normal((G, HD)).astype(np.float32)
        p = rng.standard_normal(HD).astype(np.float32)
        if kind == 1:            # six decades of element scale in both operands
            q *= np.exp(rng.uniform(np.log(1e-3), np.log(1e3), (G, HD))).astype(np.float32)
            p *= np.exp(rng.uniform(np.log(1e-3), np.log(1e3), HD)).astype(np.float32)
        elif kind == 2:          # a cancelling dot: p nearly orthogonal to every head
            p -= (q.sum(0) @ p) / (q.sum(0) @ q.sum(0)) * q.sum(0)
        elif kind == 3:          # one large element per head, the rest tiny
            q *= 1e-4
            q[np.arange(G), rng.integers(0, HD, G)] = rng.choice([-1e3, 1e3], G)
        elif kind == 4:          # heads of very different magnitude
            q *= np.float32(10.0) ** rng.integers(-6, 6, (G, 1))
        yield q.astype(np.float32), p.astype(np.float32)


@pytest.mark.parametrize("relu", [False, True])
def test_approx_score_within_bound(relu):
    rng = np.random.default_rng(1234 + relu)
    worst = 0.0
    for q, p in _cases(rng, 150):
        s = float(exact_score(q, p, relu))
        e = bound(q, p)
        for rev in (False, True):
            a = float(approx_score(q, p, relu, rev))
            assert abs(a - s) <= e, (a, s, e)
            worst = max(worst, abs(a - s) / e)
    assert worst < 0.5                      # the bound is not drawn tight around these cases


def test_bound_fails_without_the_rounding_term():
    """A plausible mistake -- a bound of only the fp32 accumulation terms (no
    fp16 rounding) -- is caught by the same cases."""
    rng = np.random.default_rng(99)
    missed = 0
    for q, p in _cases(rng, 60):
        s = float(exact_score(q, p, False))
        a = float(approx_score(q, p, False))
        qn = sum(float(np.linalg.norm(q[h].astype(np.float64))) for h in range(8))
        small = 2.0e-5 * qn * float(np.linalg.norm(p.astype(np.float64)))
        missed += abs(a - s) > small
    assert missed > 0


# (head_dim, group) pairs with the matrix-core scoring: every instantiation
# of qsa_kernels.hip's QWFN_FOR_EACH_SHAPE whose group * head_dim <= 1024
SHAPES = [(128, 8), (128, 4), (128, 2), (64, 8)]


def test_kparel_covers_the_budget_of_every_shape():
    """kPaRel against its terms, per instantiated shape and relu flag: fp16
    rounding of both operands (2 * 2^-11 + 2^-22), the matrix cores' fp32 sums
    with one accumulator a chain of CH heads (CH * HD - 1 adds) and the G / CH
    chain sums (G / CH - 1 adds), the exact score's own rounding (80 * 2^-24),
    with 5 % to spare.  A single accumulator over all G * HD products (the
    mistake of summing every head in one chain) would need (G * HD - 1) * 2^-24
    and is caught at G * HD = 1024."""
    u = 2.0 ** -24
    text = open(SRC).read()
    shapes = re.search(r"#define QWFN_FOR_EACH_SHAPE\(X\) (.*)", text).group(1)
    inst = {(int(a), int(b)) for a, b in re.findall(r"X\((\d+), (\d+), \d+\)", shapes)}
    assert set(SHAPES) == {(h, g) for h, g in inst if h * g <= 1024}
    assert chain_heads(128, 8, False) == 2 and chain_heads(64, 8, False) == 4 and chain_heads(128, 8, True) == 1
    for hd, g in SHAPES:
        for relu in (False, True):
            ch = chain_heads(hd, g, relu)
            assert g % ch == 0
            need = 2 * 2.0 ** -11 + 2.0 ** -22 + (ch * hd - 1 + g // ch - 1) * u + 80 * u
            assert KPA_REL >= 1.05 * need, (hd, g, relu, need)
    one_chain = 2 * 2.0 ** -11 + 2.0 ** -22 + (1024 - 1) * u + 80 * u
    assert KPA_REL < 1.05 * one_chain


@pytest.mark.parametrize("relu", [False, True])
def test_approx_score_within_bound_at_1024_products(relu):
    """Eight heads of 128 (G * HD = 1024, the largest group of the matrix-core
    scoring), each chain's products (one head with relu, two heads' 256
    without) summed in one fp32 chain taken in both orders, against the exact
    order."""
    rng = np.random.default_rng(4321 + relu)
    for q, p in _cases(rng, 60):
        s = float(exact_score(q, p, relu))
        e = bound(q, p)
        for rev in (False, True):
            assert abs(float(approx_score(q, p, relu, rev)) - s) <= e
