"""Independent restatements that pin the C oracle.

Written from the mathematics (and numpy's own IEEE routines), not from the
oracle's code: numpy float16 for the fp16 scale, numpy rint / a float64
half-away rounding for q8_0, exact rational arithmetic for fmaf, a plain sort
for the selection, float64 textbook softmax for attention.  Small sizes only.
"""
from __future__ import annotations

from dataclasses import dataclass
from fractions import Fraction

import numpy as np


@dataclass(frozen=True)
class Cfg:
    """Field names match qwfnfer_amd.qsa.QsaConfig (usable with oracle.shape_of)."""
    n_head: int = 16
    n_head_kv: int = 2
    head_dim: int = 128
    block_tokens: int = 64
    page_tokens: int = 256
    top_k_blocks: int = 64
    sink_blocks: int = 1
    local_tokens: int = 512
    relu_per_head: int = 0
    shared_selection: int = 0
    quant_variant: int = 0
    topk_counts_forced: int = 0
    kv_type: int = 0
    kv_round_f16: int = 0

    @property
    def group(self):
        return self.n_head // self.n_head_kv


BASELINE = Cfg()
TINY = Cfg(n_head=4, n_head_kv=2, head_dim=128, block_tokens=4, page_tokens=64, top_k_blocks=5,
           sink_blocks=1, local_tokens=9)


# ---- q8_0 -------------------------------------------------------------------

def q8_block_ref(x: np.ndarray, variant: int):
    """ggml q8_0 for one 32-value block (finite inputs)."""
    x = np.asarray(x, dtype=np.float32)
    amax = np.float32(np.max(np.abs(x)))
    d = np.float32(amax / np.float32(127.0))
    d16 = np.array([d], dtype=np.float32).astype(np.float16).view(np.uint16)[0]
    if variant == 0:
        idv = np.float32(np.float32(127.0) / amax) if amax != 0 else np.float32(0)
        v = (x * idv).astype(np.float32)
        q = np.rint(v)
    else:
        idv = np.float32(np.float32(1.0) / d) if d != 0 else np.float32(0)
        v = (x * idv).astype(np.float32)
        a = np.floor(np.abs(v).astype(np.float64) + 0.5)
        q = np.sign(v) * a
    q = np.clip(q, -128, 127).astype(np.int8)
    return int(d16), q


def dequant_ref(d16: int, q: np.ndarray) -> np.ndarray:
    d = np.array([d16], dtype=np.uint16).view(np.float16).astype(np.float32)[0]
    return (d * q.astype(np.float32)).astype(np.float32)


# ---- exact fmaf -----------------------------------------------------------------

def round_f32(x: Fraction) -> np.float32:
    """Nearest binary32 to an exact rational, ties to even (subnormals kept)."""
    if x == 0:
        return np.float32(0.0)
    sign = -1 if x < 0 else 1
    a = abs(x)
    e = a.numerator.bit_length() - a.denominator.bit_length()
    if Fraction(2) ** e > a:
        e -= 1
    while Fraction(2) ** (e + 1) <= a:
        e += 1
    e = max(e, -126)                       # subnormal range shares 2^-149 units
    unit = Fraction(2) ** (e - 23)
    m = a / unit
    fl = m.numerator // m.denominator
    rem = m - fl
    if rem > Fraction(1, 2) or (rem == Fraction(1, 2) and fl % 2 == 1):
        fl += 1
    val = Fraction(fl) * unit
    if val >= Fraction(2) ** 128:
        return np.float32(sign * np.inf)
    return np.float32(sign * float(val))


def fmaf_exact(a, b, c) -> np.float32:
    return round_f32(Fraction(float(a)) * Fraction(float(b)) + Fraction(float(c)))


def block_score_exact(q_group: np.ndarray, p: np.ndarray, relu: bool) -> np.float32:
    """The score order of the HIP indexer: per head four fmaf chains over the
    dims with (d//4) % 4 == j, combined (c0+c1)+(c2+c3); heads summed in order."""
    G, hd = q_group.shape
    score = None
    for h in range(G):
        c = []
        for j in range(4):
            acc = np.float32(0.0)
            for d in range(hd):
                if (d // 4) % 4 == j:
                    acc = fmaf_exact(q_group[h, d], p[d], acc)
            c.append(acc)
        dot = np.float32(np.float32(c[0] + c[1]) + np.float32(c[2] + c[3]))
        if relu:
            dot = dot if dot > 0 else np.float32(0.0)
        score = dot if score is None else np.float32(score + dot)
    return score


# ---- selection -------------------------------------------------------------------

def select_ref(cfg: Cfg, scores: np.ndarray, seq_len: int) -> np.ndarray:
    """Kept blocks from the definition: F = sink blocks U blocks meeting the last
    local_tokens tokens; E = whole blocks not in F; F U top-k(E) by (score desc,
    index asc), NaN lowest; ascending.  k = top_k_blocks, less |F| when
    topk_counts_forced."""
    bt = cfg.block_tokens
    last = seq_len - 1
    blocks = range(last // bt + 1)
    if cfg.top_k_blocks <= 0:
        return np.array(list(blocks), dtype=np.int32)
    lo = last - cfg.local_tokens + 1
    F = {b for b in blocks if b < cfg.sink_blocks or b * bt + bt - 1 >= lo}
    E = [b for b in blocks if (b + 1) * bt <= seq_len and b not in F]
    k = cfg.top_k_blocks
    if getattr(cfg, "topk_counts_forced", 0):
        k = max(k - len(F), 0)
    if len(E) > k:
        def key(b):
            s = float(scores[b])
            return (1, 0.0, b) if s != s else (0, -s, b)
        E = sorted(E, key=key)[:k]
    return np.array(sorted(F | set(E)), dtype=np.int32)


# ---- attention --------------------------------------------------------------------

def attention_ref(q: np.ndarray, K: np.ndarray, V: np.ndarray) -> np.ndarray:
    """Softmax attention of one query head over rows K, V (float64)."""
    lg = K.astype(np.float64) @ q.astype(np.float64) / np.sqrt(q.shape[-1])
    lg -= lg.max()
    p = np.exp(lg)
    p /= p.sum()
    return p @ V.astype(np.float64)
