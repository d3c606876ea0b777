"""The q4_0 and fp16 cache types in the oracle, pinned independently of its
loops:
  - q4_0 closed forms: a zero block (d = -0, every nibble 8); a block on the
    exact grid x = 8 - q (d = -1, the nibbles recovered exactly); the extremes
    (m -> 0, -m -> 15 clamped from 16, 0 -> 8); magnitude ties (the first index
    wins, so a leading -m gives a positive d); power-of-two scaling (same
    nibbles, d scaled); the reconstruction bound |x - x'| <= |d| (and
    <= |d|/2 away from the clamp);
  - fp16 cache rows are numpy's float16 casts;
  - the page layouts of both types are bijections onto the quant bytes;
  - append followed by dequant reproduces the closed-form reconstruction."""
import numpy as np
import pytest

from oracle import oracle as O
from _refs import Cfg, TINY


def h(bits):
    return float(np.array([bits], np.uint16).view(np.float16)[0])


def nibbles(qs):
    qs = np.asarray(qs, np.uint8)
    return np.concatenate([qs & 15, qs >> 4]).astype(int)


def test_q4_zero_block():
    d, qs = O.quantize_block_q4_0(np.zeros(32, np.float32))
    assert d == 0x8000                       # 0 / -8 = -0
    assert (qs == 0x88).all()


def test_q4_exact_grid():
    rng = np.random.default_rng(1)
    for _ in range(50):
        q = rng.integers(0, 16, 32)
        q[rng.integers(0, 32)] = 0           # x = 8 somewhere: m = 8, d = -1
        x = (8 - q).astype(np.float32)
        d, qs = O.quantize_block_q4_0(x)
        assert h(d) == -1.0
        np.testing.assert_array_equal(nibbles(qs), q)


@pytest.mark.parametrize("m", [3.0, -3.0, 1e-3, -250.0])
def test_q4_extremes_and_sign(m):
    x = np.zeros(32, np.float32)
    x[5], x[20], x[9] = m, -m, 0.0
    d, qs = O.quantize_block_q4_0(x)
    assert h(d) == pytest.approx(m / -8, rel=1e-3)
    q = nibbles(qs)
    assert q[5] == 0 and q[20] == 15 and q[9] == 8


def test_q4_first_largest_magnitude_wins():
    x = np.zeros(32, np.float32)
    x[1], x[3] = -5.0, 5.0                   # tie of magnitude: index 1 first
    d, qs = O.quantize_block_q4_0(x)
    assert h(d) == 0.625
    q = nibbles(qs)
    assert q[1] == 0 and q[3] == 15
    x[1], x[3] = 5.0, -5.0
    d, qs = O.quantize_block_q4_0(x)
    assert h(d) == -0.625


def test_q4_power_of_two_scaling():
    rng = np.random.default_rng(2)
    for _ in range(30):
        x = rng.standard_normal(32).astype(np.float32)
        d0, q0 = O.quantize_block_q4_0(x)
        for k in (-3, 5):
            d1, q1 = O.quantize_block_q4_0(x * np.float32(2.0 ** k))
            np.testing.assert_array_equal(q1, q0)
            assert h(d1) == h(d0) * 2.0 ** k


def test_q4_reconstruction_bound():
    rng = np.random.default_rng(3)
    for _ in range(500):
        x = (rng.standard_normal(32) * np.exp(rng.uniform(-3, 3))).astype(np.float32)
        d, qs = O.quantize_block_q4_0(x)
        dd = h(d)
        xr = (nibbles(qs) - 8) * dd
        err = np.abs(x.astype(np.float64) - xr)
        # the fp16 rounding of d adds a relative 2^-11 on top of the grid error
        assert (err <= abs(dd) * (1 + 1e-3) + abs(x) * 2e-3).all()
        m = np.argmax(np.abs(x))
        away = np.sign(x) != np.sign(x[m])   # the clamp only bites on the far side
        assert (err[~away] <= abs(dd) * 0.5 * (1 + 1e-3) + abs(x[~away]) * 2e-3).all()


def test_f16_rows_are_numpy_casts():
    rng = np.random.default_rng(4)
    x = (rng.standard_normal(256) * 100).astype(np.float32)
    x[:4] = [65504.0, 1e-8, -0.0, 65520.0]
    got = O.quantize_row_type(x, 2).view(np.uint16)
    with np.errstate(over="ignore"):                 # 65520 rounds to inf, as in the oracle
        want = x.astype(np.float16).view(np.uint16)
    np.testing.assert_array_equal(got, want)


@pytest.mark.parametrize("kv_type", [1, 2])
def test_layout_is_a_bijection(kv_type):
    cfg = Cfg(n_head=16, n_head_kv=2, head_dim=128, page_tokens=128, kv_type=kv_type)
    qbytes = 2 * 128 * (64 if kv_type == 1 else 256)
    seen = np.zeros(qbytes, np.int32)
    for g in range(2):
        for row in range(128):
            for d in range(128):
                o = O.quant_offset(cfg, g, row, d, which=1)
                if kv_type == 1:
                    if d % 32 < 16:              # one byte holds dims d and d + 16
                        seen[o] += 1
                else:
                    seen[o] += 1
                    seen[o + 1] += 1
    assert (seen == 1).all()
    assert O.lib().qwfn_oracle_page_bytes(O.C.byref(O.shape_of(cfg))) == qbytes + (2 * 128 * 4 * 2 if kv_type == 1 else 0)


@pytest.mark.parametrize("kv_type", [1, 2])
@pytest.mark.parametrize("base", ["tiny", "baseline"])
def test_append_dequant_round_trip(kv_type, base):
    cfg = Cfg(**{**(TINY if base == "tiny" else Cfg()).__dict__, "kv_type": kv_type})
    rng = np.random.default_rng(5 + kv_type)
    host = O.HostCache(cfg, 1, 2)
    n = 2 * cfg.page_tokens
    k = (rng.standard_normal((n, cfg.n_head_kv, cfg.head_dim)) * 3).astype(np.float32)
    assert host.append(k, -k, np.arange(n, dtype=np.int32)) == 0
    for t in rng.integers(0, n, 20):
        for g in range(cfg.n_head_kv):
            row = O.quantize_row_type(k[t, g], kv_type)
            if kv_type == 2:
                want = row.view(np.float16).astype(np.float32)
            else:
                want = np.concatenate([(nibbles(row[18 * j + 2:18 * j + 18]) - 8) *
                                       h(row[18 * j:18 * j + 2].view(np.uint16)[0]) for j in range(cfg.head_dim // 32)])
            np.testing.assert_array_equal(host.dequant_row("k", 0, int(t), g), want.astype(np.float32))
