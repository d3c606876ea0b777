"""The oracle's paged layout, append, dequant and pooling, pinned by an
independent offset formula, a bijection check, exact round trips and a numpy
float32 add chain."""
import numpy as np
import pytest

from _refs import BASELINE, TINY, Cfg, dequant_ref, q8_block_ref


def _offsets_ref(cfg, g, row, d, which=0):
    tiles, ch = cfg.page_tokens // 64, cfg.head_dim // 16
    if which and cfg.block_tokens % 64 == 0:       # V quants: dim-major 64-token tiles
        q = ((g * tiles + row // 64) * cfg.head_dim + d) * 64 + row % 64
    else:
        q = ((g * tiles + row // 64) * ch + d // 16) * 1024 + (row % 64) * 16 + d % 16
    qbytes = cfg.n_head_kv * cfg.page_tokens * cfg.head_dim
    s = qbytes + ((g * cfg.page_tokens + row) * (cfg.head_dim // 32) + d // 32) * 2
    return q, s


@pytest.mark.parametrize("which", [0, 1])
@pytest.mark.parametrize("cfg", [BASELINE, TINY, Cfg(head_dim=256, n_head=24, page_tokens=128)])
def test_layout_is_a_bijection(oracle, cfg, which):
    pb = cfg.n_head_kv * cfg.page_tokens * (cfg.head_dim + cfg.head_dim // 16)
    from oracle.oracle import shape_of, lib
    import ctypes as C
    assert lib().qwfn_oracle_page_bytes(C.byref(shape_of(cfg))) == pb
    hits = np.zeros(pb, dtype=np.int32)
    rng = np.random.default_rng(0)
    for g in range(cfg.n_head_kv):
        for row in range(cfg.page_tokens):
            for d in range(cfg.head_dim):
                qo, so = _offsets_ref(cfg, g, row, d, which)
                hits[qo] += 1
                if d % 32 == 0:
                    hits[so] += 1
                    hits[so + 1] += 1
            if rng.random() < 0.05:   # spot-check the oracle's own offsets
                d = int(rng.integers(cfg.head_dim))
                assert oracle.quant_offset(cfg, g, row, d, which) == _offsets_ref(cfg, g, row, d, which)[0]
                assert oracle.scale_offset(cfg, g, row, d // 32) == _offsets_ref(cfg, g, row, d)[1]
    assert (hits == 1).all()


@pytest.mark.parametrize("variant", [0, 1])
def test_append_bytes_and_dequant_roundtrip(oracle, variant):
    cfg = Cfg(quant_variant=variant)
    rng = np.random.default_rng(10 + variant)
    pt = np.array([[3, 0, 2], [1, 5, 4]], dtype=np.int32)        # 2 seqs, 3 pages each, permuted
    c = oracle.HostCache(cfg, 2, 3, page_table=pt, n_phys_pages=6)
    n = 40
    seq = rng.integers(0, 2, n).astype(np.int32)
    pos = rng.integers(0, 3 * cfg.page_tokens, n).astype(np.int32)
    # unique (seq, pos) so the last write is the only one
    _, keep = np.unique(seq.astype(np.int64) * 10**6 + pos, return_index=True)
    seq, pos = seq[keep], pos[keep]
    k = rng.standard_normal((len(pos), 2, 128)).astype(np.float32)
    v = (rng.standard_normal((len(pos), 2, 128)) * 7).astype(np.float32)
    assert c.append(k, v, pos, seq) == 0
    for i in range(len(pos)):
        phys = pt[seq[i], pos[i] // cfg.page_tokens]
        row = pos[i] % cfg.page_tokens
        for g in range(2):
            for which, src, pool in (("k", k, c.k_pages), ("v", v, c.v_pages)):
                page = pool[phys * c.page_bytes:(phys + 1) * c.page_bytes]
                deq = c.dequant_row(which, int(seq[i]), int(pos[i]), g)
                wh = 0 if which == "k" else 1
                for j in range(4):
                    d16, q = q8_block_ref(src[i, g, 32 * j:32 * j + 32], variant)
                    qo, so = _offsets_ref(cfg, g, row, 32 * j, wh)
                    assert int(page[so:so + 2].view(np.uint16)[0]) == d16
                    got_q = np.array([page[_offsets_ref(cfg, g, row, 32 * j + e, wh)[0]] for e in range(32)],
                                     dtype=np.uint8).view(np.int8)
                    np.testing.assert_array_equal(got_q, q)
                    np.testing.assert_array_equal(deq[32 * j:32 * j + 32], dequant_ref(d16, q))


def test_append_is_idempotent_and_reports_bad_rows(oracle):
    cfg = BASELINE
    c = oracle.HostCache(cfg, 1, 2)
    rng = np.random.default_rng(11)
    k = rng.standard_normal((3, 2, 128)).astype(np.float32)
    v = rng.standard_normal((3, 2, 128)).astype(np.float32)
    pos = np.array([5, 300, 17], np.int32)
    assert c.append(k, v, pos) == 0
    snap = c.k_pages.copy(), c.v_pages.copy()
    assert c.append(k, v, pos) == 0
    np.testing.assert_array_equal(c.k_pages, snap[0])
    np.testing.assert_array_equal(c.v_pages, snap[1])
    # position beyond capacity, bad sequence, bad page: skipped + status bits
    assert c.append(k[:1], v[:1], np.array([512], np.int32)) == 0x1
    assert c.append(k[:1], v[:1], np.array([0], np.int32), np.array([1], np.int32)) == 0x2
    c.page_table[0, 1] = 99
    assert c.append(k[:1], v[:1], np.array([300], np.int32)) == 0x4
    np.testing.assert_array_equal(c.k_pages, snap[0])


def test_append_f16_source_equals_f32_of_same_values(oracle):
    cfg = BASELINE
    rng = np.random.default_rng(12)
    k16 = rng.standard_normal((4, 2, 128)).astype(np.float16)
    v16 = rng.standard_normal((4, 2, 128)).astype(np.float16)
    pos = np.arange(4, dtype=np.int32)
    a, b = oracle.HostCache(cfg, 1, 1), oracle.HostCache(cfg, 1, 1)
    assert a.append(k16, v16, pos) == 0
    assert b.append(k16.astype(np.float32), v16.astype(np.float32), pos) == 0
    np.testing.assert_array_equal(a.k_pages, b.k_pages)
    np.testing.assert_array_equal(a.v_pages, b.v_pages)


@pytest.mark.parametrize("cfg", [BASELINE, TINY])
def test_pool_is_sequential_f32_mean(oracle, cfg):
    rng = np.random.default_rng(13)
    n_tok = 2 * cfg.page_tokens
    c = oracle.HostCache(cfg, 1, 2)
    k = (rng.standard_normal((n_tok, cfg.n_head_kv, cfg.head_dim)) * rng.uniform(0.1, 10, (n_tok, 1, 1))).astype(np.float32)
    c.append(k, k, np.arange(n_tok, dtype=np.int32))
    bt = cfg.block_tokens
    for b in range(n_tok // bt):
        assert c.pool_block(0, b) == 0
        for g in range(cfg.n_head_kv):
            rows = [c.dequant_row("k", 0, t, g) for t in range(b * bt, b * bt + bt)]
            acc = rows[0].copy()
            for r in rows[1:]:
                acc = (acc + r).astype(np.float32)
            ref = (acc * np.float32(1.0 / bt)).astype(np.float32)
            np.testing.assert_array_equal(c.pooled[0, g, b], ref)


def test_pool_constant_block_is_the_constant(oracle):
    cfg = BASELINE
    c = oracle.HostCache(cfg, 1, 1)
    row = np.ldexp(np.arange(128, dtype=np.float32) - 60, -3)      # exact in q8_0 (amax 67/8)
    k = np.broadcast_to(row, (64, 2, 128)).astype(np.float32).copy()
    c.append(k, k, np.arange(64, dtype=np.int32))
    c.pool_block(0, 0)
    deq = c.dequant_row("k", 0, 0, 0)
    np.testing.assert_array_equal(c.pooled[0, 0, 0], deq)
    np.testing.assert_array_equal(c.pooled[0, 1, 0], deq)
