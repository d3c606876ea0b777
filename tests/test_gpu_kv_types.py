"""Parity of the q4_0 and fp16 cache types (the reference's --kv q4_0 / f16,
tools/qwfn_gen.cpp:55-57) with the CPU oracle, through the C ABI.

Bit-exact: cache bytes after appends (f32 and f16 sources, permuted pages),
pooled keys, selected blocks, exported rows (ggml's block_q4_0 / fp16 rows).
Attention within 2e-3 + 1e-3 |ref| of the fp64 oracle over the same
dequantized cache: fused decode steps and prefill chunks, at BASELINE shapes
(the general attention kernel for these types), the tiny shape and the
checkpoint head shape."""
import numpy as np
import pytest
import torch

from _gpu import assert_close_attn, cfg_of, decode_steps, fill, kv_rows, make_pair, np_of
from _refs import BASELINE, TINY, Cfg
from oracle import oracle as O
from qwfnfer_amd import qsa, snapshot
from test_gpu_parity import _decode_steps, _prefill_case

pytestmark = pytest.mark.gpu

TYPES = [1, 2]                              # QWFN_KV_Q4_0, QWFN_KV_F16
G12 = Cfg(n_head=24, n_head_kv=2, head_dim=256, block_tokens=4, page_tokens=128, top_k_blocks=40,
          sink_blocks=1, local_tokens=16)


def with_type(cfg, kt):
    return Cfg(**{**cfg.__dict__, "kv_type": kt})


@pytest.mark.parametrize("kt", TYPES)
@pytest.mark.parametrize("dtype", [np.float32, np.float16])
def test_append_bytes_match_oracle(kt, dtype):
    cfg = with_type(BASELINE, kt)
    rng = np.random.default_rng(950 + kt)
    dev, host = make_pair(cfg, 2, 3, seed=951, spare=2)
    n = 300
    seq = rng.integers(0, 2, n).astype(np.int32)
    pos = rng.permutation(3 * 256)[:n].astype(np.int32)
    k, v = kv_rows(rng, n, cfg)
    k[0, 0, :32] = 0.0                                 # a zero block: d = -0
    k[1, 0, :32] = np.arange(32) % 16 - 8              # magnitude ties
    k, v = k.astype(dtype), v.astype(dtype)
    assert host.append(k, v, pos, seq) == 0
    for _ in range(2):                                 # idempotent overwrite
        qsa.append_q8_0(dev, torch.from_numpy(k).cuda(), torch.from_numpy(v).cuda(),
                        torch.from_numpy(pos).cuda(), torch.from_numpy(seq).cuda())
        torch.cuda.synchronize()
        np.testing.assert_array_equal(np_of(dev.k_pages), host.k_pages)
        np.testing.assert_array_equal(np_of(dev.v_pages), host.v_pages)
    assert qsa.read_status(dev) == 0


@pytest.mark.parametrize("kt", TYPES)
def test_pool_and_select_match_oracle(kt):
    cfg = with_type(BASELINE, kt)
    rng = np.random.default_rng(960 + kt)
    L = 6000
    dev, host = make_pair(cfg, 1, L // 256 + 1, seed=961)
    fill(dev, host, rng, [L])                          # appends + pool_rebuild, compared below
    np.testing.assert_array_equal(np_of(dev.pooled)[:, :, :L // 64], host.pooled[:, :, :L // 64])
    q = rng.standard_normal((1, 16, 128), dtype=np.float32)
    ws = qsa.Workspace(cfg_of(cfg), 1, L)
    sel, nsel = qsa.indexer_topk(dev, torch.from_numpy(q).cuda(), torch.tensor([L], dtype=torch.int32,
                                                                                 device="cuda"), L, ws)
    out = qsa.sparse_decode_attn(dev, torch.from_numpy(q).cuda(), torch.tensor([L], dtype=torch.int32,
                                                                                  device="cuda"), L, ws, sel, nsel)
    torch.cuda.synchronize()
    hs, hn = host.indexer_topk(q, [L], max_sel=sel.shape[-1])
    np.testing.assert_array_equal(np_of(nsel), hn)
    for g in range(2):
        np.testing.assert_array_equal(np_of(sel)[0, g, :hn[0, g]], hs[0, g, :hn[0, g]])
    from _gpu import assert_close_attn
    assert_close_attn(np_of(out), host.attention_f64(q, [L], hs, hn), f"kv_type {kt}")


@pytest.mark.parametrize("kt", TYPES)
def test_decode_steps(kt):
    _decode_steps(with_type(BASELINE, kt), [4096 - 3], steps=6, seed=970 + kt)
    _decode_steps(with_type(TINY, kt), [130, 61], steps=6, seed=972 + kt, dtype=np.float16)


@pytest.mark.parametrize("kt", TYPES)
def test_decode_steps_attention_selects(kt):
    # up to eight sequences, the general attention's workgroups select for
    # themselves: several lengths, and 4-token blocks past 4096 eligible ones
    # (the larger per-thread key counts of the 256-thread selection)
    _decode_steps(with_type(BASELINE, kt), [3000, 64 * 70 + 5, 100], steps=3, seed=990 + kt)
    _decode_steps(with_type(TINY, kt), [20000, 9000], steps=2, seed=992 + kt)


@pytest.mark.parametrize("kt", TYPES)
def test_decode_steps_checkpoint_heads(kt):
    _decode_steps(with_type(G12, kt), [700], steps=5, seed=975 + kt)


@pytest.mark.parametrize("kt", TYPES)
def test_prefill(kt):
    _prefill_case(with_type(BASELINE, kt), 3000, 150, seed=980 + kt)
    _prefill_case(with_type(TINY, kt), 90, 70, seed=982 + kt, dtype=np.float16)


@pytest.mark.parametrize("kt", TYPES)
def test_export_import_rows(kt):
    cfg = with_type(BASELINE, kt)
    rng = np.random.default_rng(990 + kt)
    dev, host = make_pair(cfg, 1, 2, seed=991)
    L = 400
    k, v = kv_rows(rng, L, cfg)
    qsa.append_q8_0(dev, torch.from_numpy(k).cuda(), torch.from_numpy(v).cuda(),
                    torch.arange(L, dtype=torch.int32, device="cuda"))
    rb = cfg_of(cfg).row_bytes()
    assert rb == (2 * 4 * 18 if kt == 1 else 2 * 128 * 2)
    kr, vr = qsa.export_rows_q8_0(dev, 0, 0, L)
    torch.cuda.synchronize()
    want_k = np.stack([O.quantize_row_type(k[t].ravel(), kt) for t in range(L)])
    want_v = np.stack([O.quantize_row_type(v[t].ravel(), kt) for t in range(L)])
    np.testing.assert_array_equal(np_of(kr), want_k)
    np.testing.assert_array_equal(np_of(vr), want_v)
    # import into a fresh cache (other pages) gives the same bytes; arbitrary bytes round-trip
    dev2, _ = make_pair(cfg, 1, 2, seed=992)
    qsa.import_rows_q8_0(dev2, 0, 0, kr, vr)
    kr2, vr2 = qsa.export_rows_q8_0(dev2, 0, 0, L)
    junk = torch.randint(0, 256, (L, rb), dtype=torch.uint8, device="cuda")
    if kt == 2:                                        # keep fp16 rows free of NaN bit patterns for the compare
        junk[:, 1::2] &= 0x3F
    qsa.import_rows_q8_0(dev2, 0, 0, junk, junk)
    kj, vj = qsa.export_rows_q8_0(dev2, 0, 0, L)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(np_of(kr2), np_of(kr))
    np.testing.assert_array_equal(np_of(vr2), np_of(vr))
    np.testing.assert_array_equal(np_of(kj), np_of(junk))
    np.testing.assert_array_equal(np_of(vj), np_of(junk))
    assert qsa.read_status(dev) == 0 and qsa.read_status(dev2) == 0


@pytest.mark.parametrize("kt", TYPES)
def test_snapshot_round_trip(kt, tmp_path):
    cfg = with_type(BASELINE, kt)
    rng = np.random.default_rng(995 + kt)
    dev, host = make_pair(cfg, 1, 3, seed=996)
    fill(dev, host, rng, [700])
    path = str(tmp_path / "kv.snap")
    h = snapshot.save_snapshot(dev, path, 0, 700)
    assert h["format"] == snapshot.FORMATS[kt] and h["kv_type"] == kt
    dev2, _ = make_pair(cfg, 2, 3, seed=997)
    assert snapshot.load_snapshot(dev2, path, 1) == 700
    torch.cuda.synchronize()
    np.testing.assert_array_equal(np_of(dev2.pooled)[1, :, :700 // 64], np_of(dev.pooled)[0, :, :700 // 64])


# kv_round_f16: the decode attention on every dequantized K and V value rounded
# to fp16, as the reference's gather casts its rows to F16 before
# flash_attn_ext (src/qwfn_graph.cpp:530-537); against the oracle run on the
# same rounded values
ROUND_TYPES = [0, 1, 2]                     # q8_0, q4_0, fp16 (a no-op for fp16 rows)


@pytest.mark.parametrize("kt", ROUND_TYPES)
def test_decode_steps_kv_round_f16(kt):
    cfg = Cfg(**{**with_type(BASELINE, kt).__dict__, "kv_round_f16": 1})
    decode_steps(cfg, [65536 - 2, 3000], steps=3, seed=1000 + kt, modes=["fused", "two_call", "fused"],
                 reattend=True)
    decode_steps(Cfg(**{**TINY.__dict__, "kv_type": kt, "kv_round_f16": 1}), [2000, 61], steps=2,
                 seed=1003 + kt, dtype=np.float16)


def test_kv_round_f16_dense_and_batched_q8_0():
    """q8_0 with kv_round_f16 on the matrix-core decode kernel's other modes:
    the dense attention call (every block, no selection), the dense fused call
    (top_k 0) and eight sequences of config 5's lengths (fused, then the
    two-call path over a given selection, several tiles a workgroup)."""
    from test_gpu_workloads import CONFIG5_LENGTHS
    cfg = Cfg(**{**BASELINE.__dict__, "top_k_blocks": 0, "kv_round_f16": 1})
    rng = np.random.default_rng(1020)
    L = 4096 + 37
    dev, host = make_pair(cfg, 1, L // 256 + 1)
    fill(dev, host, rng, [L], pool=False)
    q = rng.standard_normal((1, 16, 128), dtype=np.float32)
    ws = qsa.Workspace(cfg_of(cfg), 1, L)
    Lt = torch.tensor([L], dtype=torch.int32, device="cuda")
    out = qsa.sparse_decode_attn(dev, torch.from_numpy(q).cuda(), Lt, L, ws)
    torch.cuda.synchronize()
    assert_close_attn(np_of(out), host.attention_f64(q, [L]), "dense attention, kv_round_f16")
    decode_steps(cfg, [4096 - 2], steps=2, seed=1021)
    decode_steps(Cfg(**{**BASELINE.__dict__, "kv_round_f16": 1}), CONFIG5_LENGTHS, steps=2, seed=1022,
                 modes=["fused", "two_call"], reattend=True)


def test_kv_round_f16_changes_q8_0_outputs():
    """The two modes on the same cache and queries, each checked against its
    own fp64 oracle inside decode_steps: q8_0 values d * q are not all fp16
    numbers, so the outputs differ.  With the configuration's per-block scales
    up to 10 the difference reaches about 1e-2, more than the 2e-3 + 1e-3 |ref|
    bound between either mode and its own reference: the reference's F16 cast
    moves its outputs that far from exact fp32 attention."""
    outs = []
    for r in (0, 1):
        cfg = Cfg(**{**BASELINE.__dict__, "kv_round_f16": r})
        outs.append(decode_steps(cfg, [20000], steps=1, seed=1010)[0])
    d = np.abs(outs[0] - outs[1])
    print(f"max |o(kv_round_f16) - o(exact)| = {d.max():.3g}", flush=True)
    assert d.max() > 0


@pytest.mark.parametrize("kt", [0, 1, 2])
def test_decode_independent_of_the_workspace_history(kt):
    """Layers sharing one workspace, as the bench's replicas do: a layer's
    fused step gives the same bytes whatever call used the workspace before
    it (here another layer of a different length), at a context whose
    selection holds 16 keys a thread; and a hipGraph replay of the step
    equals the eager one."""
    cfg = qsa.QsaConfig(kv_type=kt)
    gen = torch.Generator(device="cuda")
    gen.manual_seed(90 + kt)
    lens = [140000, 90000]
    max_len = 140000 + 8
    pps = max_len // cfg.page_tokens + 1
    caches = []
    for L in lens:
        c = qsa.KvCache.allocate(cfg, 1, pps)
        for t0 in range(0, L, 32768):
            n = min(32768, L - t0)
            k = torch.randn((n, cfg.n_head_kv, cfg.head_dim), device="cuda", generator=gen)
            v = torch.randn((n, cfg.n_head_kv, cfg.head_dim), device="cuda", generator=gen)
            qsa.append_q8_0(c, k, v, torch.arange(t0, t0 + n, dtype=torch.int32, device="cuda"))
        qsa.pool_rebuild(c, 0, L // cfg.block_tokens)
        caches.append(c)
    ws = qsa.Workspace(cfg, 1, max_len)
    q = [torch.randn((1, cfg.n_head, cfg.head_dim), device="cuda", generator=gen) for _ in lens]
    kn = [torch.randn((1, cfg.n_head_kv, cfg.head_dim), device="cuda", generator=gen) for _ in lens]
    sl = [torch.tensor([L + 1], dtype=torch.int32, device="cuda") for L in lens]
    outs = [torch.empty((1, cfg.n_head, cfg.head_dim), device="cuda") for _ in lens]

    def step(i):
        qsa.sparse_attn_decode(caches[i], q[i], kn[i], kn[i], sl[i], max_len, ws, out=outs[i])

    step(0)
    torch.cuda.synchronize()
    ref = outs[0].clone()
    for order in ([1, 0], [0, 1, 0], [1, 1, 0]):
        for i in order:
            step(i)
        torch.cuda.synchronize()
        assert torch.equal(outs[0], ref), f"kv_type {kt}: layer 0 after {order} differs"
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    g = torch.cuda.CUDAGraph()
    with torch.cuda.stream(s):
        with torch.cuda.graph(g, stream=s):
            step(1)
            step(0)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    for rep in range(3):
        outs[0].fill_(float("nan"))
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(outs[0], ref), f"kv_type {kt}: graph replay {rep} differs"
        step(0)
        torch.cuda.synchronize()


def test_q4_0_negative_scale_dominant_cell():
    """ggml's q4_0 scale is signed (d = max / -8, max the element of largest
    magnitude): a cell whose V blocks have large negative scales and which
    takes nearly all the softmax weight, among cells of small positive
    scales.  The attention's weight range must follow the scales' magnitudes
    (a range set by the largest positive scale overflows fp16 here)."""
    cfg = Cfg(**{**BASELINE.__dict__, "kv_type": 1, "top_k_blocks": 0})
    rng = np.random.default_rng(1030)
    L = 200
    k = rng.standard_normal((L, cfg.n_head_kv, cfg.head_dim)).astype(np.float32) * 0.05
    v = rng.standard_normal((L, cfg.n_head_kv, cfg.head_dim)).astype(np.float32)
    blocks = v.reshape(L, cfg.n_head_kv, cfg.head_dim // 32, 32)
    # every block's element of largest magnitude negative (d > 0), small
    idx = np.abs(blocks).argmax(-1)
    np.put_along_axis(blocks, idx[..., None], -np.abs(np.take_along_axis(blocks, idx[..., None], -1)) - 1.0, -1)
    blocks *= 0.1
    hot = [7, 131]
    for t in hot:                              # large positive maxima: d < 0, |d| 1000x the others
        blocks[t] = np.abs(blocks[t]) * 1000.0
    q = np.zeros((1, cfg.n_head, cfg.head_dim), np.float32)
    for g in range(cfg.n_head_kv):
        q[0, g * cfg.group:(g + 1) * cfg.group] = k[hot[g], g] * 400.0
    dev, host = make_pair(cfg, 1, 1)
    pos = np.arange(L, dtype=np.int32)
    assert host.append(k, v, pos) == 0
    qsa.append_q8_0(dev, torch.from_numpy(k).cuda(), torch.from_numpy(v).cuda(), torch.from_numpy(pos).cuda())
    Lt = torch.tensor([L], dtype=torch.int32, device="cuda")
    ws = qsa.Workspace(cfg_of(cfg), 1, L)
    out = qsa.sparse_decode_attn(dev, torch.from_numpy(q).cuda(), Lt, L, ws)
    torch.cuda.synchronize()
    got = np_of(out)
    assert np.isfinite(got).all(), "non-finite attention output"
    assert_close_attn(got, host.attention_f64(q, [L]), "q4_0, negative scales dominating")
