"""libqwfn_qsa.so loads, exports every function include/qwfn_qsa.h declares,
and validates shapes/arguments on the host (no GPU call is reached)."""
import ctypes as C
import os
import re

import pytest

from qwfnfer_amd import _lib, qsa
from qwfnfer_amd.qsa import QsaConfig

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _declared():
    txt = open(os.path.join(ROOT, "include", "qwfn_qsa.h")).read()
    txt = re.sub(r"/\*.*?\*/", "", txt, flags=re.S)
    return set(re.findall(r"\b(qwfn_[a-z0-9_]+)\s*\(", txt))


def test_header_and_binding_agree():
    assert _declared() == set(_lib.EXPORTS)


def test_library_exports_every_declared_symbol():
    lib = _lib.load()
    for name in _declared():
        assert hasattr(lib, name), name
    assert lib.qwfn_qsa_abi_version() == 5


def _code(name, *args):
    return getattr(_lib.load(), name)(*args)


def test_shape_validation():
    ok = QsaConfig()
    s = ok.shape()
    assert _code("qwfn_qsa_check_shape", C.byref(s)) == 0
    bad = [
        dict(n_head=15), dict(head_dim=100), dict(page_tokens=100), dict(block_tokens=48),
        dict(local_tokens=-1), dict(sink_blocks=-1), dict(quant_variant=3), dict(relu_per_head=2),
        dict(topk_counts_forced=2), dict(topk_counts_forced=1, top_k_blocks=1),   # 1 < sink + window
        dict(kv_type=3), dict(kv_type=-1),
    ]
    for kw in bad:
        s = QsaConfig(**{**ok.__dict__, **kw}).shape()
        assert _code("qwfn_qsa_check_shape", C.byref(s)) == _lib.QWFN_EINVAL, kw
        assert _lib.load().qwfn_qsa_last_error()
    s = QsaConfig(**{**ok.__dict__, "shared_selection": 1}).shape()
    assert _code("qwfn_qsa_check_shape", C.byref(s)) == 0          # one selection for all KV heads
    s = QsaConfig(**{**ok.__dict__, "shared_selection": 2}).shape()
    assert _code("qwfn_qsa_check_shape", C.byref(s)) == _lib.QWFN_EINVAL
    s = QsaConfig(**{**ok.__dict__, "n_head": 6, "n_head_kv": 2, "head_dim": 96}).shape()
    assert _code("qwfn_qsa_check_shape", C.byref(s)) == _lib.QWFN_ENOTSUP
    # the checkpoint's rule: only a partial tail forced, counted in top_k
    s = qsa.checkpoint_config().shape()
    assert _code("qwfn_qsa_check_shape", C.byref(s)) == 0


def test_idx_argument_validation():
    cfg = qsa.checkpoint_config()
    icfg = qsa.IdxConfig()
    out, out2 = C.c_size_t(), C.c_size_t()
    assert _code("qwfn_idx_cache_bytes", C.byref(cfg.shape()), C.byref(icfg.shape()), 1, 4, C.byref(out),
                 C.byref(out2)) == 0
    assert out.value == 256 * 128 * 2 and out2.value == 4 * 256 // 4 * 128 * 2
    bad = [dict(idx_dim=96), dict(rope_dim=63), dict(rope_dim=256), dict(rope_freq_base=0.0),
           dict(rms_eps=-1.0), dict(n_idx_head=0)]
    for kw in bad:
        i = qsa.IdxConfig(**{**icfg.__dict__, **kw}).shape()
        rc = _code("qwfn_idx_cache_bytes", C.byref(cfg.shape()), C.byref(i), 1, 4, C.byref(out), C.byref(out2))
        assert rc in (_lib.QWFN_EINVAL, _lib.QWFN_ENOTSUP), kw
    i = qsa.IdxConfig(n_idx_head=3).shape()                 # no (128, 3) indexer instantiation
    assert _code("qwfn_idx_workspace_bytes", C.byref(cfg.shape()), C.byref(i), 1, 100, C.byref(out)) == \
        _lib.QWFN_ENOTSUP
    # NULL views and misaligned rows are rejected before any launch
    view = _lib.KvView(0, 0, 0, 0, 0, 1, 1, 1)
    iv = _lib.IdxView(0, 0, 0)
    assert _code("qwfn_idx_append_pool", C.byref(cfg.shape()), C.byref(view), C.byref(icfg.shape()), C.byref(iv),
                 None, 0, None, None, 1, None) == _lib.QWFN_EINVAL
    assert _code("qwfn_idx_select", C.byref(cfg.shape()), C.byref(view), C.byref(icfg.shape()), C.byref(iv),
                 None, None, 1, 1, None, None, 1, None, 0, None) == _lib.QWFN_EINVAL


def test_sizes():
    cfg = QsaConfig()
    assert cfg.page_bytes() == 2 * 256 * (128 + 8) == 69632
    assert cfg.max_selected(32768) == 64 + 1 + 9
    assert cfg.max_selected(4096) == 64
    assert cfg.dense().max_selected(4096) == 64
    assert cfg.workspace_bytes(8, 262144) > 0
    out = C.c_size_t()
    s = cfg.shape()
    assert _code("qwfn_qsa_pooled_bytes", C.byref(s), 1, 640, C.byref(out)) == 0
    assert out.value == 2560 * 2 * 128 * 4


def _view(k=1, v=1, pooled=16, pt=16, n_seq=1, pps=4, nphys=4):
    return _lib.KvView(k * 4096, v * 4096, pooled * 4096, pt * 4096, None, n_seq, pps, nphys)


def test_append_rejects_bad_arguments_before_launch():
    cfg = QsaConfig()
    s = cfg.shape()
    v = _view()
    f = "qwfn_kv_append_q8_0"
    assert _code(f, C.byref(s), None, 4096, 4096, 0, None, 4096, 1, None) == _lib.QWFN_EINVAL
    assert _code(f, C.byref(s), C.byref(v), None, 4096, 0, None, 4096, 1, None) == _lib.QWFN_EINVAL
    assert _code(f, C.byref(s), C.byref(v), 4096, 4096, 2, None, 4096, 1, None) == _lib.QWFN_EINVAL
    assert _code(f, C.byref(s), C.byref(v), 4100, 4096, 0, None, 4096, 1, None) == _lib.QWFN_EINVAL
    assert _code(f, C.byref(s), C.byref(v), 4096, 4096, 0, None, 4096, 0, None) == _lib.QWFN_EINVAL
    bad = _lib.KvView(4097 * 16 + 1, 4096, 4096, 4096, None, 1, 4, 4)
    assert _code(f, C.byref(s), C.byref(bad), 4096, 4096, 0, None, 4096, 1, None) == _lib.QWFN_EINVAL


def test_decode_rejects_exhausted_context_and_small_workspace():
    cfg = QsaConfig()
    s = cfg.shape()
    v = _view(pps=4)                       # capacity 1024 tokens
    f = "qwfn_sparse_attn_decode"
    args = lambda max_len, ws_bytes, n_seq=1: (C.byref(s), C.byref(v), 4096, 4096, 4096, 0, 4096, n_seq,
                                               max_len, 4096, None, None, 256 * 64, ws_bytes, None)
    assert _code(f, *args(1025, 1 << 30)) == _lib.QWFN_ERANGE
    assert _code(f, *args(1024, 100)) == _lib.QWFN_ERANGE
    assert _code(f, *args(0, 1 << 30)) == _lib.QWFN_EINVAL
    assert _code(f, *args(1024, 1 << 30, n_seq=2)) == _lib.QWFN_EINVAL
    msg = _lib.load().qwfn_qsa_last_error().decode()
    assert "n_seq" in msg


def test_decode_chain_rejects_bad_position_counts():
    """qwfn_sparse_attn_decode_chain takes 1 .. 8 positions; the checks run
    before any launch (n_pos = 1 is qwfn_sparse_attn_decode's own path)."""
    cfg = QsaConfig()
    s = cfg.shape()
    v = _view(pps=4)
    f = "qwfn_sparse_attn_decode_chain"
    args = lambda n_pos, max_len=1024: (C.byref(s), C.byref(v), 4096, 4096, 4096, 0, 4096, 1, n_pos, max_len,
                                        4096, None, None, 256 * 64, 1 << 30, None)
    for n_pos in (0, -1, 9):
        assert _code(f, *args(n_pos)) == _lib.QWFN_EINVAL, n_pos
        assert "n_pos" in _lib.load().qwfn_qsa_last_error().decode()
    assert _code(f, *args(2, 1025)) == _lib.QWFN_ERANGE      # past the view's 1024 tokens


def test_indexer_rejects_short_selection_buffer():
    cfg = QsaConfig()
    s = cfg.shape()
    v = _view(pps=256)
    rc = _code("qwfn_indexer_topk", C.byref(s), C.byref(v), 4096, 4096, 1, 32768, 4096, 4096, 70,
               256 * 64, 1 << 30, None)
    assert rc == _lib.QWFN_ERANGE


def test_python_errors_carry_the_message():
    cfg = QsaConfig(n_head=15)
    with pytest.raises(_lib.QsaError) as ei:
        cfg.check()
    assert ei.value.code == _lib.QWFN_EINVAL and "n_head" in str(ei.value)


def test_prefill_rejects_bad_arguments_before_launch():
    cfg = QsaConfig()
    s = cfg.shape()
    v = _view(pps=8, nphys=8)              # capacity 2048 tokens
    f = "qwfn_sparse_attn_prefill"

    def call(seq=0, pos0=0, n_q=16, k=4096, vv=4096, ws_bytes=1 << 30, sel=None, nsel=None, max_sel=0):
        return _code(f, C.byref(s), C.byref(v), 4096, k, vv, 0, seq, pos0, n_q, 4096, sel, nsel, max_sel,
                     256 * 64, ws_bytes, None)

    assert call(n_q=0) == _lib.QWFN_EINVAL
    assert call(pos0=-1) == _lib.QWFN_EINVAL
    assert call(seq=1) == _lib.QWFN_EINVAL
    assert call(pos0=2040, n_q=9) == _lib.QWFN_ERANGE          # past the view's capacity
    assert call(k=None) == _lib.QWFN_EINVAL                    # K without V
    assert call(ws_bytes=1000) == _lib.QWFN_ERANGE             # holds no query batch
    assert call(sel=4096, nsel=None) == _lib.QWFN_EINVAL
    assert call(pos0=1000, sel=4096, nsel=4096, max_sel=10) == _lib.QWFN_ERANGE
    out = C.c_size_t()
    assert _code("qwfn_qsa_prefill_workspace_bytes", C.byref(s), 163840, 256, C.byref(out)) == 0
    one = C.c_size_t()
    assert _code("qwfn_qsa_prefill_workspace_bytes", C.byref(s), 163840, 1, C.byref(one)) == 0
    assert out.value > one.value > 0
    assert _code("qwfn_qsa_prefill_workspace_bytes", C.byref(s), 163840, 1 << 20, C.byref(out)) == _lib.QWFN_ERANGE


def test_row_interop_rejects_bad_arguments_before_launch():
    cfg = QsaConfig()
    s = cfg.shape()
    v = _view(pps=4)                       # capacity 1024 tokens
    out = C.c_size_t()
    assert _code("qwfn_kv_row_bytes", C.byref(s), C.byref(out)) == 0
    assert out.value == 2 * 4 * 34 == cfg.row_bytes()
    for f in ("qwfn_kv_export_q8_0", "qwfn_kv_import_q8_0"):
        call = lambda seq=0, pos0=0, n=4, k=4096, vv=4096: _code(f, C.byref(s), C.byref(v), seq, pos0, n, k, vv,
                                                                 None)
        assert call(k=None, vv=None) == _lib.QWFN_EINVAL      # nothing to move
        assert call(k=4097) == _lib.QWFN_EINVAL               # rows are 2-byte aligned
        assert call(seq=1) == _lib.QWFN_EINVAL
        assert call(seq=-1) == _lib.QWFN_EINVAL
        assert call(pos0=-1) == _lib.QWFN_EINVAL
        assert call(n=0) == _lib.QWFN_EINVAL
        assert call(pos0=1020, n=5) == _lib.QWFN_ERANGE       # past the view's capacity
        assert "capacity" in _lib.load().qwfn_qsa_last_error().decode()


def test_noalloc_decode_rejects_what_its_array_cannot_hold():
    """qwfn_sparse_attn_decode_noalloc checks the workspace its arguments need
    against the library's 8 MiB scratch array before any device call."""
    cfg = QsaConfig()
    s = cfg.shape()
    v = _view(pps=4)
    call = lambda n_seq, max_len: _code("qwfn_sparse_attn_decode_noalloc", C.byref(s), C.byref(v), 4096, 4096,
                                        4096, 0, 4096, n_seq, max_len, 4096, None, None, None)
    assert call(16, 1 << 20) == _lib.QWFN_ERANGE          # 15.4 MiB of workspace
    assert "scratch" in _lib.load().qwfn_qsa_last_error().decode()
    assert call(0, 1024) == _lib.QWFN_EINVAL
    need = C.c_size_t()
    assert _code("qwfn_qsa_workspace_bytes", C.byref(s), 8, 1 << 20, C.byref(need)) == 0
    assert need.value <= 8 << 20                          # eight sequences of 1M tokens fit


def test_time_next_call_arms_pairs_only():
    """The timing hook takes (start, stop) pairs; half a pair is refused, NULL
    disarms (no GPU call: arming only stores the handles)."""
    lib = _lib.load()
    arr = (C.c_void_p * 6)()
    assert lib.qwfn_qsa_time_next_call(arr) == 0                 # all NULL: nothing armed
    arr[2] = 0x1000                                              # attention start without its stop
    assert lib.qwfn_qsa_time_next_call(arr) == _lib.QWFN_EINVAL
    assert "stop" in lib.qwfn_qsa_last_error().decode()
    assert lib.qwfn_qsa_time_next_call(None) == 0                # disarm


def test_cut_poll_bound_hook():
    """qwfn_qsa_test_set_cut_polls swaps the bound (default 65536) and returns
    the one it replaces; a negative bound is refused and changes nothing."""
    prev = C.c_int32(-1)
    assert _code("qwfn_qsa_test_set_cut_polls", 7, C.byref(prev)) == 0
    try:
        assert prev.value == 65536
        again = C.c_int32(-1)
        assert _code("qwfn_qsa_test_set_cut_polls", -1, C.byref(again)) == _lib.QWFN_EINVAL
        assert again.value == -1
        assert _code("qwfn_qsa_test_set_cut_polls", 9, None) == 0
        assert _code("qwfn_qsa_test_set_cut_polls", 7, C.byref(again)) == 0 and again.value == 9
    finally:
        assert _code("qwfn_qsa_test_set_cut_polls", prev.value, None) == 0
