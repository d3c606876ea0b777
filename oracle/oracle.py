"""ctypes/numpy binding of the CPU oracle (libqwfn_oracle.so).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py -- never by the qwfnfer_amd package.  Host-memory
caches here use exactly the device layout of include/qwfn_qsa.h, so device
buffers copied back compare byte-for-byte.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libqwfn_oracle.so")

Q8_X86_RNE = 0
Q8_REF_ROUNDF = 1
SRC_F32 = 0
SRC_F16 = 1


class Shape(C.Structure):
    _fields_ = [(n, C.c_int32) for n in (
        "n_head", "n_head_kv", "head_dim", "block_tokens", "page_tokens", "top_k_blocks",
        "sink_blocks", "local_tokens", "relu_per_head", "shared_selection", "quant_variant",
        "topk_counts_forced", "kv_type", "kv_round_f16")]


class IdxShape(C.Structure):
    _fields_ = [("idx_dim", C.c_int32), ("n_idx_head", C.c_int32), ("rope_dim", C.c_int32),
                ("rope_freq_base", C.c_float), ("rms_eps", C.c_float)]


class View(C.Structure):
    _fields_ = [
        ("k_pages", C.c_void_p), ("v_pages", C.c_void_p), ("pooled", C.c_void_p),
        ("page_table", C.c_void_p), ("status", C.c_void_p),
        ("n_seq", C.c_int32), ("pages_per_seq", C.c_int32), ("n_phys_pages", C.c_int32)]


def build() -> str:
    """Compile the oracle with its Makefile (gcc)."""
    subprocess.run(["make", "-s", "-C", HERE], check=True)
    return LIB_PATH


_lib = None


def lib() -> C.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        L = C.CDLL(LIB_PATH)
        P, I, S, V = C.c_void_p, C.c_int32, C.POINTER(Shape), C.POINTER(View)
        sig = {
            "qwfn_oracle_f32_to_f16": (C.c_uint16, [C.c_float]),
            "qwfn_oracle_f16_to_f32": (C.c_float, [C.c_uint16]),
            "qwfn_oracle_f32_to_f16_n": (None, [P, C.c_int64, P]),
            "qwfn_oracle_quantize_block": (None, [P, I, P, P]),
            "qwfn_oracle_quantize_row_ggml": (None, [P, C.c_int64, I, P]),
            "qwfn_oracle_quantize_block_q4_0": (None, [P, P, P]),
            "qwfn_oracle_quantize_row_type": (None, [P, C.c_int64, I, I, P]),
            "qwfn_oracle_page_bytes": (C.c_size_t, [S]),
            "qwfn_oracle_quant_offset": (C.c_int64, [S, I, I, I, I]),
            "qwfn_oracle_scale_offset": (C.c_int64, [S, I, I, I]),
            "qwfn_oracle_append": (C.c_int, [S, V, P, P, I, P, P, I]),
            "qwfn_oracle_dequant_row": (C.c_int, [S, V, P, I, I, I, P]),
            "qwfn_oracle_pool_block": (C.c_int, [S, V, I, I]),
            "qwfn_oracle_block_score": (C.c_float, [S, P, P]),
            "qwfn_oracle_select": (I, [S, P, I, P, I]),
            "qwfn_oracle_max_selected": (I, [S, I]),
            "qwfn_oracle_indexer_topk": (C.c_int, [S, V, P, P, I, P, P, I]),
            "qwfn_oracle_attention_f64": (C.c_int, [S, V, P, P, I, P, P, I, P]),
            "qwfn_oracle_decode_step_f32": (C.c_int, [S, V, P, P, P, P, I, P, P, P, I]),
            "qwfn_oracle_prefill_f64": (C.c_int, [S, V, P, I, I, I, P, P, I, P]),
            "qwfn_oracle_prefill_f64_strided": (C.c_int, [S, V, P, I, I, I, I, P, P, I, P]),
            "qwfn_oracle_idx_pool_block": (C.c_int, [S, C.POINTER(IdxShape), P, P, I, P]),
        }
        for name, (res, args) in sig.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def _p(a: np.ndarray | None):
    if a is None:
        return None
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data


def shape_of(cfg) -> Shape:
    """A Shape from any object with the QsaConfig field names."""
    return Shape(cfg.n_head, cfg.n_head_kv, cfg.head_dim, cfg.block_tokens, cfg.page_tokens,
                 cfg.top_k_blocks, cfg.sink_blocks, cfg.local_tokens, cfg.relu_per_head,
                 cfg.shared_selection, cfg.quant_variant, getattr(cfg, "topk_counts_forced", 0),
                 getattr(cfg, "kv_type", 0), getattr(cfg, "kv_round_f16", 0))


# ---- scalar / block helpers -------------------------------------------------

def f32_to_f16_bits(x) -> np.ndarray:
    x = np.ascontiguousarray(np.asarray(x, dtype=np.float32))
    out = np.empty(x.shape, dtype=np.uint16)
    lib().qwfn_oracle_f32_to_f16_n(_p(x), x.size, _p(out))
    return out


def f16_bits_to_f32(h) -> np.ndarray:
    h = np.asarray(h, dtype=np.uint16)
    f = np.vectorize(lambda v: lib().qwfn_oracle_f16_to_f32(int(v)), otypes=[np.float32])
    return f(h) if h.size else h.astype(np.float32)


def quantize_block(x, variant: int = Q8_X86_RNE):
    x = np.ascontiguousarray(np.asarray(x, dtype=np.float32))
    assert x.size == 32
    d = np.zeros(1, dtype=np.uint16)
    qs = np.zeros(32, dtype=np.int8)
    lib().qwfn_oracle_quantize_block(_p(x), variant, _p(d), _p(qs))
    return int(d[0]), qs


def quantize_row_ggml(x, variant: int = Q8_X86_RNE) -> np.ndarray:
    x = np.ascontiguousarray(np.asarray(x, dtype=np.float32).ravel())
    out = np.zeros(x.size // 32 * 34, dtype=np.uint8)
    lib().qwfn_oracle_quantize_row_ggml(_p(x), x.size, variant, _p(out))
    return out


def quantize_block_q4_0(x):
    """(d fp16 bits, qs uint8[16]) of one 32-value q4_0 block."""
    x = np.ascontiguousarray(np.asarray(x, dtype=np.float32).ravel())
    assert x.size == 32
    d = np.zeros(1, dtype=np.uint16)
    qs = np.zeros(16, dtype=np.uint8)
    lib().qwfn_oracle_quantize_block_q4_0(_p(x), _p(d), _p(qs))
    return int(d[0]), qs


def quantize_row_type(x, kv_type: int, variant: int = Q8_X86_RNE) -> np.ndarray:
    """ggml's row bytes of the cache type for values x (a multiple of 32)."""
    x = np.ascontiguousarray(np.asarray(x, dtype=np.float32).ravel())
    per = {0: 34, 1: 18, 2: 64}[kv_type]
    out = np.zeros(x.size // 32 * per, dtype=np.uint8)
    lib().qwfn_oracle_quantize_row_type(_p(x), x.size, kv_type, variant, _p(out))
    return out


# ---- host cache ---------------------------------------------------------------

class HostCache:
    """Host mirror of one layer's paged cache (same bytes as the device)."""

    def __init__(self, cfg, n_seq: int, pages_per_seq: int, page_table=None, n_phys_pages=None):
        self.cfg = cfg
        self.shape = shape_of(cfg)
        self.n_seq = n_seq
        self.pages_per_seq = pages_per_seq
        if page_table is None:
            page_table = np.arange(n_seq * pages_per_seq, dtype=np.int32).reshape(n_seq, pages_per_seq)
        self.page_table = np.ascontiguousarray(np.asarray(page_table, dtype=np.int32))
        self.n_phys_pages = int(n_phys_pages if n_phys_pages is not None else n_seq * pages_per_seq)
        self.page_bytes = int(lib().qwfn_oracle_page_bytes(C.byref(self.shape)))
        self.k_pages = np.zeros(self.n_phys_pages * self.page_bytes, dtype=np.uint8)
        self.v_pages = np.zeros_like(self.k_pages)
        bps = pages_per_seq * cfg.page_tokens // cfg.block_tokens
        self.pooled = np.zeros((n_seq, cfg.n_head_kv, bps, cfg.head_dim), dtype=np.float32)
        self.status = np.zeros(1, dtype=np.int32)

    @property
    def capacity(self) -> int:
        return self.pages_per_seq * self.cfg.page_tokens

    def view(self) -> View:
        return View(_p(self.k_pages), _p(self.v_pages), _p(self.pooled), _p(self.page_table),
                    _p(self.status), self.n_seq, self.pages_per_seq, self.n_phys_pages)

    # ---- operations --------------------------------------------------------
    def append(self, k, v, pos, seq_ids=None) -> int:
        k = np.ascontiguousarray(k)
        v = np.ascontiguousarray(v)
        dt = SRC_F16 if k.dtype == np.float16 else SRC_F32
        if dt == SRC_F32:
            k = k.astype(np.float32, copy=False)
            v = v.astype(np.float32, copy=False)
        pos = np.ascontiguousarray(np.asarray(pos, dtype=np.int32).ravel())
        sid = None if seq_ids is None else np.ascontiguousarray(np.asarray(seq_ids, dtype=np.int32).ravel())
        view = self.view()
        return lib().qwfn_oracle_append(C.byref(self.shape), C.byref(view), _p(k), _p(v), dt, _p(sid),
                                        _p(pos), pos.size)

    def dequant_row(self, which: str, seq: int, t: int, g: int) -> np.ndarray:
        out = np.zeros(self.cfg.head_dim, dtype=np.float32)
        pool = self.k_pages if which == "k" else self.v_pages
        view = self.view()
        rc = lib().qwfn_oracle_dequant_row(C.byref(self.shape), C.byref(view), _p(pool), seq, t, g, _p(out))
        if rc:
            raise IndexError(f"dequant_row status {rc}")
        return out

    def pool_block(self, seq: int, b: int) -> int:
        view = self.view()
        return lib().qwfn_oracle_pool_block(C.byref(self.shape), C.byref(view), seq, b)

    def indexer_topk(self, q, seq_len, max_sel=None):
        q = np.ascontiguousarray(np.asarray(q, dtype=np.float32))
        seq_len = np.ascontiguousarray(np.asarray(seq_len, dtype=np.int32).ravel())
        n_seq = seq_len.size
        if max_sel is None:
            max_sel = max_selected(self.cfg, int(seq_len.max()))
        sel = np.full((n_seq, self.cfg.n_head_kv, max_sel), -1, dtype=np.int32)
        nsel = np.zeros((n_seq, self.cfg.n_head_kv), dtype=np.int32)
        view = self.view()
        rc = lib().qwfn_oracle_indexer_topk(C.byref(self.shape), C.byref(view), _p(q), _p(seq_len), n_seq,
                                            _p(sel), _p(nsel), max_sel)
        if rc < 0:
            raise RuntimeError(f"oracle indexer_topk -> {rc}")
        return sel, nsel

    def attention_f64(self, q, seq_len, sel=None, nsel=None):
        q = np.ascontiguousarray(np.asarray(q, dtype=np.float32))
        seq_len = np.ascontiguousarray(np.asarray(seq_len, dtype=np.int32).ravel())
        n_seq = seq_len.size
        out = np.zeros((n_seq, self.cfg.n_head, self.cfg.head_dim), dtype=np.float64)
        max_sel = 0 if sel is None else sel.shape[-1]
        if sel is not None:
            sel = np.ascontiguousarray(sel, dtype=np.int32)
            nsel = np.ascontiguousarray(nsel, dtype=np.int32)
        view = self.view()
        rc = lib().qwfn_oracle_attention_f64(C.byref(self.shape), C.byref(view), _p(q), _p(seq_len), n_seq,
                                             _p(sel), _p(nsel), max_sel, _p(out))
        if rc < 0:
            raise RuntimeError(f"oracle attention -> {rc}")
        return out

    def prefill_f64(self, q, seq: int, pos0: int, max_sel=None, attn_stride: int = 1):
        """Selections and fp64 outputs of prefill queries pos0.. of sequence seq
        (rows and pooled keys already in place).  attn_stride > 1: outputs of
        every attn_stride-th query and the last one only (the rest zero)."""
        q = np.ascontiguousarray(np.asarray(q, dtype=np.float32))
        n_q = q.size // (self.cfg.n_head * self.cfg.head_dim)
        if max_sel is None:
            max_sel = max_selected(self.cfg, pos0 + n_q)
        sel = np.full((n_q, self.cfg.n_head_kv, max_sel), -1, dtype=np.int32)
        nsel = np.zeros((n_q, self.cfg.n_head_kv), dtype=np.int32)
        out = np.zeros((n_q, self.cfg.n_head, self.cfg.head_dim), dtype=np.float64)
        view = self.view()
        rc = lib().qwfn_oracle_prefill_f64_strided(C.byref(self.shape), C.byref(view), _p(q), seq, pos0, n_q,
                                                   attn_stride, _p(sel), _p(nsel), max_sel, _p(out))
        if rc < 0:
            raise RuntimeError(f"oracle prefill -> {rc}")
        return sel, nsel, out

    def decode_step_f32(self, q, k_new, v_new, seq_len):
        q = np.ascontiguousarray(np.asarray(q, dtype=np.float32))
        k_new = np.ascontiguousarray(np.asarray(k_new, dtype=np.float32))
        v_new = np.ascontiguousarray(np.asarray(v_new, dtype=np.float32))
        seq_len = np.ascontiguousarray(np.asarray(seq_len, dtype=np.int32).ravel())
        n_seq = seq_len.size
        max_sel = max_selected(self.cfg, int(seq_len.max()))
        sel = np.full((n_seq, self.cfg.n_head_kv, max_sel), -1, dtype=np.int32)
        nsel = np.zeros((n_seq, self.cfg.n_head_kv), dtype=np.int32)
        out = np.zeros((n_seq, self.cfg.n_head, self.cfg.head_dim), dtype=np.float32)
        view = self.view()
        threads = lib().qwfn_oracle_decode_step_f32(C.byref(self.shape), C.byref(view), _p(q), _p(k_new),
                                                    _p(v_new), _p(seq_len), n_seq, _p(out), _p(sel),
                                                    _p(nsel), max_sel)
        if threads < 0:
            raise RuntimeError(f"oracle decode_step -> {threads}")
        return out, sel, nsel, threads


def block_score(cfg, q_group, p) -> float:
    s = shape_of(cfg)
    q_group = np.ascontiguousarray(np.asarray(q_group, dtype=np.float32))
    p = np.ascontiguousarray(np.asarray(p, dtype=np.float32))
    return float(lib().qwfn_oracle_block_score(C.byref(s), _p(q_group), _p(p)))


def select(cfg, scores, seq_len: int, max_sel: int | None = None) -> np.ndarray:
    s = shape_of(cfg)
    scores = np.ascontiguousarray(np.asarray(scores, dtype=np.float32))
    if max_sel is None:
        max_sel = max_selected(cfg, seq_len)
    out = np.zeros(max(max_sel, 1), dtype=np.int32)
    n = lib().qwfn_oracle_select(C.byref(s), _p(scores), seq_len, _p(out), max_sel)
    if n < 0:
        raise RuntimeError(f"oracle select -> {n}")
    return out[:n].copy()


def idx_shape_of(icfg) -> IdxShape:
    """An IdxShape from any object with the qwfnfer_amd.qsa.IdxConfig field names."""
    return IdxShape(icfg.idx_dim, icfg.n_idx_head, icfg.rope_dim, icfg.rope_freq_base, icfg.rms_eps)


def idx_pool_block(cfg, icfg, members_f16, k_norm, b: int) -> np.ndarray:
    """The checkpoint indexer's pooled key of block b from its block_tokens raw
    fp16 members ([bt][idx_dim], float16 or uint16 bits)."""
    s, i = shape_of(cfg), idx_shape_of(icfg)
    m = np.ascontiguousarray(np.asarray(members_f16).astype(np.float16).view(np.uint16)
                             if np.asarray(members_f16).dtype != np.uint16 else members_f16)
    assert m.shape == (cfg.block_tokens, icfg.idx_dim), m.shape
    w = np.ascontiguousarray(np.asarray(k_norm, dtype=np.float32))
    out = np.zeros(icfg.idx_dim, dtype=np.float32)
    rc = lib().qwfn_oracle_idx_pool_block(C.byref(s), C.byref(i), _p(m), _p(w), b, _p(out))
    if rc < 0:
        raise RuntimeError(f"oracle idx_pool_block -> {rc}")
    return out


def max_selected(cfg, max_seq_len: int) -> int:
    s = shape_of(cfg)
    return int(lib().qwfn_oracle_max_selected(C.byref(s), max_seq_len))


def quant_offset(cfg, g: int, row: int, d: int, which: int = 0) -> int:
    s = shape_of(cfg)
    return int(lib().qwfn_oracle_quant_offset(C.byref(s), which, g, row, d))


def scale_offset(cfg, g: int, row: int, j: int) -> int:
    s = shape_of(cfg)
    return int(lib().qwfn_oracle_scale_offset(C.byref(s), g, row, j))
