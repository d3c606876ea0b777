"""Host-side mirror of the reference's KV-cache / QSA decode interface.

The reference engine owns the per-layer caches in ``qwfn::state``
(/root/reference src/qwfn_state.cpp:18-96) and the pooled block keys in
``engine`` (src/qwfn_engine.cpp:382-435); ``graph_builder::sparse_attn_decode``
(src/qwfn_graph.cpp:450-546) appends the decode token, pools its block, scores,
selects and attends.  This module keeps those roles -- ``KvState`` owns the
device memory of every attention layer, the functions below issue the same
steps -- but every step is one call into the C ABI of libqwfn_qsa.so
(include/qwfn_qsa.h).  torch is used for device memory and streams only.

Every function takes device tensors and enqueues on the current HIP stream
(or ``stream=``); nothing here synchronises except :func:`read_status`.
"""
from __future__ import annotations

import ctypes as C
from dataclasses import dataclass, field
from typing import List, Optional, Sequence

import torch

from . import _lib
from ._lib import IdxShape, IdxView, KvView, QsaShape, call

__all__ = [
    "QsaConfig", "KvCache", "KvState", "Workspace",
    "append_q8_0", "pool_update", "pool_rebuild", "indexer_topk", "gather_dequant",
    "sparse_decode_attn", "decode_append_select", "sparse_attn_decode", "sparse_attn_prefill",
    "export_rows_q8_0", "import_rows_q8_0", "read_status", "time_next_call",
    "IdxConfig", "IdxCache", "idx_append_pool", "idx_pool_rebuild", "idx_select", "idx_sparse_attn_prefill",
    "checkpoint_config",
]


@dataclass(frozen=True)
class QsaConfig:
    """Shape of the sparse-attention layer (the reference's hparams subset,
    src/qwfn_hparams.h:22-36, generalised: BASELINE pools K itself in 64-token
    blocks and keeps top-64 blocks + block 0 + the last 512 tokens)."""
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
    quant_variant: int = _lib.Q8_X86_RNE
    topk_counts_forced: int = 0
    kv_type: int = _lib.KV_Q8_0
    kv_round_f16: int = 0          # 1: decode attention on fp16-rounded K/V (the reference's F16 cast)

    @property
    def group(self) -> int:
        return self.n_head // self.n_head_kv

    @property
    def kv_dim(self) -> int:
        return self.n_head_kv * self.head_dim

    def shape(self) -> QsaShape:
        return QsaShape(self.n_head, self.n_head_kv, self.head_dim, self.block_tokens,
                        self.page_tokens, self.top_k_blocks, self.sink_blocks,
                        self.local_tokens, self.relu_per_head, self.shared_selection,
                        self.quant_variant, self.topk_counts_forced, self.kv_type, self.kv_round_f16)

    def check(self) -> None:
        s = self.shape()
        call("qwfn_qsa_check_shape", C.byref(s))

    def page_bytes(self) -> int:
        out = C.c_size_t()
        s = self.shape()
        call("qwfn_qsa_page_bytes", C.byref(s), C.byref(out))
        return out.value

    def max_selected(self, max_seq_len: int) -> int:
        out = C.c_int32()
        s = self.shape()
        call("qwfn_qsa_max_selected", C.byref(s), max_seq_len, C.byref(out))
        return out.value

    def workspace_bytes(self, n_seq: int, max_seq_len: int) -> int:
        out = C.c_size_t()
        s = self.shape()
        call("qwfn_qsa_workspace_bytes", C.byref(s), n_seq, max_seq_len, C.byref(out))
        return out.value

    def row_bytes(self) -> int:
        """Bytes of one token's row in the reference's q8_0 cache tensor
        (n_head_kv * head_dim / 32 ggml blocks of 34 bytes)."""
        out = C.c_size_t()
        s = self.shape()
        call("qwfn_kv_row_bytes", C.byref(s), C.byref(out))
        return out.value

    def prefill_workspace_bytes(self, max_seq_len: int, q_batch: int) -> int:
        out = C.c_size_t()
        s = self.shape()
        call("qwfn_qsa_prefill_workspace_bytes", C.byref(s), max_seq_len, q_batch, C.byref(out))
        return out.value

    def dense(self) -> "QsaConfig":
        """The same layer with the selection switched off (the reference's
        ``qsa == nullptr`` dense path, src/qwfn_graph.cpp:85-89)."""
        return QsaConfig(**{**self.__dict__, "top_k_blocks": 0})


def _ptr(t: Optional[torch.Tensor]) -> Optional[int]:
    return None if t is None else t.data_ptr()


def _stream(stream) -> int:
    if stream is None:
        return torch.cuda.current_stream().cuda_stream
    if isinstance(stream, torch.cuda.Stream):
        return stream.cuda_stream
    return int(stream)


def _need(t: torch.Tensor, name: str, dtype: torch.dtype, numel: Optional[int] = None) -> None:
    if not isinstance(t, torch.Tensor):
        raise TypeError(f"{name} must be a torch.Tensor")
    if t.device.type != "cuda":
        raise ValueError(f"{name} must be a device tensor, got {t.device}")
    if t.dtype != dtype:
        raise TypeError(f"{name} must be {dtype}, got {t.dtype}")
    if not t.is_contiguous():
        raise ValueError(f"{name} must be contiguous")
    if numel is not None and t.numel() != numel:
        raise ValueError(f"{name} has {t.numel()} elements, expected {numel}")


@dataclass
class KvCache:
    """One attention layer's paged q8_0 K/V pools and pooled block keys.

    ``page_table[s, p]`` is the physical page of logical page p of sequence s.
    Pages hold K quants in 16-byte chunks of 64-token tiles, V quants dim-major
    per tile (q8_0 in whole 64-token blocks) and the fp16 scales in a region
    of their own, so the reference's token-major block_q8_0 rows
    (src/qwfn_state.cpp:52-54) enter and leave through export_rows_q8_0 /
    import_rows_q8_0."""
    cfg: QsaConfig
    k_pages: torch.Tensor
    v_pages: torch.Tensor
    pooled: torch.Tensor
    page_table: torch.Tensor
    status: torch.Tensor
    _view: KvView = field(default=None, repr=False)

    @classmethod
    def allocate(cls, cfg: QsaConfig, n_seq: int, pages_per_seq: int,
                 page_table: Optional[torch.Tensor] = None, n_phys_pages: Optional[int] = None,
                 device="cuda") -> "KvCache":
        cfg.check()
        if page_table is None:
            page_table = torch.arange(n_seq * pages_per_seq, dtype=torch.int32).view(n_seq, pages_per_seq)
        page_table = page_table.to(device=device, dtype=torch.int32).contiguous()
        if tuple(page_table.shape) != (n_seq, pages_per_seq):
            raise ValueError(f"page_table shape {tuple(page_table.shape)} != ({n_seq}, {pages_per_seq})")
        if n_phys_pages is None:
            n_phys_pages = n_seq * pages_per_seq
        pb = cfg.page_bytes()
        bps = pages_per_seq * cfg.page_tokens // cfg.block_tokens
        # The reference leaves its caches unzeroed (src/qwfn_state.cpp:89); zeros
        # here only make never-written rows deterministic.
        k = torch.zeros(n_phys_pages * pb, dtype=torch.uint8, device=device)
        v = torch.zeros(n_phys_pages * pb, dtype=torch.uint8, device=device)
        pooled = torch.zeros((n_seq, cfg.n_head_kv, bps, cfg.head_dim), dtype=torch.float32, device=device)
        status = torch.zeros(1, dtype=torch.int32, device=device)
        return cls(cfg, k, v, pooled, page_table, status)

    @property
    def n_seq(self) -> int:
        return self.page_table.shape[0]

    @property
    def pages_per_seq(self) -> int:
        return self.page_table.shape[1]

    @property
    def capacity(self) -> int:
        return self.pages_per_seq * self.cfg.page_tokens

    @property
    def n_phys_pages(self) -> int:
        return self.k_pages.numel() // self.cfg.page_bytes()

    def view(self) -> KvView:
        if self._view is None:
            self._view = KvView(self.k_pages.data_ptr(), self.v_pages.data_ptr(),
                                self.pooled.data_ptr(), self.page_table.data_ptr(),
                                self.status.data_ptr(), self.n_seq, self.pages_per_seq,
                                self.n_phys_pages)
        return self._view


class KvState:
    """Per-sequence-batch state of every sparse-attention layer: the
    reference's ``state`` (K/V caches, src/qwfn_state.cpp:18-96) plus the
    engine's pooled-key caches (src/qwfn_engine.cpp:382-435)."""

    def __init__(self, cfg: QsaConfig, n_layer: int, n_ctx: int, n_seq: int = 1,
                 page_table: Optional[torch.Tensor] = None, device="cuda"):
        if n_ctx % cfg.page_tokens:
            raise ValueError(f"n_ctx {n_ctx} must be a multiple of page_tokens {cfg.page_tokens}")
        self.cfg = cfg
        self.n_ctx = n_ctx
        pps = n_ctx // cfg.page_tokens
        self.layers: List[KvCache] = [
            KvCache.allocate(cfg, n_seq, pps, page_table=page_table, device=device)
            for _ in range(n_layer)]

    def k_cache(self, il: int) -> torch.Tensor:
        return self.layers[il].k_pages

    def v_cache(self, il: int) -> torch.Tensor:
        return self.layers[il].v_pages

    def pool_cache(self, il: int) -> torch.Tensor:
        return self.layers[il].pooled

    def reset(self) -> None:
        """The reference's reset leaves the caches alone and invalidates the
        pooled keys (src/qwfn_engine.cpp:716-725); rows are rewritten as the
        positions are decoded again, so nothing needs clearing here."""
        for c in self.layers:
            c.status.zero_()

    def bytes(self) -> int:
        return sum(c.k_pages.numel() + c.v_pages.numel() + c.pooled.numel() * 4 for c in self.layers)


class Workspace:
    """Caller-owned scratch of the indexer and the attention merge, sized for
    (n_seq, max_seq_len) and zero-initialised once (a fill kernel)."""

    def __init__(self, cfg: QsaConfig, n_seq: int, max_seq_len: int, device="cuda", stream=None,
                 nbytes: Optional[int] = None):
        self.nbytes = cfg.workspace_bytes(n_seq, max_seq_len) if nbytes is None else nbytes
        self.buf = torch.empty(self.nbytes, dtype=torch.uint8, device=device)
        call("qwfn_qsa_workspace_init", self.buf.data_ptr(), self.nbytes, _stream(stream))

    @classmethod
    def for_prefill(cls, cfg: QsaConfig, max_seq_len: int, q_batch: int, device="cuda",
                    stream=None) -> "Workspace":
        """Workspace for :func:`sparse_attn_prefill` taking q_batch queries per launch pair."""
        return cls(cfg, 1, max_seq_len, device, stream, nbytes=cfg.prefill_workspace_bytes(max_seq_len, q_batch))

    def ptr(self) -> int:
        return self.buf.data_ptr()


def append_q8_0(cache: KvCache, k: torch.Tensor, v: torch.Tensor, pos: torch.Tensor,
                seq_ids: Optional[torch.Tensor] = None, stream=None) -> None:
    """ggml_set_rows / ggml_cpy into the q8_0 cache (src/qwfn_graph.cpp:520-528,
    349-360): rows k, v [n_rows, n_head_kv, head_dim] (f32 or f16) written at
    positions ``pos`` (int32, device) of ``seq_ids`` (default 0)."""
    cfg = cache.cfg
    if k.dtype not in (torch.float32, torch.float16) or v.dtype != k.dtype:
        raise TypeError("k and v must both be float32 or both float16")
    n_rows = pos.numel()
    _need(k, "k", k.dtype, n_rows * cfg.kv_dim)
    _need(v, "v", k.dtype, n_rows * cfg.kv_dim)
    _need(pos, "pos", torch.int32)
    if seq_ids is not None:
        _need(seq_ids, "seq_ids", torch.int32, n_rows)
    s = cfg.shape()
    call("qwfn_kv_append_q8_0", C.byref(s), C.byref(cache.view()), k.data_ptr(), v.data_ptr(),
         _lib.SRC_F16 if k.dtype == torch.float16 else _lib.SRC_F32, _ptr(seq_ids), pos.data_ptr(),
         n_rows, _stream(stream))


def pool_update(cache: KvCache, block_ids: torch.Tensor, seq_ids: Optional[torch.Tensor] = None,
                stream=None) -> None:
    """Recompute the pooled keys of the listed blocks (src/qwfn_graph.cpp:471-476)."""
    _need(block_ids, "block_ids", torch.int32)
    if seq_ids is not None:
        _need(seq_ids, "seq_ids", torch.int32, block_ids.numel())
    s = cache.cfg.shape()
    call("qwfn_pool_update", C.byref(s), C.byref(cache.view()), _ptr(seq_ids), block_ids.data_ptr(),
         block_ids.numel(), _stream(stream))


def pool_rebuild(cache: KvCache, seq: int, n_whole: int, stream=None) -> None:
    """qsa_pool_rebuild after a prefill: pool blocks [0, n_whole) of ``seq``
    (src/qwfn_graph.cpp:431-448, src/qwfn_engine.cpp:761-798)."""
    s = cache.cfg.shape()
    call("qwfn_pool_rebuild", C.byref(s), C.byref(cache.view()), seq, n_whole, _stream(stream))


def export_rows_q8_0(cache: KvCache, seq: int, pos0: int, n_tokens: int, k: bool = True, v: bool = True,
                     stream=None):
    """Positions [pos0, pos0+n_tokens) of ``seq`` as the reference's cache rows:
    uint8 [n_tokens, row_bytes] device tensors, row t = the token's ggml
    block_q8_0 blocks, head-major (src/qwfn_state.cpp:40, 52-53).  Returns
    (k_rows, v_rows); a side not asked for is None."""
    cfg = cache.cfg
    rb = cfg.row_bytes()
    dev = cache.k_pages.device
    kr = torch.empty((n_tokens, rb), dtype=torch.uint8, device=dev) if k else None
    vr = torch.empty((n_tokens, rb), dtype=torch.uint8, device=dev) if v else None
    s = cfg.shape()
    call("qwfn_kv_export_q8_0", C.byref(s), C.byref(cache.view()), seq, pos0, n_tokens, _ptr(kr), _ptr(vr),
         _stream(stream))
    return kr, vr


def import_rows_q8_0(cache: KvCache, seq: int, pos0: int, k_rows: Optional[torch.Tensor],
                     v_rows: Optional[torch.Tensor], stream=None) -> None:
    """Write the reference's cache rows (uint8 [n_tokens, row_bytes], device)
    into positions [pos0, pos0+n_tokens) of ``seq``, byte for byte.  The pooled
    keys are left alone: pool the completed blocks afterwards
    (:func:`pool_rebuild` / :func:`pool_update`)."""
    cfg = cache.cfg
    rb = cfg.row_bytes()
    ref = k_rows if k_rows is not None else v_rows
    if ref is None:
        raise ValueError("import_rows_q8_0: k_rows and v_rows are both None")
    n_tokens = ref.numel() // rb
    for t, name in ((k_rows, "k_rows"), (v_rows, "v_rows")):
        if t is not None:
            _need(t, name, torch.uint8, n_tokens * rb)
    s = cfg.shape()
    call("qwfn_kv_import_q8_0", C.byref(s), C.byref(cache.view()), seq, pos0, n_tokens, _ptr(k_rows),
         _ptr(v_rows), _stream(stream))


def indexer_topk(cache: KvCache, q: torch.Tensor, seq_len: torch.Tensor, max_seq_len: int,
                 ws: Workspace, sel: Optional[torch.Tensor] = None,
                 n_sel: Optional[torch.Tensor] = None, stream=None):
    """Scores + top-k of one decode token per sequence (src/qwfn_graph.cpp:477-495).
    Returns (sel [n_seq, n_head_kv, max_sel] ascending block ids, n_sel [n_seq, n_head_kv])."""
    cfg = cache.cfg
    n_seq = seq_len.numel()
    _need(q, "q", torch.float32, n_seq * cfg.n_head * cfg.head_dim)
    _need(seq_len, "seq_len", torch.int32)
    max_sel = cfg.max_selected(max_seq_len)
    if sel is None:
        sel = torch.empty((n_seq, cfg.n_head_kv, max_sel), dtype=torch.int32, device=q.device)
    if n_sel is None:
        n_sel = torch.empty((n_seq, cfg.n_head_kv), dtype=torch.int32, device=q.device)
    _need(sel, "sel", torch.int32)
    _need(n_sel, "n_sel", torch.int32, n_seq * cfg.n_head_kv)
    s = cfg.shape()
    call("qwfn_indexer_topk", C.byref(s), C.byref(cache.view()), q.data_ptr(), seq_len.data_ptr(), n_seq,
         max_seq_len, sel.data_ptr(), n_sel.data_ptr(), sel.shape[-1], ws.ptr(), ws.nbytes, _stream(stream))
    return sel, n_sel


def gather_dequant(cache: KvCache, seq_len: torch.Tensor, sel: Optional[torch.Tensor],
                   n_sel: Optional[torch.Tensor], max_sel: int, stream=None):
    """Dequantized cells of a selection (src/qwfn_graph.cpp:494-495, 530-537):
    (k [n_seq, Hkv, max_sel*bt, hd], v, cells [n_seq, Hkv, max_sel*bt])."""
    cfg = cache.cfg
    n_seq = seq_len.numel()
    nc = max_sel * cfg.block_tokens
    dev = seq_len.device
    k = torch.empty((n_seq, cfg.n_head_kv, nc, cfg.head_dim), dtype=torch.float32, device=dev)
    v = torch.empty_like(k)
    cells = torch.empty((n_seq, cfg.n_head_kv, nc), dtype=torch.int32, device=dev)
    s = cfg.shape()
    call("qwfn_gather_dequant", C.byref(s), C.byref(cache.view()), seq_len.data_ptr(), n_seq, _ptr(sel),
         _ptr(n_sel), max_sel, k.data_ptr(), v.data_ptr(), cells.data_ptr(), _stream(stream))
    return k, v, cells


def sparse_decode_attn(cache: KvCache, q: torch.Tensor, seq_len: torch.Tensor, max_seq_len: int,
                       ws: Workspace, sel: Optional[torch.Tensor] = None,
                       n_sel: Optional[torch.Tensor] = None, out: Optional[torch.Tensor] = None,
                       stream=None) -> torch.Tensor:
    """Masked GQA softmax attention over a selection (sel None: dense), the
    reference's cell mask + ggml_flash_attn_ext (src/qwfn_graph.cpp:497-542)."""
    cfg = cache.cfg
    n_seq = seq_len.numel()
    _need(q, "q", torch.float32, n_seq * cfg.n_head * cfg.head_dim)
    if out is None:
        out = torch.empty((n_seq, cfg.n_head, cfg.head_dim), dtype=torch.float32, device=q.device)
    _need(out, "out", torch.float32, n_seq * cfg.n_head * cfg.head_dim)
    max_sel = sel.shape[-1] if sel is not None else 0
    s = cfg.shape()
    call("qwfn_sparse_decode_attn", C.byref(s), C.byref(cache.view()), q.data_ptr(), seq_len.data_ptr(),
         n_seq, max_seq_len, _ptr(sel), _ptr(n_sel), max_sel, out.data_ptr(), ws.ptr(), ws.nbytes,
         _stream(stream))
    return out


def sparse_attn_decode(cache: KvCache, q: torch.Tensor, k_new: torch.Tensor, v_new: torch.Tensor,
                       seq_len: torch.Tensor, max_seq_len: int, ws: Workspace,
                       out: Optional[torch.Tensor] = None, sel: Optional[torch.Tensor] = None,
                       n_sel: Optional[torch.Tensor] = None, stream=None) -> torch.Tensor:
    """One decode token of graph_builder::sparse_attn_decode
    (src/qwfn_graph.cpp:450-546) from the projections on: append k_new/v_new at
    seq_len-1, pool the block it completes, select, attend.  ``sel``/``n_sel``
    (optional, both or neither) receive the selection."""
    cfg = cache.cfg
    n_seq = seq_len.numel()
    _need(q, "q", torch.float32, n_seq * cfg.n_head * cfg.head_dim)
    if k_new.dtype not in (torch.float32, torch.float16) or v_new.dtype != k_new.dtype:
        raise TypeError("k_new and v_new must both be float32 or both float16")
    _need(k_new, "k_new", k_new.dtype, n_seq * cfg.kv_dim)
    _need(v_new, "v_new", k_new.dtype, n_seq * cfg.kv_dim)
    _need(seq_len, "seq_len", torch.int32)
    if out is None:
        out = torch.empty((n_seq, cfg.n_head, cfg.head_dim), dtype=torch.float32, device=q.device)
    if (sel is None) != (n_sel is None):
        raise ValueError("pass both sel and n_sel or neither")
    if sel is not None:                            # the kernels write max_selected entries a (sequence, KV head)
        _need(sel, "sel", torch.int32, n_seq * cfg.n_head_kv * cfg.max_selected(max_seq_len))
        _need(n_sel, "n_sel", torch.int32, n_seq * cfg.n_head_kv)
    s = cfg.shape()
    call("qwfn_sparse_attn_decode", C.byref(s), C.byref(cache.view()), q.data_ptr(), k_new.data_ptr(),
         v_new.data_ptr(), _lib.SRC_F16 if k_new.dtype == torch.float16 else _lib.SRC_F32,
         seq_len.data_ptr(), n_seq, max_seq_len, out.data_ptr(), _ptr(sel), _ptr(n_sel), ws.ptr(),
         ws.nbytes, _stream(stream))
    return out


def sparse_attn_decode_chain(cache: KvCache, q: torch.Tensor, k_new: torch.Tensor, v_new: torch.Tensor,
                             seq_len: torch.Tensor, max_seq_len: int, ws: Workspace,
                             out: Optional[torch.Tensor] = None, sel: Optional[torch.Tensor] = None,
                             n_sel: Optional[torch.Tensor] = None, stream=None) -> torch.Tensor:
    """n_pos chained decode positions of every sequence in one call, the
    multi-position decode of the MTP verify step (src/qwfn_engine.cpp:1892-1906):
    q [n_pos][n_seq][n_head][head_dim], k_new / v_new [n_pos][n_seq][n_head_kv]
    [head_dim]; position k appends at seq_len - 1 + k and attends with length
    seq_len + k, reading through the writes of the positions before it.
    ``sel`` [n_pos][n_seq][n_head_kv][max_selected] / ``n_sel`` [n_pos][n_seq]
    [n_head_kv] (optional, both or neither) receive each position's selection."""
    cfg = cache.cfg
    n_seq = seq_len.numel()
    if q.dim() != 4 or q.shape[1] != n_seq:
        raise ValueError("q must be [n_pos][n_seq][n_head][head_dim]")
    n_pos = q.shape[0]
    _need(q, "q", torch.float32, n_pos * n_seq * cfg.n_head * cfg.head_dim)
    if k_new.dtype not in (torch.float32, torch.float16) or v_new.dtype != k_new.dtype:
        raise TypeError("k_new and v_new must both be float32 or both float16")
    _need(k_new, "k_new", k_new.dtype, n_pos * n_seq * cfg.kv_dim)
    _need(v_new, "v_new", k_new.dtype, n_pos * n_seq * cfg.kv_dim)
    _need(seq_len, "seq_len", torch.int32)
    if out is None:
        out = torch.empty((n_pos, n_seq, cfg.n_head, cfg.head_dim), dtype=torch.float32, device=q.device)
    _need(out, "out", torch.float32, n_pos * n_seq * cfg.n_head * cfg.head_dim)
    if (sel is None) != (n_sel is None):
        raise ValueError("pass both sel and n_sel or neither")
    if sel is not None:
        _need(sel, "sel", torch.int32, n_pos * n_seq * cfg.n_head_kv * cfg.max_selected(max_seq_len))
        _need(n_sel, "n_sel", torch.int32, n_pos * n_seq * cfg.n_head_kv)
    s = cfg.shape()
    call("qwfn_sparse_attn_decode_chain", C.byref(s), C.byref(cache.view()), q.data_ptr(), k_new.data_ptr(),
         v_new.data_ptr(), _lib.SRC_F16 if k_new.dtype == torch.float16 else _lib.SRC_F32,
         seq_len.data_ptr(), n_seq, n_pos, max_seq_len, out.data_ptr(), _ptr(sel), _ptr(n_sel), ws.ptr(),
         ws.nbytes, _stream(stream))
    return out


def sparse_attn_decode_noalloc(cache: KvCache, q: torch.Tensor, k_new: torch.Tensor, v_new: torch.Tensor,
                               seq_len: torch.Tensor, max_seq_len: int, out: torch.Tensor,
                               sel: Optional[torch.Tensor] = None, n_sel: Optional[torch.Tensor] = None,
                               stream=None) -> torch.Tensor:
    """:func:`sparse_attn_decode` without a workspace: the library's own
    per-device scratch array serves as one (qwfn_sparse_attn_decode_noalloc).
    ``out`` is required, so the call allocates nothing."""
    cfg = cache.cfg
    n_seq = seq_len.numel()
    _need(q, "q", torch.float32, n_seq * cfg.n_head * cfg.head_dim)
    if k_new.dtype not in (torch.float32, torch.float16) or v_new.dtype != k_new.dtype:
        raise TypeError("k_new and v_new must both be float32 or both float16")
    _need(k_new, "k_new", k_new.dtype, n_seq * cfg.kv_dim)
    _need(v_new, "v_new", k_new.dtype, n_seq * cfg.kv_dim)
    _need(seq_len, "seq_len", torch.int32)
    _need(out, "out", torch.float32, n_seq * cfg.n_head * cfg.head_dim)
    if (sel is None) != (n_sel is None):
        raise ValueError("pass both sel and n_sel or neither")
    if sel is not None:                            # the kernels write max_selected entries a (sequence, KV head)
        _need(sel, "sel", torch.int32, n_seq * cfg.n_head_kv * cfg.max_selected(max_seq_len))
        _need(n_sel, "n_sel", torch.int32, n_seq * cfg.n_head_kv)
    s = cfg.shape()
    call("qwfn_sparse_attn_decode_noalloc", C.byref(s), C.byref(cache.view()), q.data_ptr(), k_new.data_ptr(),
         v_new.data_ptr(), _lib.SRC_F16 if k_new.dtype == torch.float16 else _lib.SRC_F32,
         seq_len.data_ptr(), n_seq, max_seq_len, out.data_ptr(), _ptr(sel), _ptr(n_sel), _stream(stream))
    return out


def sparse_attn_prefill(cache: KvCache, q: torch.Tensor, seq: int, pos0: int, ws: Workspace,
                        k_new: Optional[torch.Tensor] = None, v_new: Optional[torch.Tensor] = None,
                        out: Optional[torch.Tensor] = None, sel: Optional[torch.Tensor] = None,
                        n_sel: Optional[torch.Tensor] = None, stream=None) -> torch.Tensor:
    """Prefill chunk of sequence ``seq`` at positions pos0 .. pos0+n_q-1, the QSA
    part of graph_builder::sparse_attn / qsa_top_k (src/qwfn_graph.cpp:235-408).
    ``k_new``/``v_new`` ([n_q][n_head_kv][head_dim]), when given, are appended
    and the blocks they complete re-pooled first.  Query i attends as a decode
    step at seq_len = pos0 + i + 1.  ``sel``/``n_sel`` (optional, both or
    neither; sel [n_q][n_head_kv][max_sel]) receive every query's selection."""
    cfg = cache.cfg
    n_q = q.numel() // (cfg.n_head * cfg.head_dim)
    _need(q, "q", torch.float32, n_q * cfg.n_head * cfg.head_dim)
    src = _lib.SRC_F32
    if (k_new is None) != (v_new is None):
        raise ValueError("pass both k_new and v_new or neither")
    if k_new is not None:
        if k_new.dtype not in (torch.float32, torch.float16) or v_new.dtype != k_new.dtype:
            raise TypeError("k_new and v_new must both be float32 or both float16")
        _need(k_new, "k_new", k_new.dtype, n_q * cfg.kv_dim)
        _need(v_new, "v_new", k_new.dtype, n_q * cfg.kv_dim)
        src = _lib.SRC_F16 if k_new.dtype == torch.float16 else _lib.SRC_F32
    if out is None:
        out = torch.empty((n_q, cfg.n_head, cfg.head_dim), dtype=torch.float32, device=q.device)
    if (sel is None) != (n_sel is None):
        raise ValueError("pass both sel and n_sel or neither")
    max_sel = 0
    if sel is not None:
        _need(sel, "sel", torch.int32)
        _need(n_sel, "n_sel", torch.int32, n_q * cfg.n_head_kv)
        max_sel = sel.shape[-1]
    s = cfg.shape()
    call("qwfn_sparse_attn_prefill", C.byref(s), C.byref(cache.view()), q.data_ptr(), _ptr(k_new), _ptr(v_new),
         src, seq, pos0, n_q, out.data_ptr(), _ptr(sel), _ptr(n_sel), max_sel, ws.ptr(), ws.nbytes,
         _stream(stream))
    return out


def decode_append_select(cache: KvCache, q: torch.Tensor, k_new: torch.Tensor, v_new: torch.Tensor,
                         seq_len: torch.Tensor, max_seq_len: int, ws: Workspace, sel: torch.Tensor,
                         n_sel: torch.Tensor, stream=None) -> None:
    """The first launch of :func:`sparse_attn_decode`: append at seq_len-1, pool
    on block completion, score and select into sel / n_sel
    (src/qwfn_graph.cpp:465-495, 520-528)."""
    cfg = cache.cfg
    n_seq = seq_len.numel()
    _need(q, "q", torch.float32, n_seq * cfg.n_head * cfg.head_dim)
    if k_new.dtype not in (torch.float32, torch.float16) or v_new.dtype != k_new.dtype:
        raise TypeError("k_new and v_new must both be float32 or both float16")
    _need(k_new, "k_new", k_new.dtype, n_seq * cfg.kv_dim)
    _need(v_new, "v_new", k_new.dtype, n_seq * cfg.kv_dim)
    _need(seq_len, "seq_len", torch.int32)
    _need(sel, "sel", torch.int32)
    _need(n_sel, "n_sel", torch.int32, n_seq * cfg.n_head_kv)
    s = cfg.shape()
    call("qwfn_decode_append_select", C.byref(s), C.byref(cache.view()), q.data_ptr(), k_new.data_ptr(),
         v_new.data_ptr(), _lib.SRC_F16 if k_new.dtype == torch.float16 else _lib.SRC_F32,
         seq_len.data_ptr(), n_seq, max_seq_len, sel.data_ptr(), n_sel.data_ptr(), sel.shape[-1], ws.ptr(),
         ws.nbytes, _stream(stream))


def read_status(cache: KvCache, stream=None) -> int:
    """Fetch and clear the device status bits of a cache (synchronises)."""
    out = C.c_int32()
    call("qwfn_qsa_read_status", C.byref(cache.view()), C.byref(out), _stream(stream))
    return out.value


TIMED_KERNELS = ("indexer", "attention", "merge")


def time_next_call(events: Optional[dict] = None) -> None:
    """Arm per-kernel timing of the next decode call on this thread
    (qwfn_qsa_time_next_call).  ``events`` maps names of TIMED_KERNELS to
    (start, end) pairs of ``torch.cuda.Event(enable_timing=True)``; after the
    stream completes, ``start.elapsed_time(end)`` is that kernel's own
    duration.  torch creates an event's handle at its first record, so each
    event must have been recorded once.  None disarms."""
    arr = (C.c_void_p * 6)()
    for k, name in enumerate(TIMED_KERNELS):
        pair = (events or {}).get(name)
        if pair is None:
            continue
        for j, ev in enumerate(pair):
            h = ev.cuda_event
            if not h:
                raise ValueError(f"time_next_call: the {name} event {j} has no handle yet (record it once)")
            arr[2 * k + j] = h
    call("qwfn_qsa_time_next_call", arr)


# ---- the checkpoint's own indexer ------------------------------------------

@dataclass(frozen=True)
class IdxConfig:
    """The released checkpoint's lightning indexer (src/qwfn_hparams.h:35, 52-53;
    src/qwfn_graph.cpp:233-305, 410-495): raw keys of idx_dim values per token,
    n_idx_head query heads, blocks pooled with RMSNorm * k_norm and rotated on
    their first rope_dim dims."""
    idx_dim: int = 128
    n_idx_head: int = 4
    rope_dim: int = 64
    rope_freq_base: float = 10000000.0
    rms_eps: float = 1e-6

    def shape(self) -> IdxShape:
        return IdxShape(self.idx_dim, self.n_idx_head, self.rope_dim, self.rope_freq_base, self.rms_eps)


def checkpoint_config(idx_top_k: int = 2048, ratio: int = 4, page_tokens: int = 256,
                      quant_variant: int = _lib.Q8_X86_RNE) -> QsaConfig:
    """The attention layer of the released checkpoint (src/qwfn_hparams.h:22-26,
    52-54): 24 query heads, 2 KV heads of 256, blocks of ``ratio`` tokens,
    k_blocks = ceil((idx_top_k + ratio - 1) / ratio) kept blocks in all
    (src/qwfn_engine.cpp:430), only a partial tail block forced
    (:748-753), relu per indexer head, one selection for both KV heads."""
    kb = (idx_top_k + ratio - 1 + ratio - 1) // ratio
    return QsaConfig(n_head=24, n_head_kv=2, head_dim=256, block_tokens=ratio, page_tokens=page_tokens,
                     top_k_blocks=kb, sink_blocks=0, local_tokens=0, relu_per_head=1, shared_selection=1,
                     quant_variant=quant_variant, topk_counts_forced=1)


@dataclass
class IdxCache:
    """One attention layer's indexer keys, paged by a :class:`KvCache`'s page
    table: raw fp16 keys [n_phys_pages, page_tokens, idx_dim] (the reference's
    idx cache) and the pooled block keys [n_seq, blocks_per_seq, idx_dim] (its
    F16 pool cache), plus k_norm [idx_dim]."""
    icfg: IdxConfig
    kv: KvCache
    raw: torch.Tensor
    pooled: torch.Tensor
    k_norm: torch.Tensor
    _view: IdxView = field(default=None, repr=False)

    @classmethod
    def allocate(cls, icfg: IdxConfig, kv: KvCache, k_norm: torch.Tensor) -> "IdxCache":
        cfg = kv.cfg
        rpb, pb = C.c_size_t(), C.c_size_t()
        call("qwfn_idx_cache_bytes", C.byref(cfg.shape()), C.byref(icfg.shape()), kv.n_seq, kv.pages_per_seq,
             C.byref(rpb), C.byref(pb))
        dev = kv.k_pages.device
        raw = torch.zeros((kv.n_phys_pages, cfg.page_tokens, icfg.idx_dim), dtype=torch.float16, device=dev)
        bps = kv.pages_per_seq * cfg.page_tokens // cfg.block_tokens
        pooled = torch.zeros((kv.n_seq, bps, icfg.idx_dim), dtype=torch.float16, device=dev)
        assert raw.numel() * 2 == rpb.value * kv.n_phys_pages and pooled.numel() * 2 == pb.value
        k_norm = k_norm.to(device=dev, dtype=torch.float32).contiguous()
        _need(k_norm, "k_norm", torch.float32, icfg.idx_dim)
        return cls(icfg, kv, raw, pooled, k_norm)

    def view(self) -> IdxView:
        if self._view is None:
            self._view = IdxView(self.raw.data_ptr(), self.pooled.data_ptr(), self.k_norm.data_ptr())
        return self._view

    def workspace_bytes(self, n_seq: int, max_seq_len: int) -> int:
        out = C.c_size_t()
        call("qwfn_idx_workspace_bytes", C.byref(self.kv.cfg.shape()), C.byref(self.icfg.shape()), n_seq,
             max_seq_len, C.byref(out))
        return out.value


def idx_append_pool(ic: IdxCache, k_raw: torch.Tensor, pos: torch.Tensor,
                    seq_ids: Optional[torch.Tensor] = None, stream=None) -> None:
    """The decode step's raw indexer key (src/qwfn_graph.cpp:463-470) and the
    re-pooled block holding it (:471-476): rows k_raw [n_rows, idx_dim] (f32
    or f16) at ``pos`` of ``seq_ids`` (default 0)."""
    n_rows = pos.numel()
    if k_raw.dtype not in (torch.float32, torch.float16):
        raise TypeError("k_raw must be float32 or float16")
    _need(k_raw, "k_raw", k_raw.dtype, n_rows * ic.icfg.idx_dim)
    _need(pos, "pos", torch.int32)
    if seq_ids is not None:
        _need(seq_ids, "seq_ids", torch.int32, n_rows)
    call("qwfn_idx_append_pool", C.byref(ic.kv.cfg.shape()), C.byref(ic.kv.view()), C.byref(ic.icfg.shape()),
         C.byref(ic.view()), k_raw.data_ptr(), _lib.SRC_F16 if k_raw.dtype == torch.float16 else _lib.SRC_F32,
         _ptr(seq_ids), pos.data_ptr(), n_rows, _stream(stream))


def idx_pool_rebuild(ic: IdxCache, seq: int, n_whole: int, stream=None) -> None:
    """Pool the indexer keys of blocks [0, n_whole) of ``seq`` (qsa_pool_rebuild,
    src/qwfn_graph.cpp:431-448)."""
    call("qwfn_idx_pool_rebuild", C.byref(ic.kv.cfg.shape()), C.byref(ic.kv.view()), C.byref(ic.icfg.shape()),
         C.byref(ic.view()), seq, n_whole, _stream(stream))


def idx_select(ic: IdxCache, q_idx: torch.Tensor, seq_len: torch.Tensor, max_seq_len: int, ws: Workspace,
               sel: Optional[torch.Tensor] = None, n_sel: Optional[torch.Tensor] = None, stream=None):
    """The checkpoint indexer's scores and top-k for one decode token per
    sequence (src/qwfn_graph.cpp:477-495): q_idx [n_seq, n_idx_head, idx_dim]
    (normed and rotated).  Returns (sel [n_seq, n_head_kv, max_sel], n_sel
    [n_seq, n_head_kv]) with one selection repeated for every KV head."""
    cfg, icfg = ic.kv.cfg, ic.icfg
    n_seq = seq_len.numel()
    _need(q_idx, "q_idx", torch.float32, n_seq * icfg.n_idx_head * icfg.idx_dim)
    _need(seq_len, "seq_len", torch.int32)
    max_sel = cfg.max_selected(max_seq_len)
    if sel is None:
        sel = torch.empty((n_seq, cfg.n_head_kv, max_sel), dtype=torch.int32, device=q_idx.device)
    if n_sel is None:
        n_sel = torch.empty((n_seq, cfg.n_head_kv), dtype=torch.int32, device=q_idx.device)
    _need(sel, "sel", torch.int32)
    _need(n_sel, "n_sel", torch.int32, n_seq * cfg.n_head_kv)
    call("qwfn_idx_select", C.byref(cfg.shape()), C.byref(ic.kv.view()), C.byref(icfg.shape()), C.byref(ic.view()),
         q_idx.data_ptr(), seq_len.data_ptr(), n_seq, max_seq_len, sel.data_ptr(), n_sel.data_ptr(), sel.shape[-1],
         ws.ptr(), ws.nbytes, _stream(stream))
    return sel, n_sel


def idx_sparse_attn_decode(ic: IdxCache, q: torch.Tensor, q_idx: torch.Tensor, k_new: torch.Tensor,
                           v_new: torch.Tensor, k_raw: torch.Tensor, seq_len: torch.Tensor, max_seq_len: int,
                           ws: Workspace, out: Optional[torch.Tensor] = None, sel: Optional[torch.Tensor] = None,
                           n_sel: Optional[torch.Tensor] = None, stream=None) -> torch.Tensor:
    """One decode token of graph_builder::sparse_attn_decode with the
    checkpoint's indexer (src/qwfn_graph.cpp:450-546): k_raw [n_seq, idx_dim]
    and k_new / v_new [n_seq, n_head_kv, head_dim] (one dtype, f32 or f16) are
    written at seq_len - 1 and the raw key's block re-pooled in one launch,
    then q_idx selects as :func:`idx_select` and q attends as
    :func:`sparse_decode_attn`.  ``sel`` / ``n_sel`` receive the selection
    (allocated here when not given); ``ws`` must hold both the attention's and
    the indexer's workspace."""
    cache, cfg, icfg = ic.kv, ic.kv.cfg, ic.icfg
    n_seq = seq_len.numel()
    _need(q, "q", torch.float32, n_seq * cfg.n_head * cfg.head_dim)
    _need(q_idx, "q_idx", torch.float32, n_seq * icfg.n_idx_head * icfg.idx_dim)
    if k_new.dtype not in (torch.float32, torch.float16) or v_new.dtype != k_new.dtype or k_raw.dtype != k_new.dtype:
        raise TypeError("k_new, v_new and k_raw must share one dtype, float32 or float16")
    _need(k_new, "k_new", k_new.dtype, n_seq * cfg.kv_dim)
    _need(v_new, "v_new", k_new.dtype, n_seq * cfg.kv_dim)
    _need(k_raw, "k_raw", k_new.dtype, n_seq * icfg.idx_dim)
    _need(seq_len, "seq_len", torch.int32)
    max_sel = cfg.max_selected(max_seq_len)
    if sel is None:
        sel = torch.empty((n_seq, cfg.n_head_kv, max_sel), dtype=torch.int32, device=q.device)
    if n_sel is None:
        n_sel = torch.empty((n_seq, cfg.n_head_kv), dtype=torch.int32, device=q.device)
    if sel.shape[-1] < max_sel:
        raise ValueError(f"sel rows of {sel.shape[-1]} < max_selected {max_sel}")
    _need(sel, "sel", torch.int32, n_seq * cfg.n_head_kv * sel.shape[-1])
    _need(n_sel, "n_sel", torch.int32, n_seq * cfg.n_head_kv)
    if out is None:
        out = torch.empty((n_seq, cfg.n_head, cfg.head_dim), dtype=torch.float32, device=q.device)
    _need(out, "out", torch.float32, n_seq * cfg.n_head * cfg.head_dim)
    call("qwfn_idx_sparse_attn_decode", C.byref(cfg.shape()), C.byref(cache.view()), C.byref(icfg.shape()),
         C.byref(ic.view()), q.data_ptr(), q_idx.data_ptr(), k_new.data_ptr(), v_new.data_ptr(), k_raw.data_ptr(),
         _lib.SRC_F16 if k_new.dtype == torch.float16 else _lib.SRC_F32, seq_len.data_ptr(), n_seq, max_seq_len,
         out.data_ptr(), sel.data_ptr(), n_sel.data_ptr(), sel.shape[-1], ws.ptr(), ws.nbytes, _stream(stream))
    return out


def idx_sparse_attn_prefill(ic: IdxCache, q: torch.Tensor, q_idx: torch.Tensor, seq: int, pos0: int,
                            ws: Workspace, k_new: Optional[torch.Tensor] = None,
                            v_new: Optional[torch.Tensor] = None, k_raw: Optional[torch.Tensor] = None,
                            out: Optional[torch.Tensor] = None, sel: Optional[torch.Tensor] = None,
                            n_sel: Optional[torch.Tensor] = None, stream=None) -> torch.Tensor:
    """:func:`sparse_attn_prefill` with the checkpoint's indexer (qsa_top_k and
    the masked attention of graph_builder::sparse_attn, src/qwfn_graph.cpp:
    233-408): k_raw [n_q, idx_dim] (with k_new / v_new) is appended and pooled,
    query i is selected by q_idx[i] and attends causally over its selection."""
    cache, cfg, icfg = ic.kv, ic.kv.cfg, ic.icfg
    n_q = q.numel() // (cfg.n_head * cfg.head_dim)
    _need(q, "q", torch.float32, n_q * cfg.n_head * cfg.head_dim)
    _need(q_idx, "q_idx", torch.float32, n_q * icfg.n_idx_head * icfg.idx_dim)
    src = _lib.SRC_F32
    if (k_new is None) != (v_new is None):
        raise ValueError("pass both k_new and v_new or neither")
    if k_raw is not None and k_new is None:
        raise ValueError("k_raw comes with k_new / v_new")
    if k_new is not None:
        if k_new.dtype not in (torch.float32, torch.float16) or v_new.dtype != k_new.dtype:
            raise TypeError("k_new and v_new must both be float32 or both float16")
        _need(k_new, "k_new", k_new.dtype, n_q * cfg.kv_dim)
        _need(v_new, "v_new", k_new.dtype, n_q * cfg.kv_dim)
        if k_raw is not None:
            _need(k_raw, "k_raw", k_new.dtype, n_q * icfg.idx_dim)
        src = _lib.SRC_F16 if k_new.dtype == torch.float16 else _lib.SRC_F32
    if out is None:
        out = torch.empty((n_q, cfg.n_head, cfg.head_dim), dtype=torch.float32, device=q.device)
    if (sel is None) != (n_sel is None):
        raise ValueError("pass both sel and n_sel or neither")
    max_sel = 0
    if sel is not None:
        _need(sel, "sel", torch.int32)
        _need(n_sel, "n_sel", torch.int32, n_q * cfg.n_head_kv)
        max_sel = sel.shape[-1]
    call("qwfn_idx_sparse_attn_prefill", C.byref(cfg.shape()), C.byref(cache.view()), C.byref(icfg.shape()),
         C.byref(ic.view()), q.data_ptr(), q_idx.data_ptr(), _ptr(k_new), _ptr(v_new), _ptr(k_raw), src, seq,
         pos0, n_q, out.data_ptr(), _ptr(sel), _ptr(n_sel), max_sel, ws.ptr(), ws.nbytes, _stream(stream))
    return out
