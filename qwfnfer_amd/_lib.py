"""ctypes binding of libqwfn_qsa.so (declarations in include/qwfn_qsa.h).

Loading fails loudly when the library is missing: there is no CPU fallback.
"""
from __future__ import annotations

import ctypes as C
import os

LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "libqwfn_qsa.so")

QWFN_OK = 0
QWFN_EHIP = -5
QWFN_EINVAL = -22
QWFN_ERANGE = -34
QWFN_ENOTSUP = -95

Q8_X86_RNE = 0
Q8_REF_ROUNDF = 1
KV_Q8_0 = 0
KV_Q4_0 = 1
KV_F16 = 2
SRC_F32 = 0
SRC_F16 = 1

STATUS_POS_RANGE = 0x1
STATUS_SEQ_RANGE = 0x2
STATUS_PAGE_RANGE = 0x4
STATUS_LEN_RANGE = 0x8
STATUS_BLOCK_RANGE = 0x10

# every symbol include/qwfn_qsa.h declares
EXPORTS = (
    "qwfn_qsa_abi_version",
    "qwfn_qsa_last_error",
    "qwfn_qsa_time_next_call",
    "qwfn_qsa_test_prefill_scores",
    "qwfn_qsa_test_select_rows",
    "qwfn_qsa_test_set_cut_polls",
    "qwfn_qsa_check_shape",
    "qwfn_qsa_page_bytes",
    "qwfn_qsa_pooled_bytes",
    "qwfn_qsa_max_selected",
    "qwfn_qsa_workspace_bytes",
    "qwfn_qsa_workspace_init",
    "qwfn_qsa_read_status",
    "qwfn_kv_row_bytes",
    "qwfn_kv_export_q8_0",
    "qwfn_kv_import_q8_0",
    "qwfn_kv_append_q8_0",
    "qwfn_pool_update",
    "qwfn_pool_rebuild",
    "qwfn_indexer_topk",
    "qwfn_gather_dequant",
    "qwfn_sparse_decode_attn",
    "qwfn_decode_append_select",
    "qwfn_sparse_attn_decode",
    "qwfn_sparse_attn_decode_chain",
    "qwfn_sparse_attn_decode_noalloc",
    "qwfn_qsa_prefill_workspace_bytes",
    "qwfn_sparse_attn_prefill",
    "qwfn_idx_cache_bytes",
    "qwfn_idx_workspace_bytes",
    "qwfn_idx_append_pool",
    "qwfn_idx_pool_rebuild",
    "qwfn_idx_select",
    "qwfn_idx_sparse_attn_decode",
    "qwfn_idx_sparse_attn_prefill",
)


class QsaShape(C.Structure):
    _fields_ = [
        ("n_head", C.c_int32),
        ("n_head_kv", C.c_int32),
        ("head_dim", C.c_int32),
        ("block_tokens", C.c_int32),
        ("page_tokens", C.c_int32),
        ("top_k_blocks", C.c_int32),
        ("sink_blocks", C.c_int32),
        ("local_tokens", C.c_int32),
        ("relu_per_head", C.c_int32),
        ("shared_selection", C.c_int32),
        ("quant_variant", C.c_int32),
        ("topk_counts_forced", C.c_int32),
        ("kv_type", C.c_int32),
        ("kv_round_f16", C.c_int32),
    ]


class KvView(C.Structure):
    _fields_ = [
        ("k_pages", C.c_void_p),
        ("v_pages", C.c_void_p),
        ("pooled", C.c_void_p),
        ("page_table", C.c_void_p),
        ("status", C.c_void_p),
        ("n_seq", C.c_int32),
        ("pages_per_seq", C.c_int32),
        ("n_phys_pages", C.c_int32),
    ]


class IdxShape(C.Structure):
    _fields_ = [
        ("idx_dim", C.c_int32),
        ("n_idx_head", C.c_int32),
        ("rope_dim", C.c_int32),
        ("rope_freq_base", C.c_float),
        ("rms_eps", C.c_float),
    ]


class IdxView(C.Structure):
    _fields_ = [
        ("raw", C.c_void_p),
        ("pooled", C.c_void_p),
        ("k_norm", C.c_void_p),
    ]


class QsaError(RuntimeError):
    """A negative return code of the C ABI, with qwfn_qsa_last_error()."""

    def __init__(self, code: int, func: str, msg: str):
        super().__init__(f"{func} -> {code}: {msg}")
        self.code = code
        self.func = func


_lib = None

_S = C.POINTER(QsaShape)
_V = C.POINTER(KvView)
_IS = C.POINTER(IdxShape)
_IV = C.POINTER(IdxView)
_P = C.c_void_p
_I = C.c_int32
_Z = C.c_size_t

_SIGS = {
    "qwfn_qsa_abi_version": (C.c_int, []),
    "qwfn_qsa_last_error": (C.c_char_p, []),
    "qwfn_qsa_time_next_call": (C.c_int, [C.POINTER(C.c_void_p)]),
    "qwfn_qsa_test_prefill_scores": (C.c_int, [_S, _V, _P, _I, _I, _I, _P, _P, _I, _P]),
    "qwfn_qsa_test_select_rows": (C.c_int, [_S, _P, _I, _P, _I, _I, _P, _P, _I, _P]),
    "qwfn_qsa_test_set_cut_polls": (C.c_int, [_I, C.POINTER(_I)]),
    "qwfn_qsa_check_shape": (C.c_int, [_S]),
    "qwfn_qsa_page_bytes": (C.c_int, [_S, C.POINTER(_Z)]),
    "qwfn_qsa_pooled_bytes": (C.c_int, [_S, _I, _I, C.POINTER(_Z)]),
    "qwfn_qsa_max_selected": (C.c_int, [_S, _I, C.POINTER(_I)]),
    "qwfn_qsa_workspace_bytes": (C.c_int, [_S, _I, _I, C.POINTER(_Z)]),
    "qwfn_qsa_workspace_init": (C.c_int, [_P, _Z, _P]),
    "qwfn_qsa_read_status": (C.c_int, [_V, C.POINTER(_I), _P]),
    "qwfn_kv_append_q8_0": (C.c_int, [_S, _V, _P, _P, _I, _P, _P, _I, _P]),
    "qwfn_pool_update": (C.c_int, [_S, _V, _P, _P, _I, _P]),
    "qwfn_pool_rebuild": (C.c_int, [_S, _V, _I, _I, _P]),
    "qwfn_kv_row_bytes": (C.c_int, [_S, C.POINTER(_Z)]),
    "qwfn_kv_export_q8_0": (C.c_int, [_S, _V, _I, _I, _I, _P, _P, _P]),
    "qwfn_kv_import_q8_0": (C.c_int, [_S, _V, _I, _I, _I, _P, _P, _P]),
    "qwfn_indexer_topk": (C.c_int, [_S, _V, _P, _P, _I, _I, _P, _P, _I, _P, _Z, _P]),
    "qwfn_gather_dequant": (C.c_int, [_S, _V, _P, _I, _P, _P, _I, _P, _P, _P, _P]),
    "qwfn_sparse_decode_attn": (C.c_int, [_S, _V, _P, _P, _I, _I, _P, _P, _I, _P, _P, _Z, _P]),
    "qwfn_decode_append_select": (C.c_int, [_S, _V, _P, _P, _P, _I, _P, _I, _I, _P, _P, _I, _P, _Z, _P]),
    "qwfn_sparse_attn_decode": (C.c_int, [_S, _V, _P, _P, _P, _I, _P, _I, _I, _P, _P, _P, _P, _Z, _P]),
    "qwfn_sparse_attn_decode_chain": (C.c_int, [_S, _V, _P, _P, _P, _I, _P, _I, _I, _I, _P, _P, _P, _P, _Z, _P]),
    "qwfn_sparse_attn_decode_noalloc": (C.c_int, [_S, _V, _P, _P, _P, _I, _P, _I, _I, _P, _P, _P, _P]),
    "qwfn_qsa_prefill_workspace_bytes": (C.c_int, [_S, _I, _I, C.POINTER(_Z)]),
    "qwfn_sparse_attn_prefill": (C.c_int, [_S, _V, _P, _P, _P, _I, _I, _I, _I, _P, _P, _P, _I, _P, _Z, _P]),
    "qwfn_idx_cache_bytes": (C.c_int, [_S, _IS, _I, _I, C.POINTER(_Z), C.POINTER(_Z)]),
    "qwfn_idx_workspace_bytes": (C.c_int, [_S, _IS, _I, _I, C.POINTER(_Z)]),
    "qwfn_idx_append_pool": (C.c_int, [_S, _V, _IS, _IV, _P, _I, _P, _P, _I, _P]),
    "qwfn_idx_pool_rebuild": (C.c_int, [_S, _V, _IS, _IV, _I, _I, _P]),
    "qwfn_idx_select": (C.c_int, [_S, _V, _IS, _IV, _P, _P, _I, _I, _P, _P, _I, _P, _Z, _P]),
    "qwfn_idx_sparse_attn_decode": (C.c_int, [_S, _V, _IS, _IV, _P, _P, _P, _P, _P, _I, _P, _I, _I, _P, _P, _P, _I,
                                              _P, _Z, _P]),
    "qwfn_idx_sparse_attn_prefill": (C.c_int, [_S, _V, _IS, _IV, _P, _P, _P, _P, _P, _I, _I, _I, _I, _P, _P, _P,
                                               _I, _P, _Z, _P]),
}


def load(path: str = LIB_PATH) -> C.CDLL:
    """Load the library (once).  Raises if it has not been built."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(path):
        raise RuntimeError(
            f"{path} is missing: build it with `python -m qwfnfer_amd.build` "
            "(the QSA path has no CPU fallback)")
    # torch ships its own libamdhip64.so.7.  Loading torch first makes this
    # library's libamdhip64.so.7 dependency bind to that copy, so the process
    # has one HIP runtime and the streams and memory torch hands over are the
    # runtime's own.
    try:
        import torch  # noqa: F401
    except ImportError:
        pass
    lib = C.CDLL(path)
    for name, (res, args) in _SIGS.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _lib = lib
    return lib


def call(name: str, *args) -> None:
    """Call an int-returning entry point; raise QsaError on a negative code."""
    lib = load()
    rc = getattr(lib, name)(*args)
    if rc < 0:
        msg = lib.qwfn_qsa_last_error().decode(errors="replace")
        raise QsaError(rc, name, msg)
