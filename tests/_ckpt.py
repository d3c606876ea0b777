"""Helpers of the checkpoint-indexer tests: the indexer's configuration and
the oracle's selection over the indexer's pooled keys."""
from __future__ import annotations

from dataclasses import dataclass

import numpy as np

from oracle import oracle as O
from _refs import Cfg


@dataclass(frozen=True)
class ICfg:
    """Field names match qwfnfer_amd.qsa.IdxConfig."""
    idx_dim: int = 128
    n_idx_head: int = 4
    rope_dim: int = 64
    rope_freq_base: float = 10000000.0
    rms_eps: float = 1e-6


# the checkpoint's attention layer (qwfnfer_amd.qsa.checkpoint_config()) with
# a shorter top-k for small contexts
CKPT = Cfg(n_head=24, n_head_kv=2, head_dim=256, block_tokens=4, page_tokens=256, top_k_blocks=513,
           sink_blocks=0, local_tokens=0, relu_per_head=1, shared_selection=1, topk_counts_forced=1)


def scoring_cfg(cfg, icfg) -> Cfg:
    """The indexer's scoring geometry: one group of n_idx_head heads over the
    indexer's pooled keys, the attention layer's selection rule."""
    return Cfg(n_head=icfg.n_idx_head, n_head_kv=1, head_dim=icfg.idx_dim, block_tokens=cfg.block_tokens,
               page_tokens=cfg.page_tokens, top_k_blocks=cfg.top_k_blocks, sink_blocks=cfg.sink_blocks,
               local_tokens=cfg.local_tokens, relu_per_head=cfg.relu_per_head, shared_selection=1,
               quant_variant=cfg.quant_variant, topk_counts_forced=cfg.topk_counts_forced)


def oracle_select(cfg, icfg, pooled: np.ndarray, q_idx: np.ndarray, seq_len: int, max_sel: int) -> np.ndarray:
    """The oracle's selection of one decode token from pooled [bps][idx_dim]
    and q_idx [n_idx_head][idx_dim]."""
    sc = scoring_cfg(cfg, icfg)
    bps = pooled.shape[0]
    pages = bps * cfg.block_tokens // cfg.page_tokens
    host = O.HostCache(sc, 1, pages)
    host.pooled[0, 0] = pooled
    sel, nsel = host.indexer_topk(q_idx[None], [seq_len], max_sel=max_sel)
    return sel[0, 0, :nsel[0, 0]].copy()


def oracle_pool_all(cfg, icfg, raw_rows: np.ndarray, k_norm: np.ndarray, n_blocks: int) -> np.ndarray:
    """Pooled keys of blocks [0, n_blocks) from raw fp16 rows [n_tokens][idx_dim]
    (rows past n_tokens read as 0, as an unwritten zeroed cache)."""
    bt = cfg.block_tokens
    need = n_blocks * bt
    rows = np.zeros((max(need, raw_rows.shape[0]), icfg.idx_dim), np.float16)
    rows[:raw_rows.shape[0]] = raw_rows
    return np.stack([O.idx_pool_block(cfg, icfg, rows[b * bt:(b + 1) * bt], k_norm, b) for b in range(n_blocks)])
