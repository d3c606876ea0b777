#!/usr/bin/env python3
"""bench.py -- sparse q8_0 decode attention on one MI355X.

Workload: 12 sparse-attention layers (16 q heads, 2 KV
heads, head_dim 128), q8_0 K/V ~ N(0,1) with a log-uniform [0.1, 10] scale per
q8_0 block, 64-token pooled blocks, top-64 blocks + block 0 + the last 512
tokens, one decode token per step at contexts 4096, 65536 and 163840.

A step = one decode token through all 12 layers; each layer is one
qwfn_sparse_attn_decode call, the fused path of graph_builder::sparse_attn_decode:
append the token's K/V (q8_0), pool the block it completes, score the pooled
blocks, select, attend.  At one sequence that is three launches: the indexer
(append, pooling, scores), the attention (each workgroup selects from the
scores, then attends over its tiles) and the partials' merge.  --two-call steps
through qwfn_decode_append_select + qwfn_sparse_decode_attn instead (the last
indexer workgroup selects).  The decode position advances one token per step
(seq_len += 1 on the device at the start of every step, one small kernel), so
one step in 64 completes a block and pools it, as in a real decode; every
replica keeps its own position and its caches have room for DECODE_ROOM more
tokens past the context.
Inputs are resident in HBM before the timed region.  Each context keeps enough
replicas of its 12-layer stack (each with its own queries and new rows) that a
step's bytes -- the selected K/V and the pooled keys it reads -- come round
again only after 512 MiB of other replicas' bytes, so the 256 MB MALL does not
serve them; consecutive steps use consecutive replicas.

The roofline is the attention launch's: its algorithmic bytes (the selected
K/V) over its own average duration, which an eager pass over the same
replicas measures per launch with HIP events that hipExtLaunchKernel stamps
with the kernel's begin and end (qwfn_qsa_time_next_call).

Prints one JSON line: value = us per layer at the largest context.
"""
from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "sparse decode attn µs/layer @4K & 160K ctx (q8_0 KV); % of HBM roofline"
HBM_PEAK_GBS = 8000.0          # MI355X published HBM3E peak
TRAFFIC_JSON = os.path.join(ROOT, "profiles", "traffic.json")   # rocprofv3 PMC summary (FETCH/WRITE_SIZE)
ROTATE_BYTES = 512 << 20
DECODE_ROOM = 2048             # tokens a replica may decode past its context


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=300)
    ap.add_argument("--warmup", type=int, default=30)
    ap.add_argument("--layers", type=int, default=12)
    ap.add_argument("--contexts", default="4096,65536,163840")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-graph", action="store_true", help="time eager launches only")
    ap.add_argument("--two-call", action="store_true",
                    help="step each layer through qwfn_decode_append_select + qwfn_sparse_decode_attn "
                         "instead of one qwfn_sparse_attn_decode")
    ap.add_argument("--no-batched", action="store_true", help="skip the config-5 batched line")
    ap.add_argument("--no-extra", action="store_true",
                    help="skip the config-1 (dense, ctx 4096) and config-2 (sparse, ctx 32768) lines")
    ap.add_argument("--no-prefill", action="store_true", help="skip the config-4 prefill-chunk line")
    ap.add_argument("--no-kv-types", action="store_true",
                    help="skip the q4_0 / fp16 cache lines (config 3 at the longest context)")
    ap.add_argument("--no-interop", action="store_true",
                    help="skip the reference-format import / export line (one layer at the longest context)")
    ap.add_argument("--no-checkpoint", action="store_true",
                    help="skip the checkpoint-layer decode line (the released model's own indexer)")
    ap.add_argument("--prefill-batch", type=int, default=8192,
                    help="queries per batch of the prefill chunk (sizes its workspace; 8192 = the whole "
                         "chunk in one batch, ~170 MB)")
    ap.add_argument("--seed", type=int, default=3)
    ap.add_argument("--copy-calib", type=int, default=0, metavar="BYTES",
                    help="first copy BYTES device-to-device 3 times (a plain copy kernel of known size, "
                         "the scale for rocprofv3 FETCH_SIZE / WRITE_SIZE counters)")
    return ap.parse_args()


# ---------------------------------------------------------------------------

def fill_layer(qsa, torch, cache, lengths, gen, chunk=32768, pool=True):
    """K/V ~ N(0,1) times a per-q8_0-block log-uniform [0.1, 10] scale, appended
    for tokens [0, L_s) of each sequence, then (pool) every whole block pooled."""
    cfg = cache.cfg
    nb = cfg.head_dim // 32
    for s, L in enumerate(lengths):
        for t0 in range(0, L, chunk):
            n = min(chunk, L - t0)
            kv = []
            for _ in range(2):
                x = torch.randn((n, cfg.n_head_kv, nb, 32), device="cuda", generator=gen)
                sc = torch.exp(torch.empty((n, cfg.n_head_kv, nb, 1), device="cuda").uniform_(
                    math.log(0.1), math.log(10.0), generator=gen))
                kv.append((x * sc).reshape(n, cfg.n_head_kv, cfg.head_dim).contiguous())
            pos = torch.arange(t0, t0 + n, dtype=torch.int32, device="cuda")
            sid = torch.full((n,), s, dtype=torch.int32, device="cuda")
            qsa.append_q8_0(cache, kv[0], kv[1], pos, sid)
        if pool and L // cfg.block_tokens:
            qsa.pool_rebuild(cache, s, L // cfg.block_tokens)


def selected_cells(sel, nsel, lengths, bt):
    """Cells attended per (sequence, KV head), from a selection read back."""
    tot = 0
    for s, L in enumerate(lengths):
        for g in range(sel.shape[1]):
            for b in sel[s, g, : nsel[s, g]]:
                tot += max(0, min(bt, L - int(b) * bt))
    return tot


def kv_row_bytes(cfg):
    """Bytes of one token's K (or V) head row: q8_0 136, q4_0 72, fp16 256 at head_dim 128."""
    return {0: cfg.head_dim + cfg.head_dim // 16, 1: cfg.head_dim // 2 + cfg.head_dim // 16,
            2: 2 * cfg.head_dim}[cfg.kv_type]


def best_launch(graph_ms, eager_ms):
    """The faster of the two ways a caller runs the step: one hipGraph replay
    a step, or the calls made one by one on the stream (the fused path's from
    prepared C arguments, Runner.prepare_direct).  Both time the same K steps
    of the same work; each graph replay also pays the runtime's fixed cost of a
    graph launch, about 7 us a step here."""
    if graph_ms is not None and graph_ms <= eager_ms:
        return graph_ms, "hipGraph (one replay a step)"
    return eager_ms, "eager (one call a layer, each kernel launched on the stream)"


def dominant_kernel(cfg, max_len, two_call):
    """rocprofv3's name of the attention launch a decode layer makes at
    sequences up to max_len tokens (the selecting variant in the fused call:
    its keys-per-thread tier covers max_len / block_tokens blocks)."""
    if two_call:
        return f"k_dec<{cfg.head_dim}, {cfg.n_head // cfg.n_head_kv}, 0, 4>"
    span = max_len // cfg.block_tokens - (cfg.sink_blocks & ~3)
    kpt = next(k for k in (4, 8, 16, 32) if span <= k * 256)
    return f"k_dec<{cfg.head_dim}, {cfg.n_head // cfg.n_head_kv}, 2, {kpt}>"


def touched_bytes_per_layer(cfg, lengths):
    """HBM bytes one decode layer touches at most: every sequence's selected
    K/V (the forced and top-k blocks whole, K and V) and its pooled keys."""
    if cfg.top_k_blocks == 0:
        keep = None
    else:
        keep = (cfg.top_k_blocks + cfg.sink_blocks + cfg.local_tokens // cfg.block_tokens + 2) * cfg.block_tokens
    tot = 0
    for L in lengths:
        tot += (L if keep is None else min(L, keep)) * cfg.n_head_kv * kv_row_bytes(cfg) * 2
        tot += (L // cfg.block_tokens) * cfg.n_head_kv * cfg.head_dim * 4
    return tot


class Runner:
    """n_inst replicas of an n_layer stack of caches at fixed sequence lengths,
    stepped one decode token at a time.  Consecutive steps use consecutive
    replicas, and there are enough of them that a step's bytes are touched
    again only after ROTATE_BYTES of other replicas' bytes, more than the
    256 MB MALL holds.  Every replica has its own queries and new K/V rows, so
    its selections differ from its neighbours'."""

    def __init__(self, qsa, torch, cfg, lengths, n_layer, pages_per_seq, page_table, gen, fused=False):
        self.qsa, self.torch, self.cfg = qsa, torch, cfg
        self.fused = fused
        self.lengths = lengths
        n_seq = len(lengths)
        self.n_seq = n_seq
        self.max_len = max(lengths) + DECODE_ROOM
        assert pages_per_seq * cfg.page_tokens >= self.max_len, "page table leaves no decode room"
        self.touched_per_step = n_layer * touched_bytes_per_layer(cfg, lengths)
        self.n_inst = max(1, math.ceil(ROTATE_BYTES / self.touched_per_step))
        self.stacks = []
        for _ in range(self.n_inst):
            layers = []
            for _ in range(n_layer):
                c = qsa.KvCache.allocate(cfg, n_seq, pages_per_seq, page_table=page_table,
                                         n_phys_pages=int(page_table.max()) + 1)
                fill_layer(qsa, torch, c, lengths, gen)
                layers.append(c)
            self.stacks.append(layers)
        r = lambda *shape: torch.randn(shape, device="cuda", generator=gen)
        self.q = [[r(n_seq, cfg.n_head, cfg.head_dim) for _ in range(n_layer)] for _ in range(self.n_inst)]
        self.kn = [[r(n_seq, cfg.n_head_kv, cfg.head_dim) for _ in range(n_layer)] for _ in range(self.n_inst)]
        self.vn = [[r(n_seq, cfg.n_head_kv, cfg.head_dim) for _ in range(n_layer)] for _ in range(self.n_inst)]
        self.out = [torch.empty((n_seq, cfg.n_head, cfg.head_dim), device="cuda") for _ in range(n_layer)]
        # one position per replica, advanced by one token at the start of every step
        self.seq_lens = [torch.tensor(lengths, dtype=torch.int32, device="cuda") for _ in range(self.n_inst)]
        self.ws = qsa.Workspace(cfg, n_seq, self.max_len)
        msel = cfg.max_selected(self.max_len)
        self.sel = torch.empty((n_seq, cfg.n_head_kv, msel), dtype=torch.int32, device="cuda")
        self.nsel = torch.empty((n_seq, cfg.n_head_kv), dtype=torch.int32, device="cuda")
        self.n_layer = n_layer
        self.graphs = None
        torch.cuda.synchronize()
        for layers in self.stacks:
            for c in layers:
                if qsa.read_status(c):
                    raise RuntimeError("cache fill reported out-of-range rows")

    def layer(self, inst, il, timers=None):
        """One layer's decode call(s).  timers: {kernel: (start, end)} events
        armed on the call(s) (qwfn_qsa_time_next_call)."""
        qsa = self.qsa
        c = self.stacks[inst][il]
        sl = self.seq_lens[inst]
        q, kn, vn = self.q[inst][il], self.kn[inst][il], self.vn[inst][il]
        if self.fused:                                  # qwfn_sparse_attn_decode: one call
            if timers:
                qsa.time_next_call(timers)
            qsa.sparse_attn_decode(c, q, kn, vn, sl, self.max_len, self.ws, out=self.out[il], sel=self.sel,
                                   n_sel=self.nsel)
            return
        if timers:
            qsa.time_next_call({"indexer": timers["indexer"]})
        qsa.decode_append_select(c, q, kn, vn, sl, self.max_len, self.ws, self.sel, self.nsel)
        if timers:
            qsa.time_next_call({k: timers[k] for k in ("attention", "merge")})
        qsa.sparse_decode_attn(c, q, sl, self.max_len, self.ws, self.sel, self.nsel, out=self.out[il])

    def advance(self, inst):
        """Next decode position of replica inst (one small device op, part of the step)."""
        self.seq_lens[inst].add_(1)

    def step(self, i):
        inst = i % self.n_inst
        self.advance(inst)
        for il in range(self.n_layer):
            self.layer(inst, il)

    def check_room(self):
        """Every replica's position is still inside its caches."""
        for sl in self.seq_lens:
            if int(sl.max().item()) > self.max_len:
                raise RuntimeError("decode ran past DECODE_ROOM; raise it or take fewer steps")

    def capture(self):
        """One hipGraph per replica holding a whole step (3 launches per layer).
        Every replay is checked against an eager step on the same inputs."""
        torch = self.torch
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        graphs = []
        with torch.cuda.stream(s):
            for inst in range(self.n_inst):
                g = torch.cuda.CUDAGraph()
                with torch.cuda.graph(g, stream=s):
                    self.advance(inst)
                    for il in range(self.n_layer):
                        self.layer(inst, il)
                graphs.append(g)
        torch.cuda.current_stream().wait_stream(s)
        torch.cuda.synchronize()
        for inst in range(self.n_inst):
            p0 = self.seq_lens[inst].clone()
            self.step(inst)
            torch.cuda.synchronize()
            ref = [o.clone() for o in self.out]
            for rep in range(3 if inst == 0 else 1):
                for o in self.out:
                    o.fill_(float("nan"))
                self.seq_lens[inst].copy_(p0)
                graphs[inst].replay()
                torch.cuda.synchronize()
                if not all(torch.equal(a, b) for a, b in zip(self.out, ref)):
                    raise RuntimeError(f"graph {inst} replay {rep} differs from the eager step")
                self.step(inst)                 # eager work between replays
                torch.cuda.synchronize()
        self.graphs = graphs

    def graph_step(self, i):
        self.graphs[i % self.n_inst].replay()

    def prepare_direct(self):
        """Every (replica, layer) call of the fused path with its C arguments
        resolved once, after the wrapper's checks, for eager steps that call
        qwfn_sparse_attn_decode straight from them as a C++ engine does (the
        wrapper's per-call checks, structs and stream lookup cost the host about
        15 us a call, which would pace the stream).  One direct step is checked
        against a step through the wrapper from the same position."""
        import ctypes as C
        qsa, torch = self.qsa, self.torch
        lib = qsa._lib.load()
        st = torch.cuda.current_stream().cuda_stream
        shape = self.cfg.shape()
        keep, calls = [shape], []
        n_seq = self.seq_lens[0].numel()
        for inst in range(self.n_inst):
            row = []
            for il in range(self.n_layer):
                view = self.stacks[inst][il].view()
                keep.append(view)
                row.append((C.byref(shape), C.byref(view), self.q[inst][il].data_ptr(), self.kn[inst][il].data_ptr(),
                            self.vn[inst][il].data_ptr(), qsa._lib.SRC_F32, self.seq_lens[inst].data_ptr(), n_seq,
                            self.max_len, self.out[il].data_ptr(), self.sel.data_ptr(), self.nsel.data_ptr(),
                            self.ws.ptr(), self.ws.nbytes, st))
            calls.append(row)
        self.direct_keep, self.direct_calls, self.direct_fn = keep, calls, lib.qwfn_sparse_attn_decode
        p0 = self.seq_lens[0].clone()
        self.step(0)
        torch.cuda.synchronize()
        ref = [o.clone() for o in self.out]
        for o in self.out:
            o.fill_(float("nan"))
        self.seq_lens[0].copy_(p0)
        self.direct_step(0)
        torch.cuda.synchronize()
        if not all(torch.equal(a, b) for a, b in zip(self.out, ref)):
            raise RuntimeError("a direct step differs from the wrapper's step")

    def direct_step(self, i):
        inst = i % self.n_inst
        self.advance(inst)
        fn = self.direct_fn
        for args in self.direct_calls[inst]:
            if fn(*args) < 0:
                raise RuntimeError(self.qsa._lib.load().qwfn_qsa_last_error().decode(errors="replace"))

    def time_eager(self, steps, warmup):
        """Eager steps, the fused path's calls made from prepared arguments."""
        if not self.fused:
            return self.time_steps(steps, warmup, graph=False)
        self.prepare_direct()
        return self.time_steps(steps, warmup, graph=False, direct=True)

    def time_steps(self, steps, warmup, graph, direct=False):
        torch = self.torch
        fn = self.graph_step if graph else self.direct_step if direct else self.step
        for i in range(warmup):
            fn(i)
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for i in range(steps):
            fn(i)
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / steps            # ms per step

    def time_kernels(self, steps):
        """Each decode kernel's own duration in us, averaged over every layer of
        `steps` eager steps that rotate the replicas as the timed region does.
        Every call is armed with qwfn_qsa_time_next_call: its indexer,
        attention and merge launches go through hipExtLaunchKernel, which
        stamps a pair of HIP events with that kernel's begin and end on the
        stream it runs on (what rocprofv3's kernel trace reports)."""
        torch, qsa = self.torch, self.qsa
        names = qsa.TIMED_KERNELS
        ev = [{k: (torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for k in names}
              for _ in range(self.n_layer)]
        for row in ev:
            for a, b in row.values():
                a.record()
                b.record()
        torch.cuda.synchronize()
        tot = dict.fromkeys(names, 0.0)
        for i in range(steps):
            inst = i % self.n_inst
            self.advance(inst)
            for il in range(self.n_layer):
                self.layer(inst, il, timers=ev[il])
            torch.cuda.synchronize()
            for row in ev:
                for k, (a, b) in row.items():
                    tot[k] += a.elapsed_time(b)
        n = steps * self.n_layer
        return {k: v / n * 1e3 for k, v in tot.items()}, n

    def bytes_per_layer(self):
        """Algorithmic bytes of one layer, averaged over one fresh step of every
        replica (its last layer's selection): the selected K/V (q8_0 / q4_0 /
        fp16 rows of K and V) the attention reads, the pooled keys the indexer
        scans."""
        cfg = self.cfg
        cells = 0
        lengths = None
        for inst in range(self.n_inst):
            self.step(inst)
            self.torch.cuda.synchronize()
            lengths = [int(x) for x in self.seq_lens[inst].tolist()]
            cells += selected_cells(self.sel.cpu().numpy(), self.nsel.cpu().numpy(), lengths, cfg.block_tokens)
        cells = cells / self.n_inst
        kv = cells * kv_row_bytes(cfg) * 2
        pooled = 0
        for L in lengths:
            last = L - 1
            fw = max(0, last - cfg.local_tokens + 1) // cfg.block_tokens
            elig = max(0, min(L // cfg.block_tokens, fw) - cfg.sink_blocks)
            if elig > cfg.top_k_blocks:
                pooled += elig * cfg.n_head_kv * cfg.head_dim * 4
        return kv, pooled, cells


PREFILL_POS0, PREFILL_N = 155648, 8192      # config 4: a chunk ending at 163840


PREFILL_WARM = 3   # untimed chunks first: a long prefill runs chunks back to back, at the
                   # clock sustained load settles on (the first chunk of a series runs ~15 % slower)


def bench_prefill(qsa, torch, cfg, gen, q_batch, reps=5):
    """Config 4: fp16 K/V rows of 8192 tokens appended at 155648 into a cache
    holding [0, 155648), the 128 blocks they complete pooled, and 8192 queries
    attending causally over their own selections -- one qwfn_sparse_attn_prefill
    call, timed with HIP events over `reps` calls after PREFILL_WARM untimed
    ones (every call rewrites the same rows, an idempotent overwrite)."""
    import numpy as np
    end = PREFILL_POS0 + PREFILL_N
    pps = end // cfg.page_tokens
    pt = torch.arange(pps, dtype=torch.int32).view(1, pps)
    cache = qsa.KvCache.allocate(cfg, 1, pps, page_table=pt, n_phys_pages=pps)
    fill_layer(qsa, torch, cache, [PREFILL_POS0], gen)
    kn = torch.randn((PREFILL_N, cfg.n_head_kv, cfg.head_dim), device="cuda", generator=gen).half()
    vn = torch.randn((PREFILL_N, cfg.n_head_kv, cfg.head_dim), device="cuda", generator=gen).half()
    q = torch.randn((PREFILL_N, cfg.n_head, cfg.head_dim), device="cuda", generator=gen)
    ws = qsa.Workspace.for_prefill(cfg, end, q_batch)
    msel = cfg.max_selected(end)
    sel = torch.empty((PREFILL_N, cfg.n_head_kv, msel), dtype=torch.int32, device="cuda")
    nsel = torch.empty((PREFILL_N, cfg.n_head_kv), dtype=torch.int32, device="cuda")
    out = torch.empty((PREFILL_N, cfg.n_head, cfg.head_dim), device="cuda")
    run = lambda: qsa.sparse_attn_prefill(cache, q, 0, PREFILL_POS0, ws, kn, vn, out=out, sel=sel, n_sel=nsel)
    for _ in range(PREFILL_WARM):
        run()
    torch.cuda.synchronize()
    if qsa.read_status(cache):
        raise RuntimeError("prefill reported out-of-range rows")
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(reps):
        run()
    e1.record()
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / reps
    # algorithmic work: every query's selected cells (<= its position), QK and PV
    s_np, n_np = sel.cpu().numpy(), nsel.cpu().numpy()
    bt = cfg.block_tokens
    cells = 0
    for i in range(PREFILL_N):
        L = PREFILL_POS0 + i + 1
        for g in range(cfg.n_head_kv):
            b = s_np[i, g, :n_np[i, g]].astype(np.int64)
            cells += int(np.minimum(bt, L - b * bt).clip(min=0).sum())
    group = cfg.n_head // cfg.n_head_kv
    flops = cells * group * cfg.head_dim * 2 * 2
    del cache, ws, sel, nsel, out
    torch.cuda.empty_cache()
    return dict(queries=PREFILL_N, pos0=PREFILL_POS0, ms_per_chunk=ms, selected_cells=cells,
                attn_gflop=flops / 1e9, attn_tflops=flops / (ms * 1e-3) / 1e12,
                mfma_bf16_peak_tflops=2500.0, frac=flops / (ms * 1e-3) / 2.5e15,
                append_bytes=PREFILL_N * cfg.n_head_kv * cfg.head_dim * 2 * 2 +
                PREFILL_N * cfg.n_head_kv * (cfg.head_dim + cfg.head_dim // 32 * 2) * 2,
                q_batch=q_batch, warm_calls=PREFILL_WARM, timed_calls=reps,
                note="QK and PV on v_mfma_f32_16x16x32_f16 (int8 quants exact in fp16, fp32 operands as "
                "fp16 hi + lo pairs); block scores as bounded fp16 matrix-core products, exact scores only "
                "where the bound leaves the selection open (selections identical); frac is against the "
                "dense fp16/bf16 MFMA peak")


def bench_checkpoint_prefill(qsa, torch, gen, reps=5):
    """The checkpoint layer's prefill chunk at config 4's place: 8192 tokens
    (K/V rows and raw indexer keys) appended at 155648 into a cache and
    indexer cache holding [0, 155648), the blocks they touch pooled, and 8192
    queries selected by their own indexer queries and attending causally --
    one qwfn_idx_sparse_attn_prefill call with a workspace for the whole chunk,
    timed with HIP events over `reps` calls after PREFILL_WARM untimed ones (an
    idempotent overwrite)."""
    cfg, icfg = qsa.checkpoint_config(), qsa.IdxConfig()
    end = PREFILL_POS0 + PREFILL_N
    pps = (end + cfg.page_tokens - 1) // cfg.page_tokens
    pt = torch.arange(pps, dtype=torch.int32).view(1, pps)
    cache = qsa.KvCache.allocate(cfg, 1, pps, page_table=pt, n_phys_pages=pps)
    fill_layer(qsa, torch, cache, [PREFILL_POS0], gen, pool=False)
    ic = qsa.IdxCache.allocate(icfg, cache, torch.rand(icfg.idx_dim, device="cuda", generator=gen) + 0.5)
    for t0 in range(0, PREFILL_POS0, 32768):
        n = min(32768, PREFILL_POS0 - t0)
        kr = torch.randn((n, icfg.idx_dim), device="cuda", generator=gen)
        qsa.idx_append_pool(ic, kr, torch.arange(t0, t0 + n, dtype=torch.int32, device="cuda"))
    r = lambda *shape: torch.randn(shape, device="cuda", generator=gen)
    q, qi = r(PREFILL_N, cfg.n_head, cfg.head_dim), r(PREFILL_N, icfg.n_idx_head, icfg.idx_dim)
    kn, vn = r(PREFILL_N, cfg.n_head_kv, cfg.head_dim).half(), r(PREFILL_N, cfg.n_head_kv, cfg.head_dim).half()
    kr = r(PREFILL_N, icfg.idx_dim).half()
    ws = qsa.Workspace.for_prefill(cfg, end, PREFILL_N)
    out = torch.empty((PREFILL_N, cfg.n_head, cfg.head_dim), device="cuda")
    run = lambda: qsa.idx_sparse_attn_prefill(ic, q, qi, 0, PREFILL_POS0, ws, k_new=kn, v_new=vn, k_raw=kr, out=out)
    for _ in range(PREFILL_WARM):
        run()
    torch.cuda.synchronize()
    if qsa.read_status(cache):
        raise RuntimeError("checkpoint prefill reported out-of-range rows")
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(reps):
        run()
    e1.record()
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / reps
    del cache, ic, ws, out
    torch.cuda.empty_cache()
    return dict(queries=PREFILL_N, pos0=PREFILL_POS0, ms_per_chunk=round(ms, 3),
                us_per_query=round(ms * 1e3 / PREFILL_N, 3))


class CheckpointRunner:
    """The released checkpoint's attention layer (24 query heads, 2 KV heads of
    256, q8_0 KV, blocks of 4 tokens pooled by its own indexer of 4 heads x 128,
    513 kept blocks) stepped one decode token at a time through
    qwfn_idx_sparse_attn_decode.  Up to 8,192 candidate blocks, three launches
    a layer: the indexer (one extra workgroup appends the K/V rows and the raw
    indexer key, re-pools its block and scores it when complete), the attention
    (every workgroup selects from the indexer's row) and its merge.  Past 8,192
    blocks, also three: the indexer launch's first workgroups append and place a
    sampled cut of the row, its scoring workgroups keep the keys above the cut
    as candidates, the attention ranks the candidates itself, and the merge."""

    def __init__(self, qsa, torch, ctx, n_layer, gen):
        self.qsa, self.torch = qsa, torch
        cfg = self.cfg = qsa.checkpoint_config()
        icfg = qsa.IdxConfig()
        self.max_len = ctx + DECODE_ROOM
        pps = (self.max_len + cfg.page_tokens - 1) // cfg.page_tokens
        pt = torch.arange(pps, dtype=torch.int32).view(1, pps)
        self.layers = []
        for _ in range(n_layer):
            c = qsa.KvCache.allocate(cfg, 1, pps, page_table=pt, n_phys_pages=pps)
            fill_layer(qsa, torch, c, [ctx], gen, pool=False)
            ic = qsa.IdxCache.allocate(icfg, c, torch.rand(icfg.idx_dim, device="cuda", generator=gen) + 0.5)
            for t0 in range(0, ctx, 32768):
                n = min(32768, ctx - t0)
                kr = torch.randn((n, icfg.idx_dim), device="cuda", generator=gen)
                qsa.idx_append_pool(ic, kr, torch.arange(t0, t0 + n, dtype=torch.int32, device="cuda"))
            self.layers.append((c, ic))
        H, Hkv, hd = cfg.n_head, cfg.n_head_kv, cfg.head_dim
        r = lambda *s: torch.randn(s, device="cuda", generator=gen)
        self.q = [r(1, H, hd) for _ in range(n_layer)]
        self.qi = [r(1, icfg.n_idx_head, icfg.idx_dim) for _ in range(n_layer)]
        self.kn = [r(1, Hkv, hd) for _ in range(n_layer)]
        self.vn = [r(1, Hkv, hd) for _ in range(n_layer)]
        self.kr = [r(1, icfg.idx_dim) for _ in range(n_layer)]
        self.out = [torch.empty((1, H, hd), device="cuda") for _ in range(n_layer)]
        self.seq_len = torch.tensor([ctx], dtype=torch.int32, device="cuda")
        ic0 = self.layers[0][1]
        self.ws = qsa.Workspace(cfg, 1, self.max_len, nbytes=max(cfg.workspace_bytes(1, self.max_len),
                                                                 ic0.workspace_bytes(1, self.max_len)))
        msel = cfg.max_selected(self.max_len)
        self.sel = torch.empty((1, Hkv, msel), dtype=torch.int32, device="cuda")
        self.nsel = torch.empty((1, Hkv), dtype=torch.int32, device="cuda")
        self.n_layer = n_layer
        torch.cuda.synchronize()

    def layer(self, il):
        _, ic = self.layers[il]
        self.qsa.idx_sparse_attn_decode(ic, self.q[il], self.qi[il], self.kn[il], self.vn[il], self.kr[il],
                                        self.seq_len, self.max_len, self.ws, out=self.out[il], sel=self.sel,
                                        n_sel=self.nsel)

    def step(self):
        self.seq_len.add_(1)
        for il in range(self.n_layer):
            self.layer(il)

    def prepare_direct(self):
        """Each layer's qwfn_idx_sparse_attn_decode arguments resolved once
        (as Runner.prepare_direct), one direct step checked against a step
        through the wrapper from the same position."""
        import ctypes as C
        qsa, torch = self.qsa, self.torch
        st = torch.cuda.current_stream().cuda_stream
        shape, ishape = self.cfg.shape(), self.layers[0][1].icfg.shape()
        keep, calls = [shape, ishape], []
        for il in range(self.n_layer):
            c, ic = self.layers[il]
            view, iview = c.view(), ic.view()
            keep += [view, iview]
            calls.append((C.byref(shape), C.byref(view), C.byref(ishape), C.byref(iview), self.q[il].data_ptr(),
                          self.qi[il].data_ptr(), self.kn[il].data_ptr(), self.vn[il].data_ptr(),
                          self.kr[il].data_ptr(), qsa._lib.SRC_F32, self.seq_len.data_ptr(), self.seq_len.numel(),
                          self.max_len, self.out[il].data_ptr(), self.sel.data_ptr(), self.nsel.data_ptr(),
                          self.sel.shape[-1], self.ws.ptr(), self.ws.nbytes, st))
        self.direct_keep, self.direct_calls = keep, calls
        self.direct_fn = qsa._lib.load().qwfn_idx_sparse_attn_decode
        p0 = self.seq_len.clone()
        self.step()
        torch.cuda.synchronize()
        ref = [o.clone() for o in self.out]
        for o in self.out:
            o.fill_(float("nan"))
        self.seq_len.copy_(p0)
        self.direct_step()
        torch.cuda.synchronize()
        if not all(torch.equal(a, b) for a, b in zip(self.out, ref)):
            raise RuntimeError("a direct checkpoint step differs from the wrapper's step")

    def direct_step(self):
        self.seq_len.add_(1)
        fn = self.direct_fn
        for args in self.direct_calls:
            if fn(*args) < 0:
                raise RuntimeError(self.qsa._lib.load().qwfn_qsa_last_error().decode(errors="replace"))

    def run(self, steps, warmup):
        torch = self.torch
        self.prepare_direct()
        for _ in range(warmup):
            self.direct_step()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(steps):
            self.direct_step()
        e1.record()
        torch.cuda.synchronize()
        eager = e0.elapsed_time(e1) / steps
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        g = torch.cuda.CUDAGraph()
        with torch.cuda.stream(s):
            with torch.cuda.graph(g, stream=s):
                self.step()
        torch.cuda.current_stream().wait_stream(s)
        torch.cuda.synchronize()
        # the replay against an eager step from the same position
        p0 = self.seq_len.clone()
        self.seq_len.copy_(p0)
        self.step()
        torch.cuda.synchronize()
        ref = [o.clone() for o in self.out]
        self.seq_len.copy_(p0)
        g.replay()
        torch.cuda.synchronize()
        if not all(torch.equal(a, b) for a, b in zip(self.out, ref)):
            raise RuntimeError("checkpoint graph replay differs from the eager step")
        for _ in range(warmup):
            g.replay()
        torch.cuda.synchronize()
        e0.record()
        for _ in range(steps):
            g.replay()
        e1.record()
        torch.cuda.synchronize()
        graph = e0.elapsed_time(e1) / steps
        if int(self.seq_len.item()) > self.max_len:
            raise RuntimeError("checkpoint decode ran past DECODE_ROOM")
        n = int(self.nsel[0, 0].item())
        L = int(self.seq_len.item())
        blocks = self.sel[0, 0, :n].cpu().tolist()
        cells = sum(max(0, min(4, L - 4 * b)) for b in blocks)
        row = self.cfg.head_dim + self.cfg.head_dim // 32 * 2
        ms, mode = best_launch(graph, eager)
        return dict(us_per_layer=ms * 1e3 / self.n_layer, launch=mode, eager_us_per_layer=eager * 1e3 / self.n_layer,
                    graph_us_per_layer=graph * 1e3 / self.n_layer, blocks_kept=n, cells_per_kv_head=cells,
                    selected_kv_bytes=cells * row * 2 * self.cfg.n_head_kv)


def round_f16_delta(qsa, torch, r):
    """Largest |o(kv_round_f16) - o(exact dequant)| over one decode call of
    every layer of replica 0: the same cache, queries and new rows (the
    append rewrites the same row), attended once in each mode.  The size of
    the reference's F16 cast of its gathered K/V (src/qwfn_graph.cpp:530-537)
    next to exact fp32 attention."""
    import dataclasses
    worst = 0.0
    for il, c in enumerate(r.stacks[0]):
        outs = []
        for rf in (1, 0):
            cc = dataclasses.replace(c, cfg=dataclasses.replace(c.cfg, kv_round_f16=rf))
            outs.append(qsa.sparse_attn_decode(cc, r.q[0][il], r.kn[0][il], r.vn[0][il], r.seq_lens[0], r.max_len,
                                               r.ws))
        torch.cuda.synchronize()
        worst = max(worst, float((outs[0] - outs[1]).abs().max()))
    return worst


def bench_interop(qsa, torch, cfg, gen, ctx, reps=20):
    """The reference-format boundary on one layer of ctx tokens: K and V rows
    in ggml's block_q8_0 row format (the reference's cache tensors) imported
    into the pages (qwfn_kv_import_q8_0), the pooled keys rebuilt from them
    (qwfn_pool_rebuild), and exported back (qwfn_kv_export_q8_0).  Each is
    timed with HIP events around `reps` calls; the rows and pages are ~90 MB
    each way, so the MALL does not hold them."""
    pps = (ctx + cfg.page_tokens - 1) // cfg.page_tokens
    pt = torch.arange(pps, dtype=torch.int32).view(1, pps)
    cache = qsa.KvCache.allocate(cfg, 1, pps, page_table=pt, n_phys_pages=pps)
    fill_layer(qsa, torch, cache, [ctx], gen)
    k_rows, v_rows = qsa.export_rows_q8_0(cache, 0, 0, ctx)
    torch.cuda.synchronize()
    res = {}
    for name, fn in (("import", lambda: qsa.import_rows_q8_0(cache, 0, 0, k_rows, v_rows)),
                     ("pool_rebuild", lambda: qsa.pool_rebuild(cache, 0, ctx // cfg.block_tokens)),
                     ("export", lambda: qsa.export_rows_q8_0(cache, 0, 0, ctx))):
        fn()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(reps):
            fn()
        e1.record()
        torch.cuda.synchronize()
        res[name] = e0.elapsed_time(e1) / reps * 1e3
    if qsa.read_status(cache):
        raise RuntimeError("interop reported out-of-range rows")
    rows = ctx * cfg.row_bytes() * 2                 # K and V rows, read or written once each way
    out = dict(context=ctx, row_bytes=cfg.row_bytes(), kv_row_bytes_total=rows,
               import_us=round(res["import"], 2), export_us=round(res["export"], 2),
               pool_rebuild_us=round(res["pool_rebuild"], 2),
               import_gbs=round(2 * rows / (res["import"] * 1e-6) / 1e9, 1),
               export_gbs=round(2 * rows / (res["export"] * 1e-6) / 1e9, 1),
               note="import/export read the rows (or pages) once and write the pages (or rows) once: "
                    "2 x kv_row_bytes_total per call")
    del cache, k_rows, v_rows
    torch.cuda.empty_cache()
    return out


def cpu_baseline(cfg, ctx, seconds, seed):
    """The oracle's fp32 decode step (the ggml CPU path restated: append,
    pool, scores, selection, attention over fp16-cast K/V) on one layer at
    ctx, repeated for about `seconds`."""
    import numpy as np
    from oracle import oracle as O
    rng = np.random.default_rng(seed)
    pps = ctx // cfg.page_tokens
    host = O.HostCache(cfg, 1, pps)
    nb = cfg.head_dim // 32
    for t0 in range(0, ctx, 16384):
        n = min(16384, ctx - t0)
        kv = []
        for _ in range(2):
            x = rng.standard_normal((n, cfg.n_head_kv, nb, 32), dtype=np.float32)
            x *= np.exp(rng.uniform(np.log(0.1), np.log(10.0), (n, cfg.n_head_kv, nb, 1))).astype(np.float32)
            kv.append(x.reshape(n, cfg.n_head_kv, cfg.head_dim))
        host.append(kv[0], kv[1], np.arange(t0, t0 + n, dtype=np.int32))
    for b in range(ctx // cfg.block_tokens):
        host.pool_block(0, b)
    q = rng.standard_normal((1, cfg.n_head, cfg.head_dim), dtype=np.float32)
    kn = rng.standard_normal((1, cfg.n_head_kv, cfg.head_dim), dtype=np.float32)
    host.decode_step_f32(q, kn, kn, [ctx])                       # warm-up
    n, t0 = 0, time.perf_counter()
    threads = 1
    while time.perf_counter() - t0 < seconds:
        _, _, _, threads = host.decode_step_f32(q, kn, kn, [ctx])
        n += 1
    dt = time.perf_counter() - t0
    return dt / n * 1e6, threads, n


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (asked for --gpus {args.gpus}); the QSA path "
              "shards across GPUs only by sequence or KV head, which this build does not run.",
              file=sys.stderr)
        sys.exit(2)
    import torch
    from qwfnfer_amd import qsa

    assert torch.cuda.is_available(), "bench.py needs a GPU"
    cfg = qsa.QsaConfig()
    contexts = [int(c) for c in args.contexts.split(",")]
    gen = torch.Generator(device="cuda")
    gen.manual_seed(args.seed)
    dev = torch.cuda.get_device_name(0)
    log(f"[bench] {dev}; {args.layers} layers, contexts {contexts}, steps {args.steps}, warmup {args.warmup}")

    if args.copy_calib:
        n = args.copy_calib // 4
        a = torch.empty(n, dtype=torch.float32, device="cuda").fill_(1.0)
        b = torch.empty_like(a)
        torch.cuda.synchronize()
        for _ in range(3):
            b.copy_(a)
        torch.cuda.synchronize()
        log(f"[bench] copy calibration: 3 x {args.copy_calib} B device-to-device")
        del a, b

    per_ctx = {}
    for ctx in contexts:
        pps = (ctx + DECODE_ROOM + cfg.page_tokens - 1) // cfg.page_tokens
        pt = torch.arange(pps, dtype=torch.int32).view(1, pps)
        r = Runner(qsa, torch, cfg, [ctx], args.layers, pps, pt, gen, fused=not args.two_call)
        eager_ms = r.time_eager(args.steps, args.warmup)
        graph_ms = None
        if not args.no_graph:
            r.capture()
            graph_ms = r.time_steps(args.steps, args.warmup, graph=True)
        kern, n_timed = r.time_kernels(args.steps)
        r.check_room()
        kv, pooled, cells = r.bytes_per_layer()
        ms, mode = best_launch(graph_ms, eager_ms)
        res = dict(us_per_layer=ms * 1e3 / args.layers, launch=mode, eager_us_per_layer=eager_ms * 1e3 / args.layers,
                   graph_us_per_layer=None if graph_ms is None else graph_ms * 1e3 / args.layers,
                   ms_per_step=ms, kernel_us=kern, kernel_launches_timed=n_timed,
                   selected_kv_bytes=kv, pooled_scan_bytes=pooled, cells_per_layer=cells,
                   replicas=r.n_inst, touched_bytes_per_step=r.touched_per_step)
        res["attn_gbs"] = kv / (kern["attention"] * 1e-6) / 1e9
        res["layer_gbs_selected"] = kv / (res["us_per_layer"] * 1e-6) / 1e9
        res["layer_gbs_all"] = (kv + pooled) / (res["us_per_layer"] * 1e-6) / 1e9
        per_ctx[ctx] = res
        log(f"[bench] ctx {ctx}: {res['us_per_layer']:.2f} us/layer (eager {res['eager_us_per_layer']:.2f}); "
            f"kernels: indexer {kern['indexer']:.2f} us, attention {kern['attention']:.2f} us "
            f"= {res['attn_gbs']:.0f} GB/s on {kv:.0f} B, merge {kern['merge']:.2f} us; "
            f"pooled scan {pooled} B; {r.n_inst} replicas x {r.touched_per_step / 2**20:.1f} MiB touched a step")
        del r
        torch.cuda.synchronize()
        torch.cuda.empty_cache()

    # configs 1 and 2: the same decode step (one call a layer, 12 layers a step)
    extra = None
    if not args.no_extra:
        extra = {}
        for name, c, ctx in (("config1_dense", qsa.QsaConfig(top_k_blocks=0), 4096), ("config2", cfg, 32768)):
            pps = (ctx + DECODE_ROOM + c.page_tokens - 1) // c.page_tokens
            pt = torch.arange(pps, dtype=torch.int32).view(1, pps)
            r = Runner(qsa, torch, c, [ctx], args.layers, pps, pt, gen, fused=not args.two_call)
            eager_ms = r.time_eager(args.steps, args.warmup)
            graph_ms = None
            if not args.no_graph:
                r.capture()
                graph_ms = r.time_steps(args.steps, args.warmup, graph=True)
            r.check_room()
            kv, _, cells = r.bytes_per_layer()
            ms, mode = best_launch(graph_ms, eager_ms)
            us = ms * 1e3 / args.layers
            extra[name] = dict(context=ctx, us_per_layer=round(us, 3), launch=mode,
                               eager_us_per_layer=round(eager_ms * 1e3 / args.layers, 3),
                               cells_per_layer=cells, selected_kv_bytes=kv,
                               layer_gbs_selected=round(kv / (us * 1e-6) / 1e9, 1))
            log(f"[bench] {name} ctx {ctx}: {us:.2f} us/layer (eager {eager_ms * 1e3 / args.layers:.2f}), "
                f"{cells} cells, {kv} B of K/V")
            del r
            torch.cuda.synchronize()
            torch.cuda.empty_cache()

    batched = None
    if not args.no_batched:
        import numpy as np
        rng = np.random.default_rng(args.seed)
        lens = [int(math.exp(rng.uniform(math.log(4096), math.log(262144)))) for _ in range(8)]
        pps = (max(lens) + DECODE_ROOM + cfg.page_tokens - 1) // cfg.page_tokens
        perm = torch.from_numpy(rng.permutation(8 * pps).astype(np.int32)).view(8, pps)
        r = Runner(qsa, torch, cfg, lens, 1, pps, perm, gen, fused=not args.two_call)
        eager_ms = r.time_eager(args.steps, args.warmup)
        graph_ms = None
        if not args.no_graph:
            r.capture()
            graph_ms = r.time_steps(args.steps, args.warmup, graph=True)
        kern, n_timed = r.time_kernels(args.steps)
        r.check_room()
        kv, pooled, cells = r.bytes_per_layer()
        ms, mode = best_launch(graph_ms, eager_ms)
        batched = dict(lengths=lens, us_per_step=ms * 1e3, launch=mode, eager_us_per_step=eager_ms * 1e3,
                       graph_us_per_step=None if graph_ms is None else graph_ms * 1e3,
                       kernel_us=kern, kernel_launches_timed=n_timed, selected_kv_bytes=kv,
                       pooled_scan_bytes=pooled, replicas=r.n_inst, touched_bytes_per_step=r.touched_per_step,
                       attn_gbs=kv / (kern["attention"] * 1e-6) / 1e9,
                       attn_frac=kv / (kern["attention"] * 1e-6) / 1e9 / HBM_PEAK_GBS,
                       step_gbs=kv / (ms * 1e-3) / 1e9)
        log(f"[bench] config 5 batched (8 seqs {lens}): {ms * 1e3:.2f} us a step (eager {eager_ms * 1e3:.2f}); "
            f"indexer {kern['indexer']:.2f} us, attention {kern['attention']:.2f} us = {batched['attn_gbs']:.0f} "
            f"GB/s, merge {kern['merge']:.2f} us; {r.n_inst} replicas")
        del r
        torch.cuda.empty_cache()

    prefill = None
    if not args.no_prefill:
        prefill = bench_prefill(qsa, torch, cfg, gen, args.prefill_batch)
        log(f"[bench] config 4 prefill chunk (8192 queries at 155648): {prefill['ms_per_chunk']:.3f} ms, "
            f"{prefill['attn_tflops']:.1f} TFLOP/s on the selected-cell FLOPs")

    kv_types = None
    if not args.no_kv_types:
        import dataclasses
        kv_types = {}
        ctx = max(contexts)
        for kt, rf, name in ((1, 0, "q4_0"), (2, 0, "f16"), (0, 1, "q8_0_round_f16")):
            c2 = dataclasses.replace(cfg, kv_type=kt, kv_round_f16=rf)
            pps = (ctx + DECODE_ROOM + c2.page_tokens - 1) // c2.page_tokens
            pt = torch.arange(pps, dtype=torch.int32).view(1, pps)
            r = Runner(qsa, torch, c2, [ctx], args.layers, pps, pt, gen, fused=not args.two_call)
            r.capture()
            ms = r.time_steps(max(30, args.steps // 3), args.warmup, graph=True)
            kern, n_timed = r.time_kernels(max(30, args.steps // 3))
            r.check_room()
            kv, pooled, cells = r.bytes_per_layer()
            kv_types[name] = dict(context=ctx, us_per_layer=round(ms * 1e3 / args.layers, 3),
                                  kernel_us={k: round(v, 3) for k, v in kern.items()},
                                  cells_per_layer=cells, selected_kv_bytes=kv,
                                  attn_gbs=round(kv / (kern["attention"] * 1e-6) / 1e9, 1), replicas=r.n_inst)
            kv_types[name]["attention_kernel"] = (
                "k_dec (q8_0 on the matrix cores, K/V rounded to fp16 in registers)" if rf else
                f"k_dec ({name} rows in the K layout on the matrix cores, read a cell at a time)")
            if rf:
                kv_types[name]["max_abs_delta_vs_exact"] = round_f16_delta(qsa, torch, r)
            log(f"[bench] kv {name} ctx {ctx}: {ms * 1e3 / args.layers:.2f} us/layer, indexer "
                f"{kern['indexer']:.2f} us, attention {kern['attention']:.2f} us, merge {kern['merge']:.2f} us "
                f"({kv_types[name]['attention_kernel']})" +
                (f", max |delta| vs exact {kv_types[name]['max_abs_delta_vs_exact']:.3g}" if rf else ""))
            del r
            torch.cuda.empty_cache()

    interop = None
    if not args.no_interop:
        interop = bench_interop(qsa, torch, cfg, gen, max(contexts))
        log(f"[bench] interop at {interop['context']}: import {interop['import_us']:.1f} us "
            f"({interop['import_gbs']:.0f} GB/s), pool rebuild {interop['pool_rebuild_us']:.1f} us, "
            f"export {interop['export_us']:.1f} us ({interop['export_gbs']:.0f} GB/s)")

    checkpoint = None
    if not args.no_checkpoint:
        ck = {}
        for ctx in sorted({min(contexts), max(contexts)}):
            r = CheckpointRunner(qsa, torch, ctx, args.layers, gen)
            ck[str(ctx)] = {k: (round(v, 3) if isinstance(v, float) else v)
                            for k, v in r.run(max(20, args.steps // 3), args.warmup).items()}
            log(f"[bench] checkpoint layer ctx {ctx}: {ck[str(ctx)]['us_per_layer']:.2f} us/layer "
                f"(eager {ck[str(ctx)]['eager_us_per_layer']:.2f}), {ck[str(ctx)]['blocks_kept']} blocks kept")
            del r
            torch.cuda.empty_cache()
        checkpoint = dict(per_context=ck, workload="the released checkpoint's attention layer: 24q/2kv heads "
                          "x 256, q8_0 KV, 4-token blocks, own indexer (4 heads x 128, RMSNorm + rotary pooled "
                          "keys), 513 kept blocks shared by both KV heads; qwfn_idx_sparse_attn_decode a layer (3 launches: "
                          "indexer with the append, attention, merge; past 8,192 blocks the indexer launch also "
                          "places a sampled cut and keeps each chunk's candidates above it); the faster of a hipGraph replay "
                          "and eager calls from prepared arguments")
        if not args.no_prefill:
            checkpoint["prefill"] = bench_checkpoint_prefill(qsa, torch, gen)
            log(f"[bench] checkpoint prefill chunk ({PREFILL_N} queries at {PREFILL_POS0}): "
                f"{checkpoint['prefill']['ms_per_chunk']:.3f} ms")

    big = max(contexts)
    small = min(contexts)
    top = per_ctx[big]
    cpu = None
    if not args.no_cpu:
        cpu_us, threads, n = cpu_baseline(cfg, big, args.cpu_seconds, args.seed)
        cpu = {"value": round(cpu_us, 2), "unit": "us/layer", "cores": threads, "kind": "port",
               "sample": f"{n} decode steps of one layer at ctx {big} (oracle/qsa_oracle.c "
                         f"qwfn_oracle_decode_step_f32, OpenMP), ~{args.cpu_seconds:.0f} s; the same step "
                         f"repeated on one cache, so the host's caches are warm (a throughput figure)"}
        log(f"[bench] cpu baseline: {cpu_us:.1f} us/layer on {threads} threads ({n} steps)")
        c1_s = max(2.0, args.cpu_seconds / 2)
        c1_us, c1_threads, c1_n = cpu_baseline(qsa.QsaConfig(top_k_blocks=0), 4096, c1_s, args.seed)
        cpu["config1_dense_4096"] = {
            "value": round(c1_us, 2), "unit": "us/layer", "cores": c1_threads, "kind": "port",
            "sample": f"{c1_n} dense decode steps of one layer at ctx 4096 (BASELINE config 1, the reference's "
                      f"CPU ggml-path case), ~{c1_s:.0f} s, warm caches"}
        log(f"[bench] cpu baseline config 1 (dense 4096): {c1_us:.1f} us/layer on {c1_threads} threads ({c1_n} steps)")

    flat_mode = {"eager": top["eager_us_per_layer"] / per_ctx[small]["eager_us_per_layer"]}
    if top["graph_us_per_layer"] is not None and per_ctx[small]["graph_us_per_layer"] is not None:
        flat_mode["hipGraph"] = top["graph_us_per_layer"] / per_ctx[small]["graph_us_per_layer"]
    # the launch mode `value` was taken in (both legs timed the same way)
    flat_key = "hipGraph" if "hipGraph" in flat_mode and top["launch"].startswith("hipGraph") else "eager"
    attn_gbs = top["attn_gbs"]
    dom = dominant_kernel(cfg, big + DECODE_ROOM, args.two_call)
    traffic = None
    if os.path.exists(TRAFFIC_JSON):
        with open(TRAFFIC_JSON) as f:
            tj = json.load(f).get(dom, {})
        if tj.get("context") == big:
            traffic = tj.get("hbm_bytes_per_launch")
    line = {
        "metric": METRIC,
        "value": round(top["us_per_layer"], 3),
        "unit": "us/layer",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(top["ms_per_step"], 4),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic",
        "config": {
            "workload": f"config3: {args.layers} sparse layers, ctx {big}, 16q/2kv heads x 128, q8_0 KV, "
                        f"top-64 64-token blocks + block 0 + 512-token window, 1 decode token/step",
            "contexts": contexts,
            "launch": top["launch"],
            "decode_call": "qwfn_decode_append_select + qwfn_sparse_decode_attn" if args.two_call
                           else "qwfn_sparse_attn_decode (fused: the attention selects)",
        },
        "us_per_layer": {str(c): round(v["us_per_layer"], 3) for c, v in per_ctx.items()},
        # the 160K layer over the 4K layer, both legs in one launch mode
        "flatness": round(flat_mode[flat_key], 4),
        "flatness_launch": flat_key,
        "flatness_by_launch": {k: round(v, 4) for k, v in flat_mode.items()},
        "per_context": {str(c): {k: (round(x, 3) if isinstance(x, float) else x) for k, x in v.items()}
                        for c, v in per_ctx.items()},
        "roofline": {
            "bound": "hbm",
            "kernel": dom,
            "kernel_role": "the timed step's attention launch: selects its (KV head's) blocks from the indexer's "
                           "scores, then attends over the selected q8_0 K/V on the matrix cores, one partial "
                           "per workgroup (k_merge combines them)" if not args.two_call else
                           "the two-call step's attention launch over a given selection",
            "achieved": round(attn_gbs, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(attn_gbs / HBM_PEAK_GBS, 4),
            "traffic": traffic,
            "bytes_per_launch": round(top["selected_kv_bytes"]),
            "bytes": "algorithmic: the selected cells' q8_0 K and V rows (136 B each per KV head)",
            "launch_us": round(top["kernel_us"]["attention"], 3),
            "launches_timed": top["kernel_launches_timed"],
            "timing": "each launch's own begin/end: HIP events stamped by hipExtLaunchKernel on its stream "
                      "(qwfn_qsa_time_next_call), over eager steps rotating the replicas like the timed region",
        },
        "layer_roofline_frac": round(top["layer_gbs_selected"] / HBM_PEAK_GBS, 4),
        "configs_1_2": extra,
        "batched_config5": batched,
        "prefill_config4": prefill,
        "checkpoint_decode": checkpoint,
        "kv_types": kv_types,
        "interop": interop,
        "cpu_baseline": cpu,
        "device": torch.cuda.get_device_name(0),
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
