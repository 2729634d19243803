#!/usr/bin/env python
"""Benchmark of the index-resident multi-adapter LoRA delta on one MI355X.

Default workload (one "step" = one sweep of all 342 FLUX.1-dev target linears at
1024^2): B = 14 samples x 4,608 tokens (4,096 image + 512 text), bf16, rank 16,
every sample routed to a distinct adapter of a 10,000-adapter bank held as
bit-packed 9-bit indices (24.0 GB resident). Each module adds its delta into a
precomputed base output: y += (x A_j^T) B_j^T with A_j, B_j decoded on the fly
inside the kernels. Inputs are synthetic (x, y ~ N(0, 1); uniformly random
9-bit fields) and already resident in HBM; x / y buffers rotate so the 256 MB
Infinity Cache cannot serve a module from a previous module's data. The
independent linears of each block stage (the image and text projections, the two
attention outputs, the two up and the two down projections, a single block's
q / k / v) run as one grouped call: one shrink and one expand launch per stage,
114 calls per sweep (``--config flux342``: one call per module).

    python bench.py [--steps K] [--warmup W] [--config grouped|flux342|fused|qkv|decoded|decoded_grouped|ffn|hb|hb_modules|decode|ingest|encode] [--rank R]

Prints ONE JSON line. ``value`` = tokens per second of the whole sweep;
``roofline`` covers the per-module delta call (shrink + expand kernels) against
the HBM roofline with the algorithmic bytes 2 d_in + 4 d_out per token (x read,
y read + write) plus the packed index words of the routed adapters;
``cpu_baseline`` times the reference's serving forward restated in torch CPU ops
(bf16 bmm, fp32 decode of the routed adapters) over one module per class on the
host cores; ``env`` records ROCm, torch, the GPU and the host CPU.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

HBM_PEAK_GBPS = 8000.0
RANK = 16


def flux_modules(img_tokens: int, txt_tokens: int):
    """(name, d_in, d_out, tokens per sample) of the 342 FLUX.1-dev target linears, model order."""
    mods = []
    for i in range(19):
        p = f"transformer_blocks.{i}."
        for n in ("attn.to_q", "attn.to_k", "attn.to_v", "attn.to_out.0"):
            mods.append((p + n, 3072, 3072, img_tokens))
        for n in ("attn.add_q_proj", "attn.add_k_proj", "attn.add_v_proj", "attn.to_add_out"):
            mods.append((p + n, 3072, 3072, txt_tokens))
        mods += [(p + "ff.net.0.proj", 3072, 12288, img_tokens), (p + "ff.net.2", 12288, 3072, img_tokens),
                 (p + "ff_context.net.0.proj", 3072, 12288, txt_tokens),
                 (p + "ff_context.net.2", 12288, 3072, txt_tokens)]
    for i in range(38):
        p = f"single_transformer_blocks.{i}."
        for n in ("attn.to_q", "attn.to_k", "attn.to_v"):
            mods.append((p + n, 3072, 3072, img_tokens + txt_tokens))
    return mods


# Stage of a FLUX target linear inside its block: the linears of one stage of a block are independent
# of each other (the image and text projections, the two attention outputs, the two up and the two down
# projections), so a serving step can issue them as one grouped call.
_STAGES = {"attn.to_q": "proj", "attn.to_k": "proj", "attn.to_v": "proj", "attn.add_q_proj": "proj",
           "attn.add_k_proj": "proj", "attn.add_v_proj": "proj", "attn.to_out.0": "out", "attn.to_add_out": "out",
           "ff.net.0.proj": "up", "ff_context.net.0.proj": "up", "ff.net.2": "down", "ff_context.net.2": "down"}
# linears that read one input: the q / k / v projections of one attention input
_SHARED_INPUT = {"attn.to_q": "img", "attn.to_k": "img", "attn.to_v": "img", "attn.add_q_proj": "txt",
                 "attn.add_k_proj": "txt", "attn.add_v_proj": "txt"}


def _split(name):
    """(block prefix, linear suffix) of a FLUX module path."""
    for suffix in _STAGES:
        if name.endswith(suffix):
            return name[: -len(suffix)], suffix
    raise ValueError(name)


def flux_groups(mods):
    """Indices of ``mods`` grouped by (block, stage), in order of first appearance."""
    groups = {}
    for i, (n, _, _, _) in enumerate(mods):
        prefix, suffix = _split(n)
        groups.setdefault((prefix, _STAGES[suffix]), []).append(i)
    return list(groups.values())


class Workload:
    """Bank, buffers and prepared per-module calls of one configuration."""

    def __init__(self, name, mods, batch, n_slots, assign, layout_mods=None, seed=0, decoded=False, qkv=False,
                 grouped=False, rank=RANK):
        import numpy as np
        import torch

        from lithe_amd.kernels import PackedBank, PackedLayout
        from lithe_amd.kernels.prepared import (group_workspace_bytes, prepare_dense, prepare_packed,
                                                prepare_packed_group, prepare_packed_shared_x, prepare_stacked_group,
                                                shared_workspace, shared_x_workspace_bytes, workspace_bytes)

        self.name, self.mods, self.batch = name, mods, batch
        dev = torch.device("cuda:0")
        layout_mods = layout_mods or mods
        layout = PackedLayout.from_modules(
            [{"name": n, "shape_a": [rank, di], "shape_b": [do, rank]} for n, di, do, _ in layout_mods],
            num_levels=3, block_size=64, scaling=1.0)
        self.bank = PackedBank(layout, dev, capacity=n_slots)
        self.bank.fill_random(n_slots, generator=torch.Generator(device=dev).manual_seed(seed))
        self.assign = torch.tensor(assign, dtype=torch.int32, device=dev)
        pools = (self.bank.pool_a.to(torch.bfloat16), self.bank.pool_b.to(torch.bfloat16))

        # rotating buffers per (feature dim, tokens) class; copies so that the reuse
        # distance of every buffer exceeds the 256 MB last-level cache
        gen = torch.Generator(device=dev).manual_seed(seed + 1)
        self._bufs, self._next = {}, {}

        def buf(d, m, avoid=()):
            """The next buffer of the (d, m) rotation that is none of ``avoid`` (the buffers of the
            other modules of the same call); a new copy joins the rotation if all are taken."""
            key = (d, m)
            if key not in self._bufs:
                nbytes = batch * m * d * 2
                copies = 2 if nbytes >= (512 << 20) else 4
                self._bufs[key] = [torch.randn(batch, m, d, device=dev, generator=gen).to(torch.bfloat16)
                                   for _ in range(copies)]
                self._next[key] = 0
            pool = self._bufs[key]
            for _ in range(len(pool)):
                i = self._next[key]
                self._next[key] = (i + 1) % len(pool)
                if all(pool[i] is not t for t in avoid):
                    return pool[i]
            pool.append(torch.randn(batch, m, d, device=dev, generator=gen).to(torch.bfloat16))
            return pool[-1]

        # per-call workspace (grouped workloads size theirs per group below; a q / k / v call of the
        # per-call path holds the three modules' intermediates)
        need = 0 if grouped else max(workspace_bytes((batch, m, di), do, rank, 1, torch.bfloat16)
                                     for _, di, do, m in mods)
        if qkv and not grouped:
            need = max([need] + [shared_x_workspace_bytes((batch, m, di), [do] * 3, rank, 1, torch.bfloat16)
                                 for _, di, do, m in mods])
        groups = flux_groups(mods) if grouped else []
        for gi in groups:
            keys = [_SHARED_INPUT.get(_split(mods[i][0])[1], str(i)) if qkv else str(i) for i in gi]
            ids = {k: j for j, k in enumerate(dict.fromkeys(keys))}
            need = max(need, group_workspace_bytes([(mods[i][3], mods[i][1], mods[i][2]) for i in gi],
                                                   [ids[k] for k in keys], batch, rank, 1, torch.bfloat16))
        self.workspace = shared_workspace(dev, need)
        self.calls = []
        self.call_mods = []
        uniq = sorted(set(np.asarray(assign).tolist()))
        self.decode_ms = None
        if decoded:
            # decoded-mode serving: the routed slots decoded once (decode-on-swap) into stacked
            # per-module bf16 factors, then every module reads dense factors
            sel_of = {s: i for i, s in enumerate(uniq)}
            self.sel = torch.tensor([sel_of[int(s)] for s in assign], dtype=torch.int32, device=dev)
            self.stacked = torch.empty(len(uniq) * layout.total_blocks * layout.block_size, dtype=torch.bfloat16,
                                       device=dev)
            self.bank.decode_stacked(uniq, out=self.stacked)
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            self.factors = self.bank.decode_stacked(uniq, out=self.stacked)
            torch.cuda.synchronize()
            self.decode_ms = (time.perf_counter() - t0) * 1e3
        for gi in groups:
            # one grouped call per (block, stage); with qkv the q / k / v of one input read one x
            xs, ys, offs, shared = [], [], [], {}
            for i in gi:
                n, di, do, m = mods[i]
                key = _SHARED_INPUT.get(_split(n)[1]) if qkv else None
                if key is None or key not in shared:
                    x = buf(di, m, xs + ys)
                    if key is not None:
                        shared[key] = x
                xs.append(shared[key] if key is not None else x)
                ys.append(buf(do, m, xs + ys))
                offs.append(layout.module(n)[3:5])
            if decoded:    # module m's factors at its layout offsets of the stacked buffer
                self.calls.append(prepare_stacked_group(xs, ys, self.stacked, len(uniq), offs, self.sel, rank, 1.0,
                                                        self.workspace, accumulate=True))
            else:
                self.calls.append(prepare_packed_group(xs, ys, self.bank.words, offs, 3, pools, self.assign, rank,
                                                       1.0, self.workspace, accumulate=True))
            self.call_mods.append([mods[i] for i in gi])
        k = len(mods) if grouped else 0
        while k < len(mods):
            n, di, do, m = mods[k]
            if qkv and (n.endswith("attn.to_q") or n.endswith("attn.add_q_proj")):
                # the three projections of one attention input read the same x
                group = mods[k:k + 3]
                x = buf(di, m)
                ys = []
                for g in group:
                    ys.append(buf(g[2], g[3], [x] + ys))
                offs = [layout.module(g[0])[3:5] for g in group]
                self.calls.append(prepare_packed_shared_x(x, ys, self.bank.words, offs, 3, pools, self.assign, rank,
                                                          1.0, self.workspace, accumulate=True))
                self.call_mods.append(group)
                k += 3
                continue
            k += 1
            self.call_mods.append([mods[k - 1]])
            _, _, _, a_off, b_off = layout.module(n)
            x = buf(di, m)
            y = buf(do, m, [x])
            if decoded:
                a, b = self.factors[n]
                self.calls.append(prepare_dense(x, y, a, b, self.sel, rank, 1.0, self.workspace, accumulate=True))
            else:
                self.calls.append(prepare_packed(x, y, self.bank.words, a_off, b_off, 3, pools, self.assign, rank,
                                                 1.0, self.workspace, accumulate=True))
        self.tokens = batch * max(m for _, _, _, m in mods) if name != "ffn" else batch * mods[0][3]
        if decoded:   # dense factors of the routed adapters instead of their packed words
            self.index_bytes = len(uniq) * sum(2 * rank * (di + do) for _, di, do, _ in mods)
        else:
            self.index_bytes = len(uniq) * layout.num_words * 8
        self.alg_bytes = sum(c.algorithmic_bytes() for c in self.calls) + self.index_bytes

    def sweep(self, stream):
        for c in self.calls:
            c(stream)


def time_sweeps(wl, steps, warmup, use_graph):
    import ctypes

    import torch
    stream = torch.cuda.current_stream()
    sp = ctypes.c_void_p(stream.cuda_stream)
    for _ in range(warmup):
        wl.sweep(sp)
    torch.cuda.synchronize()
    graph = None
    if use_graph:
        side = torch.cuda.Stream()
        side.wait_stream(stream)
        with torch.cuda.stream(side):
            wl.sweep(ctypes.c_void_p(side.cuda_stream))
        stream.wait_stream(side)
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            wl.sweep(ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
        for _ in range(max(1, warmup)):
            graph.replay()
        torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    start.record(stream)
    for _ in range(steps):
        if graph is not None:
            graph.replay()
        else:
            wl.sweep(sp)
    end.record(stream)
    torch.cuda.synchronize()
    return start.elapsed_time(end) / steps, graph is not None


def per_call_times(wl, sweeps=2):
    """Mean duration (ms) of every module's delta call, from HIP events on the launch stream."""
    import ctypes

    import torch
    stream = torch.cuda.current_stream()
    sp = ctypes.c_void_p(stream.cuda_stream)
    n = len(wl.calls)
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(n + 1)]
    tot = [0.0] * n
    for _ in range(sweeps):
        ev[0].record(stream)
        for i, c in enumerate(wl.calls):
            c(sp)
            ev[i + 1].record(stream)
        torch.cuda.synchronize()
        for i in range(n):
            tot[i] += ev[i].elapsed_time(ev[i + 1])
    return [t / sweeps for t in tot]


def copy_bandwidth_gbps():
    import torch
    a = torch.empty(1 << 30, dtype=torch.uint8, device="cuda")
    b = torch.empty_like(a)
    for _ in range(3):
        b.copy_(a)
    torch.cuda.synchronize()
    s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    s.record()
    for _ in range(10):
        b.copy_(a)
    e.record()
    torch.cuda.synchronize()
    ms = s.elapsed_time(e) / 10
    del a, b
    return 2 * (1 << 30) / (ms * 1e-3) / 1e9


def host_threads() -> int:
    """Host threads the CPU baselines use: the process's CPU affinity, capped by OMP_NUM_THREADS
    (the box's CPU share) when that is set."""
    n = len(os.sched_getaffinity(0))
    omp = os.environ.get("OMP_NUM_THREADS")
    if omp and omp.isdigit() and int(omp) > 0:
        n = min(n, int(omp))
    return n


def cpu_model() -> str:
    try:
        with open("/proc/cpuinfo") as fh:
            for line in fh:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def environment() -> dict:
    """ROCm, torch, GPU and host CPU of this run."""
    import torch
    rocm = None
    for p in ("/opt/rocm/.info/version", "/opt/rocm/.info/version-dev"):
        if os.path.exists(p):
            with open(p) as fh:
                rocm = fh.read().strip()
            break
    props = torch.cuda.get_device_properties(0)
    return {"rocm": rocm, "torch": torch.__version__, "torch_hip": torch.version.hip, "gpu": props.name,
            "gfx": getattr(props, "gcnArchName", None), "cus": props.multi_processor_count,
            "gpu_mem_GB": round(props.total_memory / 1e9, 1), "cpu_model": cpu_model(),
            "host_threads": host_threads()}


def cpu_baseline(mods, batch, n_slots, budget_s=20.0, rank=RANK):
    """The reference's serving forward restated in torch CPU ops (oracle.torch_cpu: fp32
    gather-sum decode of the routed adapters every forward, alpha / r folded into B, two bf16
    torch.bmm, the add into the base output) on the host cores.

    Sample: every sample of one module of each (d_in, d_out, tokens) class with the batch's
    routing (B distinct adapters of 3 levels of uniformly random indices), timed until about
    budget_s seconds of work (at least one pass), scaled to the sweep by class multiplicity.
    """
    import numpy as np
    import torch

    from oracle import codebook as ocb
    from oracle import torch_cpu
    threads = host_threads()
    torch.set_num_threads(threads)
    classes = {}
    for _, di, do, m in mods:
        classes[(di, do, m)] = classes.get((di, do, m), 0) + 1
    pa, pb = (torch.from_numpy(p) for p in ocb.twin_pools())
    g = torch.Generator().manual_seed(0)
    per_class = {}
    t_start = time.perf_counter()
    passes = 0
    while True:
        for (di, do, m) in sorted(classes):
            nba, nbb = rank * di // 64, do * rank // 64
            ia = [torch.randint(0, 512, (3, nba), generator=g, dtype=torch.int16) for _ in range(batch)]
            ib = [torch.randint(0, 512, (3, nbb), generator=g, dtype=torch.int16) for _ in range(batch)]
            x = torch.randn(batch, m, di, generator=g).bfloat16()
            y = torch.randn(batch, m, do, generator=g).bfloat16()
            ids = torch.arange(batch).view(batch, 1)
            w = torch.ones(batch, 1)
            scales = torch.ones(batch)
            t = time.perf_counter()
            torch_cpu.routed_add(x, y, ids, w, ia, ib, scales, pa, pb, rank)
            dt = time.perf_counter() - t
            per_class[(di, do, m)] = min(per_class.get((di, do, m), dt), dt)
            del x, y
        passes += 1
        if time.perf_counter() - t_start > budget_s:
            break
    sweep_s = sum(per_class[k] * c for k, c in classes.items())
    tokens = batch * max(m for _, _, _, m in mods)
    return {"value": round(tokens / sweep_s, 1), "unit": "tokens/s", "cores": threads, "kind": "port",
            "cpu_model": cpu_model(), "sweep_s": round(sweep_s, 3),
            "sample": f"torch CPU restatement of the reference's serve.py forward (bf16 bmm, per-forward fp32 decode "
                      f"of the {batch} routed adapters), all {batch} samples of one module of each of {len(classes)} "
                      f"(d_in, d_out, tokens) classes, best of {passes} pass(es), scaled by class count to the "
                      f"{len(mods)}-module sweep; {threads} threads"}


def cpu_decode_baseline(layout, budget_s=10.0):
    """Oracle C restatement of the bulk decode (OpenMP over the host cores): adapters decoded
    one after another until about budget_s seconds of decode time (at least 2)."""
    import numpy as np

    from oracle import codebook as ocb
    from oracle import native
    pa, pb = ocb.twin_pools()
    rng = np.random.default_rng(0)
    n_idx = layout.num_indices
    sides = layout.sides.numpy()
    words = [native.pack(rng.integers(0, 512, n_idx).astype(np.uint16)) for _ in range(2)]
    t, n_sample = 0.0, 0
    while n_sample < 2 or t < budget_s:
        t0 = time.perf_counter()
        native.decode(words[n_sample % 2], layout.total_blocks, layout.num_levels, sides, pa, pb, want="bf16")
        t += time.perf_counter() - t0
        n_sample += 1
    per = t / n_sample
    nbytes = layout.num_words * 8 + layout.total_blocks * 64 * 2
    return {"value": round(nbytes / per / 1e9, 3), "unit": "GB/s", "adapters_per_s": round(1.0 / per, 3),
            "cores": int(os.environ.get("OMP_NUM_THREADS", len(os.sched_getaffinity(0)))), "kind": "port",
            "sample": f"oracle C decode (lo_decode, OpenMP) of {n_sample} packed adapters of the 342-linear "
                      f"layout to bf16 ({t:.1f} s)"}


def run_decode(args):
    """Bulk decode of a 10,000-adapter packed bank to dense bf16 A/B, chunked into a reused buffer."""
    import torch

    from lithe_amd.kernels import PackedBank, PackedLayout
    rank = args.rank
    dev = torch.device("cuda:0")
    mods = flux_modules(4096, 512)
    layout = PackedLayout.from_modules(
        [{"name": n, "shape_a": [rank, di], "shape_b": [do, rank]} for n, di, do, _ in mods],
        num_levels=3, block_size=64, scaling=1.0)
    n_slots = args.slots or 10_000
    bank = PackedBank(layout, dev, capacity=n_slots)
    bank.fill_random(n_slots, generator=torch.Generator(device=dev).manual_seed(0))
    out_per = layout.total_blocks * 64 * 2
    in_per = layout.num_words * 8
    chunk = max(1, min(n_slots, (6 << 30) // out_per))     # ~6 GB output buffer, reused
    out = torch.empty((chunk, layout.total_blocks, 64), dtype=torch.bfloat16, device=dev)
    chunks = [torch.arange(s, min(n_slots, s + chunk), dtype=torch.int32, device=dev)
              for s in range(0, n_slots, chunk)]

    def step():
        for c in chunks:
            bank.decode_slots(c, out=out[: c.numel()])

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream()
    s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    s.record(stream)
    for _ in range(args.steps):
        step()
    e.record(stream)
    torch.cuda.synchronize()
    ms = s.elapsed_time(e) / args.steps
    # per-launch duration of the full chunks, HIP events on the launch stream
    full = [c for c in chunks if c.numel() == chunk]
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(len(full) + 1)]
    ev[0].record(stream)
    for i, c in enumerate(full):
        bank.decode_slots(c, out=out)
        ev[i + 1].record(stream)
    torch.cuda.synchronize()
    launch_ms = sum(ev[i].elapsed_time(ev[i + 1]) for i in range(len(full))) / len(full)
    launch_bytes = chunk * (in_per + out_per)
    achieved = launch_bytes / (launch_ms * 1e-3) / 1e9
    total_bytes = n_slots * (in_per + out_per)
    traffic = None
    tpath = os.path.join(ROOT, "profiles", f"traffic_decode_r{rank}.json")
    if os.path.exists(tpath):
        with open(tpath) as fh:
            traffic = json.load(fh).get("hbm_bytes_per_launch")
    line = {
        "metric": "bulk decode GB/s (packed 9-bit indices -> dense bf16 A/B), 342 FLUX linears",
        "value": round(total_bytes / (ms * 1e-3) / 1e9, 1),
        "unit": "GB/s",
        "n_gpus": 1, "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(ms, 3),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "bf16", "data": "synthetic",
        "config": {"workload": f"bulk decode of a {n_slots}-adapter packed bank (342 FLUX.1-dev linears, rank "
                               f"{rank}) to dense bf16, {chunk} adapters per launch into a reused buffer",
                   "rank": rank, "bank_slots": n_slots, "bank_GB": round(n_slots * in_per / 1e9, 2),
                   "adapters_per_launch": chunk, "out_MB_per_adapter": round(out_per / 1e6, 2)},
        "adapters_per_s": round(n_slots / (ms * 1e-3), 1),
        "roofline": {"kernel": "decode_packed3_lines_kernel (lithe_decode)", "bound": "hbm", "achieved": round(achieved, 1),
                     "peak": HBM_PEAK_GBPS, "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBPS, 4),
                     "traffic": traffic, "algorithmic_bytes_per_launch": launch_bytes,
                     "mean_launch_ms": round(launch_ms, 4)},
        "copy_GBps": round(copy_bandwidth_gbps(), 1),
        "cpu_baseline": None if args.no_cpu else cpu_decode_baseline(layout),
    }
    print(json.dumps(line), flush=True)


def run_ingest(args):
    """Cold swap into a resident 10,000-slot bank: adapter file on disk -> packed slot ready to serve."""
    import tempfile

    import numpy as np
    import torch

    from lithe_amd import fileio
    from lithe_amd.kernels import PackedBank, PackedLayout, _hip
    from oracle import packing as opk
    dev = torch.device("cuda:0")
    mods = flux_modules(4096, 512)
    modules = [{"name": n, "shape_a": [RANK, di], "shape_b": [do, RANK]} for n, di, do, _ in mods]
    layout = PackedLayout.from_modules(modules, num_levels=3, block_size=64, scaling=1.0)
    n_slots = args.slots or 10_000
    bank = PackedBank(layout, dev, capacity=n_slots)
    bank.fill_random(n_slots, generator=torch.Generator(device=dev).manual_seed(0))
    rng = np.random.default_rng(0)
    n_files = 4
    tmp = tempfile.mkdtemp(prefix="lithe_ingest_")
    lithe_paths, blob_paths, streams = [], [], []
    for i in range(n_files):
        idx = {m["name"]: {"A": rng.integers(0, 512, (3, opk.num_blocks(m["shape_a"]))).astype(np.uint16),
                           "B": rng.integers(0, 512, (3, opk.num_blocks(m["shape_b"]))).astype(np.uint16)}
               for m in modules}
        ad = fileio.LitheAdapter(modules=modules, indices=idx, rank=RANK, alpha=float(RANK))
        p = os.path.join(tmp, f"a{i}.lithe")
        fileio.save_lithe(p, ad)
        lithe_paths.append(p)
        b = os.path.join(tmp, f"a{i}.int16.bin")
        opk.stream_order(ad, opk.layout_of(ad)).astype(np.int16).tofile(b)
        blob_paths.append(b)
        streams.append(np.frombuffer(ad.raw_stream(), "<u2"))
    file_mb = sum(os.path.getsize(p) for p in lithe_paths) / n_files / 1e6

    def timed(fn, n):
        for i in range(2):
            fn(i)
        torch.cuda.synchronize()
        ts = []
        for i in range(n):
            t0 = time.perf_counter()
            fn(i)
            torch.cuda.synchronize()
            ts.append((time.perf_counter() - t0) * 1e3)
        ts.sort()
        return {"mean_ms": round(sum(ts) / len(ts), 4), "p50_ms": round(ts[len(ts) // 2], 4),
                "p99_ms": round(ts[min(len(ts) - 1, int(0.99 * len(ts)))], 4)}

    slot = n_slots - 1
    n = max(8, args.steps)
    res = {
        "lithe_file": timed(lambda i: bank.load_lithe(lithe_paths[i % n_files], slot=slot), n),
        "lithe_file_noverify": timed(lambda i: bank.load_lithe(lithe_paths[i % n_files], slot=slot, verify=False), n),
        "raw_blob": timed(lambda i: bank.load_blob(blob_paths[i % n_files], slot=slot), n),
        "stream_device_pack": timed(lambda i: bank.load_stream(streams[i % n_files], slot=slot), n),
        "stream_host_pack": timed(lambda i: bank.load_stream(streams[i % n_files], slot=slot, on_device=False), n),
        "decode_on_swap": timed(lambda i: bank.decode(slot), n),
    }
    # the device reorder + pack kernel alone, HIP events on the launch stream
    stream_t = torch.from_numpy(streams[0].view(np.int16).copy()).to(dev)
    table = layout.ingest_table().to(dev)
    err = torch.zeros(1, dtype=torch.int32, device=dev)
    lib = _hip.load()
    row = bank.words[slot]
    cs = torch.cuda.current_stream()
    s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    for _ in range(3):
        lib.lithe_ingest(_hip.ptr(stream_t), stream_t.numel(), 3, table.shape[0], _hip.ptr(table), _hip.ptr(row),
                         layout.num_words, _hip.ptr(err), _hip.stream_of(dev))
    s.record(cs)
    reps = 50
    for _ in range(reps):
        lib.lithe_ingest(_hip.ptr(stream_t), stream_t.numel(), 3, table.shape[0], _hip.ptr(table), _hip.ptr(row),
                         layout.num_words, _hip.ptr(err), _hip.stream_of(dev))
    e.record(cs)
    torch.cuda.synchronize()
    k_ms = s.elapsed_time(e) / reps
    k_bytes = layout.num_indices * 2 + layout.num_words * 8
    assert int(err.item()) == 0
    cpu = None
    if not args.no_cpu:
        # the same raw-blob path in the oracle: read the residency-ordered int16 blob, 9-bit pack
        t0, k = time.perf_counter(), 0
        while k < 20 or time.perf_counter() - t0 < 10.0:
            opk.pack(np.fromfile(blob_paths[k % n_files], dtype=np.int16))
            k += 1
        per = (time.perf_counter() - t0) / k
        t1, kl = time.perf_counter(), 0
        while kl < 2 or time.perf_counter() - t1 < 5.0:
            _, st = fileio.read_stream(lithe_paths[kl % n_files])
            opk.pack(opk.residency_from_file_stream(st, modules, 3))
            kl += 1
        res["oracle_lithe_file_ms"] = round((time.perf_counter() - t1) / kl * 1e3, 2)
        cpu = {"value": round(per * 1e3, 3), "unit": "ms per swap", "cores": 1, "kind": "port",
               "sample": f"oracle (numpy) read of the residency-ordered int16 blob + 9-bit pack, {k} blobs of the "
                         f"342-linear layout (the .lithe path, LZMA included: {kl} files, in paths)"}
    for p in lithe_paths + blob_paths:
        os.remove(p)
    os.rmdir(tmp)
    line = {
        "metric": "cold-swap latency: adapter index blob on disk -> packed bank slot ready to serve "
                  "(342 FLUX linears, rank 16)",
        "value": res["raw_blob"]["mean_ms"], "unit": "ms", "n_gpus": 1, "steps": n, "warmup": 2,
        "ms_per_step": res["raw_blob"]["mean_ms"], "higher_is_better": False, "scaling": "weak",
        "vs_baseline": None, "dtype": "u16->u64", "data": "synthetic",
        "config": {"workload": f"cold swap of one adapter ({layout.num_indices} indices: residency-ordered int16 "
                               f"blob of {layout.num_indices * 2 / 1e6:.2f} MB, or a .lithe file of {file_mb:.2f} "
                               f"MB) into slot {slot} of a resident {n_slots}-slot packed bank",
                   "bank_slots": n_slots, "slot_MB": round(layout.num_words * 8 / 1e6, 3)},
        "paths": res,
        "roofline": {"kernel": "ingest_kernel (lithe_ingest)", "bound": "hbm",
                     "achieved": round(k_bytes / (k_ms * 1e-3) / 1e9, 1), "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                     "frac": round(k_bytes / (k_ms * 1e-3) / 1e9 / HBM_PEAK_GBPS, 4), "traffic": None,
                     "algorithmic_bytes_per_launch": k_bytes, "mean_launch_ms": round(k_ms, 5)},
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)


def run_encode(args):
    """GPU re-quantisation: a dense rank-16 adapter of the 342 FLUX linears -> packed bank slot."""
    import ctypes

    import numpy as np
    import torch

    from lithe_amd.kernels import PackedBank, PackedLayout, _hip
    dev = torch.device("cuda:0")
    mods = flux_modules(4096, 512)
    layout = PackedLayout.from_modules(
        [{"name": n, "shape_a": [RANK, di], "shape_b": [do, RANK]} for n, di, do, _ in mods],
        num_levels=3, block_size=64, scaling=1.0)
    bank = PackedBank(layout, dev, capacity=4)
    gen = torch.Generator(device=dev).manual_seed(0)
    # synthetic dense factors at the codebook's scales (A ~ 0.06 N(0,1), B ~ 0.0025 N(0,1))
    factors = {n: (0.06 * torch.randn(RANK, di, device=dev, generator=gen),
                   0.0025 * torch.randn(do, RANK, device=dev, generator=gen)) for n, di, do, _ in mods}
    for _ in range(args.warmup):
        bank.encode_factors(factors, slot=0 if bank.num_slots else None)
    torch.cuda.synchronize()
    n = max(5, args.steps)
    t0 = time.perf_counter()
    for _ in range(n):
        bank.encode_factors(factors, slot=0)
    torch.cuda.synchronize()
    e2e_ms = (time.perf_counter() - t0) / n * 1e3
    # the encode kernel alone over the adapter's blocks (residency order, both pools)
    blocks = torch.randn(layout.total_blocks, 64, device=dev, generator=gen) * 0.01
    idx = torch.empty(layout.total_blocks * 3, dtype=torch.int16, device=dev)
    lut_a = _hip.lut_from_pools(bank.pool_a, torch.float32)
    lut_b = _hip.lut_from_pools(bank.pool_b, torch.float32)
    lib = _hip.load()
    sides = layout.sides_on(dev)

    def launch():
        lib.lithe_encode(_hip.ptr(blocks), layout.total_blocks, _hip.ptr(sides), ctypes.byref(lut_a),
                         ctypes.byref(lut_b), _hip.ptr(idx), _hip.DT_I16, 1, 3, None, _hip.stream_of(dev))

    for _ in range(3):
        launch()
    cs = torch.cuda.current_stream()
    s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    s.record(cs)
    reps = 50
    for _ in range(reps):
        launch()
    e.record(cs)
    torch.cuda.synchronize()
    k_ms = s.elapsed_time(e) / reps
    k_bytes = layout.total_blocks * (64 * 4 + 3 * 2 + 1)      # fp32 block in, 3 int16 indices + side byte
    cpu = None
    if not args.no_cpu:
        from oracle import codebook as ocb
        from oracle import search as osr
        pa, _ = ocb.twin_pools()
        sample = blocks[:100_000].cpu().numpy()
        t0, k = time.perf_counter(), 0
        while k < 1 or time.perf_counter() - t0 < 10.0:
            osr.rvq_encode_blocks(sample, pa)
            k += 1
        per_block = (time.perf_counter() - t0) / (k * sample.shape[0])
        cpu = {"value": round(per_block * layout.total_blocks * 1e3, 1), "unit": "ms per adapter", "cores": 1,
               "kind": "port", "sample": f"oracle greedy encode (numpy, float64 projections) of {k} x 100,000 blocks, "
                                       f"scaled to the adapter's {layout.total_blocks} blocks"}
    line = {
        "metric": "GPU re-quantisation latency: dense rank-16 adapter (342 FLUX linears) -> packed bank slot",
        "value": round(e2e_ms, 3), "unit": "ms", "n_gpus": 1, "steps": n, "warmup": args.warmup,
        "ms_per_step": round(e2e_ms, 3), "higher_is_better": False, "scaling": "weak", "vs_baseline": None,
        "dtype": "f32", "data": "synthetic",
        "config": {"workload": f"closed-form greedy 3-level encode of {layout.total_blocks} blocks (fp32 factors "
                               f"blockified in layout order) + 9-bit pack into a slot", "rank": RANK,
                   "blocks": layout.total_blocks},
        "roofline": {"kernel": "encode_kernel (lithe_encode)", "bound": "hbm",
                     "achieved": round(k_bytes / (k_ms * 1e-3) / 1e9, 1), "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                     "frac": round(k_bytes / (k_ms * 1e-3) / 1e9 / HBM_PEAK_GBPS, 4), "traffic": None,
                     "algorithmic_bytes_per_launch": k_bytes, "mean_launch_ms": round(k_ms, 4)},
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)


def main():
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=None, help="timed steps (default 20; 200 for --config ffn, "
                    "whose step is 0.35 ms)")
    ap.add_argument("--warmup", type=int, default=None, help="untimed steps (default 3; 20 for --config ffn)")
    ap.add_argument("--config", default="grouped",
                    choices=["grouped", "flux342", "fused", "qkv", "decoded", "decoded_grouped", "ffn", "hb",
                             "hb_modules", "decode",
                             "ingest", "encode"])
    ap.add_argument("--rank", type=int, default=RANK, help="adapter rank (a multiple of 16; the headline and the "
                    "decode's first line are rank 16, its second rank 64)")
    ap.add_argument("--no-graph", action="store_true", help="launch every call from Python instead of a HIP graph")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--slots", type=int, default=None, help="bank size (default: the configuration's)")
    args = ap.parse_args()
    short = args.config == "ffn"
    args.steps = args.steps if args.steps is not None else (200 if short else 20)
    args.warmup = args.warmup if args.warmup is not None else (20 if short else 3)
    if args.gpus != 1:
        print(f"bench.py measures one GPU; --gpus {args.gpus} is not supported (the path needs no "
              "collective: samples shard across GPUs with no exchange).", file=sys.stderr)
        sys.exit(2)

    import numpy as np
    import torch

    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        sys.exit(2)
    from lithe_amd.kernels import _hip
    _hip.load()
    if args.config == "decode":
        run_decode(args)
        return
    if args.config == "ingest":
        run_ingest(args)
        return
    if args.config == "encode":
        run_encode(args)
        return
    rng = np.random.default_rng(1234)
    if args.config in ("flux342", "decoded", "decoded_grouped", "qkv", "grouped", "fused"):
        mods, batch, n_slots = flux_modules(4096, 512), 14, args.slots or 10_000
        assign = rng.choice(n_slots, batch, replace=False)
        wl = Workload(args.config, mods, batch, n_slots, assign, decoded=args.config in ("decoded", "decoded_grouped"),
                      qkv=args.config in ("qkv", "fused"),
                      grouped=args.config in ("grouped", "fused", "decoded_grouped"), rank=args.rank)
        workload = "FLUX.1-dev 342 linears, 1024^2: B=14 x 4608 tokens (4096 img + 512 txt), 10k-adapter packed bank"
        if args.config in ("decoded", "decoded_grouped"):
            workload += (", decoded mode: the 14 routed adapters decoded once to stacked bf16 factors "
                         "(decode-on-swap), modules read dense factors")
        if args.config in ("qkv", "fused"):
            workload += ", q/k/v fused: the three projections of each attention input read x once"
        if args.config in ("grouped", "fused", "decoded_grouped"):
            workload += (", grouped: the independent linears of each block stage (image + text projections, "
                         "attention outputs, up and down projections) in one shrink + one expand launch")
        if args.config != "flux342":
            workload += f" ({len(wl.calls)} calls per sweep)"
    elif args.config in ("hb", "hb_modules"):
        mods, batch, n_slots = flux_modules(256, 512), 96, args.slots or 10_000
        ranks = np.arange(1, n_slots + 1, dtype=np.float64)
        p = ranks ** -1.1
        p /= p.sum()
        perm = rng.permutation(n_slots)
        assign = perm[rng.choice(n_slots, batch, p=p)]
        wl = Workload("hb", mods, batch, n_slots, assign, grouped=args.config == "hb", rank=args.rank)
        workload = "FLUX.1-dev 342 linears, 256^2: B=96 x 768 tokens (256 img + 512 txt), Zipf(1.1) over 10k bank"
        workload += (", grouped: one shrink + one expand launch per block stage" if args.config == "hb"
                     else ", one call per module") + f" ({len(wl.calls)} calls per sweep)"
    else:
        full = flux_modules(1024, 512)
        mods = [("transformer_blocks.0.ff.net.0.proj", 3072, 12288, 1536),
                ("transformer_blocks.0.ff.net.2", 12288, 3072, 1536)]
        batch, n_slots = 14, args.slots or 1_000
        assign = rng.choice(n_slots, batch, replace=False)
        wl = Workload("ffn", mods, batch, n_slots, assign, layout_mods=full, rank=args.rank)
        workload = "FLUX FFN pair 3072->12288->3072 at 512^2: B=14 x 1536 tokens, 1k-adapter packed bank"

    if args.rank != RANK:
        workload += f", rank {args.rank}"
    ms, graphed = time_sweeps(wl, args.steps, args.warmup, not args.no_graph)
    # the kernels record bad slot ids and out-of-range indices in the workspace's error word
    import ctypes
    from lithe_amd.kernels import _hip
    kflags = ctypes.c_int32(0)
    _hip.check(_hip.load().lithe_workspace_errors(_hip.ptr(wl.workspace), ctypes.byref(kflags), 1, None),
               "lithe_workspace_errors")
    if kflags.value:
        raise RuntimeError(f"the delta kernels recorded errors during the timed sweeps (flags {kflags.value})")
    tokens = wl.tokens
    value = tokens / (ms * 1e-3)
    per = per_call_times(wl)
    call_ms = sum(per)
    achieved = wl.alg_bytes / (call_ms * 1e-3) / 1e9
    classes = {}
    for group, t, c in zip(wl.call_mods, per, wl.calls):
        _, di, do, m = group[0]
        if len(group) == 1:
            k = f"{di}->{do} x {m}"
        elif args.config in ("grouped", "fused", "hb", "decoded_grouped"):
            k = "group " + " + ".join(sorted({f"{g[1]}->{g[2]} x {g[3]}" for g in group}))
        else:
            k = f"{di}->{len(group)}x{do} x {m} (shared x)"
        e = classes.setdefault(k, {"count": 0, "ms": 0.0, "bytes": 0})
        e["count"] += 1
        e["ms"] += t
        e["bytes"] += c.algorithmic_bytes()
    for e in classes.values():
        e["GBps"] = round(e["bytes"] / (e["ms"] * 1e-3) / 1e9, 1)
        e["ms"] = round(e["ms"], 3)
        del e["bytes"]
    traffic = None
    tpath = os.path.join(ROOT, "profiles", f"traffic_{args.config}.json")
    if os.path.exists(tpath) and args.rank == RANK:     # the committed counter runs are rank 16
        with open(tpath) as fh:
            traffic = json.load(fh).get("hbm_bytes_per_launch")
    copy_gbps = copy_bandwidth_gbps()
    cpu = None if args.no_cpu else cpu_baseline(wl.mods, batch, n_slots, rank=args.rank)
    line = {
        "metric": "adapter-delta tokens/s + achieved HBM GB/s (% peak), FLUX linears, B=14 mixed",
        "value": round(value, 1),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {"workload": workload, "modules": len(wl.mods), "global_batch": batch,
                   "tokens_per_step": tokens, "rank": args.rank, "bank_slots": n_slots,
                   "bank_GB": round(wl.bank.words.numel() * 8 / 1e9, 2), "hip_graph": graphed,
                   "calls_per_step": len(wl.calls)},
        "achieved_GBps": round(wl.alg_bytes / (ms * 1e-3) / 1e9, 1),
        "frac_of_peak": round(wl.alg_bytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBPS, 4),
        "roofline": {"kernel": {"qkv": "lithe_lora_delta per module; lithe_lora_delta_shared_x for q / k / v (one shrink + "
                                       "one grouped expand launch)",
                                "grouped": "lithe_lora_delta_grouped (one shrink + one expand launch per block stage)",
                                "fused": "lithe_lora_delta_grouped (one shrink + one expand launch per block stage, "
                                         "q/k/v sharing x)",
                                "hb": "lithe_lora_delta_grouped (one shrink + one expand launch per block stage)",
                                "decoded_grouped": "lithe_lora_delta_grouped over dense stacked factors (one shrink + "
                                                   "one expand launch per block stage)"}.get(
                                    args.config,
                                                                 "lithe_lora_delta (shrink + expand, one call per module)"),
                     "bound": "hbm",
                     "achieved": round(achieved, 1), "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBPS, 4), "traffic": traffic,
                     "algorithmic_bytes_per_step": wl.alg_bytes,
                     "mean_call_ms": round(call_ms / len(per), 5)},
        "classes": classes,
        "copy_GBps": round(copy_gbps, 1),
        "kernel_error_flags": kflags.value,
        "cpu_baseline": cpu,
        "env": environment(),
    }
    if wl.decode_ms is not None:
        line["decode_on_swap_ms"] = round(wl.decode_ms, 4)
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
