"""GPU checks of the delta under the serving patterns the bench uses: HIP-graph replay
(every replay equal to the eager result, bit for bit), calls on two streams at once, repeated
slots (Zipf-style batches where several samples share an adapter) and empty routes (-1: the
base output stays untouched)."""
import ctypes

import numpy as np
import pytest
import torch

from lithe_amd.kernels import PackedBank
from lithe_amd.kernels.prepared import prepare_packed, shared_workspace, workspace_bytes
from oracle import codebook as ocb
from oracle import delta as odelta

from helpers import random_adapter, rel, to_np

pytestmark = pytest.mark.gpu
MODS = [("q", 3072, 3072), ("up", 3072, 12288), ("txt", 3072, 3072)]


def _bank(n=5):
    ads = [random_adapter(MODS, rank=16, seed=40 + s) for s in range(n)]
    bank, words = PackedBank.from_adapters(ads, "cuda")
    for w in words:
        bank.add(w)
    return ads, bank


def _calls(bank, slots, shapes, seed=0):
    gen = torch.Generator(device="cuda").manual_seed(seed)
    pools = (bank.pool_a.bfloat16(), bank.pool_b.bfloat16())
    need = max(workspace_bytes((len(slots), m, di), do, 16, 1, torch.bfloat16) for _, di, do, m in shapes)
    ws = shared_workspace("cuda", need)
    out = []
    for name, di, do, m in shapes:
        _, _, _, a_off, b_off = bank.layout.module(name)
        x = torch.randn(len(slots), m, di, device="cuda", generator=gen).bfloat16()
        y0 = torch.randn(len(slots), m, do, device="cuda", generator=gen).bfloat16()
        y = y0.clone()
        c = prepare_packed(x, y, bank.words, a_off, b_off, 3, pools, slots, 16, 0.75, ws)
        out.append((c, x, y0, y))
    return out, ws


def test_graph_replays_match_eager():
    _, bank = _bank()
    slots = torch.tensor([4, 1, 1, 0], dtype=torch.int32, device="cuda")
    calls, ws = _calls(bank, slots, [("q", 3072, 3072, 130), ("up", 3072, 12288, 64), ("txt", 3072, 3072, 17)])
    stream = torch.cuda.current_stream()
    for c, _, y0, y in calls:
        y.copy_(y0)
        c(ctypes.c_void_p(stream.cuda_stream))
    torch.cuda.synchronize()
    eager = [y.clone() for _, _, _, y in calls]

    side = torch.cuda.Stream()
    side.wait_stream(stream)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=side):
        for c, _, y0, y in calls:
            y.copy_(y0)
            c(ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
    torch.cuda.synchronize()
    noise = torch.randn(1024, 1024, device="cuda")
    for rep in range(4):
        for _, _, _, y in calls:
            y.fill_(7.0)
        g.replay()
        torch.cuda.synchronize()
        for i, (_, _, _, y) in enumerate(calls):
            assert torch.equal(y, eager[i]), (rep, i)
        noise = noise @ noise.T / 1024.0     # eager work between replays
        torch.cuda.synchronize()


def test_repeated_slots_and_empty_routes():
    ads, bank = _bank()
    slot_list = [3, 3, 0, -1, 3, 1, 1, -1]     # heavy repeats, two samples without an adapter
    slots = torch.tensor(slot_list, dtype=torch.int32, device="cuda")
    calls, _ = _calls(bank, slots, [("q", 3072, 3072, 40), ("up", 3072, 12288, 24)], seed=3)
    for c, x, y0, y in calls:
        x[1].copy_(x[0])      # samples 0 and 1 share slot 3 and now their inputs
        y0[1].copy_(y0[0])
        y.copy_(y0)
        c()
    torch.cuda.synchronize()
    opa, opb = ocb.twin_pools()
    for (c, x, y0, y), name in zip(calls, ("q", "up")):
        live = [i for i, s in enumerate(slot_list) if s >= 0]
        ia = np.stack([a.indices[name]["A"].astype(np.int64) for a in ads])
        ib = np.stack([a.indices[name]["B"].astype(np.int64) for a in ads])
        xs = to_np(x)[live]
        d = odelta.shared_delta(xs, ia, opa, ib, opb, [slot_list[i] for i in live], 16, y.shape[2], 0.75, "bf16")
        want = to_np(y0).copy()
        want[live] = odelta.index_linear(to_np(y0)[live], d, "bf16")
        got = to_np(y)
        empty = [i for i, s in enumerate(slot_list) if s < 0]
        assert np.array_equal(got[empty], to_np(y0)[empty])       # untouched, bit for bit
        assert rel(got[live], want[live]) < 2e-3
        # samples routed to the same slot see the same factors: equal inputs give equal outputs
        assert np.array_equal(got[0], got[1])


def test_two_streams_at_once_match_one_stream():
    """Calls enqueued on two streams at the same time (each stream has its own workspace) give
    the results of the same calls on one stream, bit for bit, on every repetition."""
    from lithe_amd.kernels import _hip, packed_lora_delta
    _, bank = _bank()
    pools = (bank.pool_a.bfloat16(), bank.pool_b.bfloat16())
    gen = torch.Generator(device="cuda").manual_seed(5)
    work = []
    for name, di, do in MODS:
        _, _, _, a_off, b_off = bank.layout.module(name)
        for assign in ([4, 1, 1, 0], [2, 3, 0, 2]):
            x = torch.randn(4, 200, di, device="cuda", generator=gen).bfloat16()
            a = torch.tensor(assign, dtype=torch.int32, device="cuda")
            work.append((x, a, a_off, b_off, do))

    def run(x, a, a_off, b_off, do):
        return packed_lora_delta(x, bank.words, a_off, b_off, 3, pools, a, 16, do, 0.75)

    want = [run(*w) for w in work]
    torch.cuda.synchronize()
    streams = (torch.cuda.Stream(), torch.cuda.Stream())
    for s in streams:
        s.wait_stream(torch.cuda.current_stream())
    for rep in range(3):
        got = []
        for i, w in enumerate(work):
            with torch.cuda.stream(streams[i % 2]):
                got.append(run(*w))
        torch.cuda.synchronize()
        for i, (g, e) in enumerate(zip(got, want)):
            assert torch.equal(g, e), (rep, i)
    assert _hip.workspace_errors() == 0


def test_grown_workspace_keeps_recorded_errors():
    """A bad slot id is recorded in the stream's workspace; a larger call that grows the workspace
    afterwards keeps the recorded bit (workspace_errors reports it once, then it is cleared)."""
    from lithe_amd.kernels import _hip, packed_lora_delta
    _, bank = _bank()
    pools = (bank.pool_a.bfloat16(), bank.pool_b.bfloat16())
    _, _, _, a_off, b_off = bank.layout.module("q")
    _hip.workspace_errors()                                          # start clean
    small = torch.randn(1, 16, 3072, device="cuda").bfloat16()
    packed_lora_delta(small, bank.words, a_off, b_off, 3, pools, torch.tensor([bank.num_slots], device="cuda"),
                      16, 3072, 1.0)
    big = torch.randn(8, 20_000, 3072, device="cuda").bfloat16()    # 5.1 MB of intermediate: a new workspace
    packed_lora_delta(big, bank.words, a_off, b_off, 3, pools, torch.zeros(8, dtype=torch.int32, device="cuda"),
                      16, 3072, 1.0)
    assert _hip.workspace_errors() == 1
    assert _hip.workspace_errors() == 0
