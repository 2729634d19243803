"""GPU parity of the shared-input call (lithe_lora_delta_shared_x): the q / k / v projections of
one attention block read x once. Where both plans give every wave a whole K range the outputs
equal three separate lithe_lora_delta calls bit for bit (same MFMA sequence per rank group);
otherwise they match the oracle at the bf16 tolerance of the other delta tests. Each test runs
both shrink forms (LITHE_SHARED_X_STACKED: the modules as rank groups of one workgroup, or one
workgroup per tile and module)."""
import ctypes

import numpy as np
import pytest
import torch

from lithe_amd.kernels import PackedBank, _delta, _hip
from lithe_amd.kernels.prepared import (PreparedSharedX, prepare_packed, prepare_packed_shared_x, shared_workspace,
                                        workspace_bytes)
from oracle import codebook as ocb
from oracle import delta as odelta

from helpers import random_adapter, rel, to_np

pytestmark = pytest.mark.gpu
MODS = [("q", 3072, 3072), ("k", 3072, 3072), ("v", 3072, 3072), ("wide", 3072, 4096)]


def _bank(rank=16, n=5):
    ads = [random_adapter(MODS, rank=rank, seed=90 + s) for s in range(n)]
    bank, words = PackedBank.from_adapters(ads, "cuda")
    for w in words:
        bank.add(w)
    return ads, bank


def _run(bank, names, slots, seq, seed, rank=16):
    gen = torch.Generator(device="cuda").manual_seed(seed)
    b = slots.shape[0]
    x = torch.randn(b, seq, 3072, device="cuda", generator=gen).bfloat16()
    dims = {n: do for n, _, do in MODS}
    y0 = [torch.randn(b, seq, dims[n], device="cuda", generator=gen).bfloat16() for n in names]
    pools = (bank.pool_a.bfloat16(), bank.pool_b.bfloat16())
    offs = [bank.layout.module(n)[3:5] for n in names]
    ws = shared_workspace("cuda", workspace_bytes((b, seq, 3072), max(dims.values()), rank, len(names), torch.bfloat16))
    fused = [y.clone() for y in y0]
    prepare_packed_shared_x(x, fused, bank.words, offs, 3, pools, slots, rank, 0.5, ws)()
    sep = [y.clone() for y in y0]
    for (ao, bo), y in zip(offs, sep):
        prepare_packed(x, y, bank.words, ao, bo, 3, pools, slots, rank, 0.5, ws)()
    torch.cuda.synchronize()
    return x, y0, fused, sep


FORMS = pytest.mark.parametrize("form", ["1", "0"], ids=["stacked", "replicated"])


@FORMS
def test_shared_x_equals_separate_calls_with_whole_k_waves(monkeypatch, form):
    monkeypatch.setenv("LITHE_SHARED_X_STACKED", form)
    _, bank = _bank()
    slots = torch.tensor([4, 1, 1, 0], dtype=torch.int32, device="cuda")
    _, y0, fused, sep = _run(bank, ["q", "k", "v"], slots, 8192, 1)      # 4 x 512 token groups: whole-K waves
    for i in range(3):
        assert torch.equal(fused[i], sep[i]), i
        assert not torch.equal(fused[i], y0[i])


@pytest.mark.parametrize("names,seq", [(["q", "k", "v"], 77), (["q", "wide"], 130), (["k", "v", "q", "wide"], 33)])
@FORMS
def test_shared_x_matches_oracle(monkeypatch, form, names, seq):
    monkeypatch.setenv("LITHE_SHARED_X_STACKED", form)
    ads, bank = _bank()
    slot_list = [3, -1, 0, 3]
    slots = torch.tensor(slot_list, dtype=torch.int32, device="cuda")
    x, y0, fused, sep = _run(bank, names, slots, seq, 2)
    pa, pb = ocb.twin_pools()
    live = [i for i, s in enumerate(slot_list) if s >= 0]
    for name, yf, ys, yb in zip(names, fused, sep, y0):
        ia = np.stack([a.indices[name]["A"].astype(np.int64) for a in ads])
        ib = np.stack([a.indices[name]["B"].astype(np.int64) for a in ads])
        d = odelta.shared_delta(to_np(x)[live], ia, pa, ib, pb, [slot_list[i] for i in live], 16, yb.shape[2], 0.5,
                                "bf16")
        want = to_np(yb).copy()
        want[live] = odelta.index_linear(to_np(yb)[live], d, "bf16")
        got = to_np(yf)
        assert np.array_equal(got[1], to_np(yb)[1])                  # empty route: untouched
        assert rel(got[live], want[live]) < 2e-3, name
        assert rel(got, to_np(ys)) < 2e-3, name


@FORMS
def test_shared_x_mixture_routes_fill_all_groups(monkeypatch, form):
    """Two route entries x rank 16 x 3 modules = 6 rank groups (the 8-group kernels); one sample
    has a single entry (its second group is empty)."""
    monkeypatch.setenv("LITHE_SHARED_X_STACKED", form)
    ads, bank = _bank()
    slot = torch.tensor([[0, 2], [4, -1], [1, 3]], dtype=torch.int32, device="cuda")
    w = torch.tensor([[0.7, 0.3], [1.0, 0.0], [0.5, 0.5]], device="cuda").sqrt().contiguous()
    gen = torch.Generator(device="cuda").manual_seed(5)
    x = torch.randn(3, 50, 3072, device="cuda", generator=gen).bfloat16()
    pools = (bank.pool_a.bfloat16(), bank.pool_b.bfloat16())
    lut_a = _hip.lut_from_pools(pools[0], x.dtype)
    lut_b = _hip.lut_from_pools(pools[1], x.dtype)
    names = ["q", "k", "v"]
    fs = [_delta.indexed_factors(_delta.packed_source(bank.words, 3, bank.layout.module(n)[3]),
                                 _delta.packed_source(bank.words, 3, bank.layout.module(n)[4]), lut_a, lut_b)
          for n in names]
    route = _delta.routes(slot, weight_sqrt=w)
    ws = shared_workspace("cuda", workspace_bytes(tuple(x.shape), 3072, 16, 2 * 3, torch.bfloat16))
    ys = [torch.zeros(3, 50, 3072, dtype=torch.bfloat16, device="cuda") for _ in names]
    PreparedSharedX(x, ys, fs, route, 16, [1.0] * 3, ws, accumulate=True)()
    sep = [torch.zeros_like(ys[0]) for _ in names]
    for f, y in zip(fs, sep):
        _delta.lora_delta(x, y, rank=16, factors=f, route=route, accumulate=True, out_scale=1.0)
    torch.cuda.synchronize()
    for i in range(3):
        assert rel(to_np(ys[i]), to_np(sep[i])) < 2e-3, i
        assert to_np(ys[i]).std() > 0


def test_shared_x_rejects_different_a_sources():
    _, bank = _bank(n=2)
    other = bank.words.clone()
    x = torch.zeros(2, 16, 3072, dtype=torch.bfloat16, device="cuda")
    ys = [torch.zeros(2, 16, 3072, dtype=torch.bfloat16, device="cuda") for _ in range(2)]
    lut = _hip.lut_from_pools(bank.pool_a.bfloat16(), x.dtype)
    lutb = _hip.lut_from_pools(bank.pool_b.bfloat16(), x.dtype)
    q, k = bank.layout.module("q"), bank.layout.module("k")
    fs = [_delta.indexed_factors(_delta.packed_source(bank.words, 3, q[3]), _delta.packed_source(bank.words, 3, q[4]),
                                 lut, lutb),
          _delta.indexed_factors(_delta.packed_source(other, 3, k[3]), _delta.packed_source(other, 3, k[4]),
                                 lut, lutb)]
    slots = torch.zeros(2, 1, dtype=torch.int32, device="cuda")
    ws = shared_workspace("cuda", workspace_bytes(tuple(x.shape), 3072, 16, 2, torch.bfloat16))
    call = PreparedSharedX(x, ys, fs, _delta.routes(slots), 16, [1.0, 1.0], ws)
    with pytest.raises(ValueError):
        call()
