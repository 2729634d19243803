"""GPU parity of lithe_lora_delta_grouped: independent modules of one batch in one shrink launch and
one expand launch, modules given the same x sharing its shrink.

* With the shrink's K split forced to one value (LITHE_SHRINK_KS), a grouped call and the
  per-module lithe_lora_delta calls compute the same sums in the same order: bit-identical
  outputs (the expand's tile width and sub-tiles change no sum). Checked on a FLUX double-block
  projection stage (image q / k / v sharing one x, text q / k / v sharing another), a stage of
  different widths, write and accumulate mode, and a two-entry mixture route.
* Without forcing, against the oracle within the bf16 tolerance of tests/test_gpu_delta.py.
* The job-by-job form (LITHE_GROUPED_SERIAL: the per-call kernels, one launch per job) equals the
  grouped launch bit for bit.
* Both shrink forms of modules that share an input (LITHE_SHARED_X_STACKED: the modules as rank
  groups of one workgroup, or one workgroup per tile and module), forced, against the oracle and
  the per-module calls.
* Modules without tokens are skipped; a group at the real FLUX shapes (B = 14, 4,096 image and
  512 text tokens) equals the per-module calls bit for bit.
* Rank 32 and 64 (2 and 4 rank groups), a three-entry mixture (three groups), the largest call
  (8 modules) and fp32 activations (no grouped kernel: job by job) equal the per-module calls.
"""
import numpy as np
import pytest
import torch

from lithe_amd.kernels import PackedBank, _delta, _hip, packed_lora_delta, workspace_errors
from lithe_amd.kernels.prepared import PreparedGroup, prepare_packed_group, shared_workspace
from oracle import codebook as ocb
from oracle import delta as odelta

from helpers import random_adapter, rel

pytestmark = pytest.mark.gpu
RANK = 16
MODS = [("q", 256, 256), ("k", 256, 256), ("v", 256, 256), ("aq", 256, 256), ("ak", 256, 256), ("av", 256, 256),
        ("up", 256, 1024), ("down", 1024, 256), ("mid", 512, 640)]


@pytest.fixture(scope="module")
def bank():
    ads = [random_adapter(MODS, rank=RANK, seed=700 + s) for s in range(5)]
    bank, words = PackedBank.from_adapters(ads, "cuda")
    for w in words:
        bank.add(w)
    return ads, bank, (bank.pool_a.bfloat16(), bank.pool_b.bfloat16())


def _inputs(spec, g, n_batch=3):
    """spec: [(name, x key, seq)] -> xs (one tensor per key), ys."""
    shape = {n: (di, do) for n, di, do in MODS}
    xs_by_key, xs, ys = {}, [], []
    for name, key, seq in spec:
        di, do = shape[name]
        if key not in xs_by_key:
            xs_by_key[key] = torch.randn(n_batch, seq, di, device="cuda", generator=g).bfloat16()
        xs.append(xs_by_key[key])
        ys.append(torch.randn(n_batch, seq, do, device="cuda", generator=g).bfloat16())
    return xs, ys


def _grouped(bk, pools, spec, xs, ys, slots, accumulate=True, scale=0.75, weights=None):
    offs = [bk.layout.module(n)[3:5] for n, _, _ in spec]
    ws = shared_workspace("cuda", 64 << 20)
    if weights is None:
        call = prepare_packed_group(xs, ys, bk.words, offs, 3, pools, slots, RANK, scale, ws, accumulate)
    else:
        lut_a = _hip.lut_from_pools(pools[0], torch.bfloat16)
        lut_b = _hip.lut_from_pools(pools[1], torch.bfloat16)
        f = _delta.indexed_factors(_delta.packed_source(bk.words, 3, 0), _delta.packed_source(bk.words, 3, 0),
                                   lut_a, lut_b)
        call = PreparedGroup(xs, ys, f, offs, _delta.routes(slots, weights), RANK, [scale] * len(xs), ws, accumulate,
                             keep=(slots, weights))
    call()
    torch.cuda.synchronize()
    return ys


def _separate(bk, pools, spec, xs, ys, slots, accumulate=True, scale=0.75):
    for (name, _, _), x, y in zip(spec, xs, ys):
        _, _, sb, a_off, b_off = bk.layout.module(name)
        if accumulate:
            packed_lora_delta(x, bk.words, a_off, b_off, 3, pools, slots, RANK, sb[0], scale, out=y, accumulate=True)
        else:
            packed_lora_delta(x, bk.words, a_off, b_off, 3, pools, slots, RANK, sb[0], scale, out=y)
    torch.cuda.synchronize()
    return ys


STAGE_PROJ = [("q", "img", 300), ("k", "img", 300), ("v", "img", 300), ("aq", "txt", 70), ("ak", "txt", 70),
              ("av", "txt", 70)]
STAGE_FF = [("up", "a", 200), ("down", "b", 90), ("q", "c", 33)]


@pytest.mark.parametrize("spec", [STAGE_PROJ, STAGE_FF], ids=["proj", "ff"])
@pytest.mark.parametrize("ks", [1, 2])
@pytest.mark.parametrize("accumulate", [True, False])
def test_grouped_equals_per_module_calls(bank, monkeypatch, spec, ks, accumulate):
    _, bk, pools = bank
    monkeypatch.setenv("LITHE_SHRINK_KS", str(ks))
    monkeypatch.setenv("LITHE_SHARED_X_STACKED", "0")
    g = torch.Generator(device="cuda").manual_seed(ks)
    xs, ys = _inputs(spec, g)
    slots = torch.tensor([3, 0, 4], dtype=torch.int32, device="cuda")
    want = _separate(bk, pools, spec, xs, [y.clone() for y in ys], slots, accumulate)
    got = _grouped(bk, pools, spec, xs, [y.clone() for y in ys], slots, accumulate)
    for (name, _, _), w, o in zip(spec, want, got):
        assert torch.equal(o, w), name
    assert workspace_errors() == 0


@pytest.mark.parametrize("form", [None, "1", "0"], ids=["auto", "stacked", "replicated"])
def test_grouped_matches_oracle_and_serial_form(bank, monkeypatch, form):
    if form is not None:
        monkeypatch.setenv("LITHE_SHARED_X_STACKED", form)
    ads, bk, pools = bank
    g = torch.Generator(device="cuda").manual_seed(11)
    spec = STAGE_PROJ + [("up", "u", 64)]
    xs, ys = _inputs(spec, g)
    slots = torch.tensor([1, 4, 2], dtype=torch.int32, device="cuda")
    got = _grouped(bk, pools, spec, xs, [y.clone() for y in ys], slots, accumulate=False)
    opa, opb = ocb.twin_pools()
    for (name, _, _), x, o in zip(spec, xs, got):
        ia = np.stack([a.indices[name]["A"] for a in ads]).astype(np.int64)
        ib = np.stack([a.indices[name]["B"] for a in ads]).astype(np.int64)
        want = odelta.shared_delta(x.float().cpu().numpy(), ia, opa, ib, opb, slots.tolist(), RANK, o.shape[2], 0.75)
        assert rel(o.float().cpu().numpy(), want) < 2e-3, name
    monkeypatch.setenv("LITHE_GROUPED_SERIAL", "1")
    serial = _grouped(bk, pools, spec, xs, [y.clone() for y in ys], slots, accumulate=False)
    for (name, _, _), s, o in zip(spec, serial, got):
        assert torch.equal(s, o), name


@pytest.mark.parametrize("accumulate", [True, False])
def test_grouped_stacked_shared_inputs_equal_per_module_calls(bank, monkeypatch, accumulate):
    """Stacked shared-input shrink with whole-K waves (two token groups per wave, the modules'
    A rows as rank groups): each rank group's MFMA sequence is the per-module call's."""
    _, bk, pools = bank
    monkeypatch.setenv("LITHE_SHRINK_KS", "1")
    monkeypatch.setenv("LITHE_SHARED_X_STACKED", "1")
    g = torch.Generator(device="cuda").manual_seed(21)
    xs, ys = _inputs(STAGE_PROJ, g)
    slots = torch.tensor([2, -1, 4], dtype=torch.int32, device="cuda")
    want = _separate(bk, pools, STAGE_PROJ, xs, [y.clone() for y in ys], slots, accumulate)
    got = _grouped(bk, pools, STAGE_PROJ, xs, [y.clone() for y in ys], slots, accumulate)
    for (name, _, _), w, o in zip(STAGE_PROJ, want, got):
        assert torch.equal(o, w), name
    assert workspace_errors() == 0


def test_grouped_mixture_routes(bank, monkeypatch):
    _, bk, pools = bank
    monkeypatch.setenv("LITHE_SHRINK_KS", "1")
    g = torch.Generator(device="cuda").manual_seed(5)
    spec = [("q", "img", 130), ("k", "img", 130), ("aq", "txt", 40)]
    xs, ys = _inputs(spec, g)
    slots = torch.tensor([[0, 3], [2, -1], [4, 1]], dtype=torch.int32, device="cuda")
    w = torch.tensor([[0.7, 0.3], [1.0, 0.0], [0.5, 0.5]], device="cuda").sqrt().contiguous()
    got = _grouped(bk, pools, spec, xs, [y.clone() for y in ys], slots, weights=w)
    ws = torch.zeros(16 << 20, dtype=torch.uint8, device="cuda")
    lut_a = _hip.lut_from_pools(pools[0], torch.bfloat16)
    lut_b = _hip.lut_from_pools(pools[1], torch.bfloat16)
    for (name, _, _), x, y, o in zip(spec, xs, ys, got):
        _, _, _, a_off, b_off = bk.layout.module(name)
        f = _delta.indexed_factors(_delta.packed_source(bk.words, 3, a_off), _delta.packed_source(bk.words, 3, b_off),
                                   lut_a, lut_b)
        want = y.clone()
        _delta.lora_delta(x, want, rank=RANK, factors=f, route=_delta.routes(slots, w), accumulate=True,
                          out_scale=0.75)
        torch.cuda.synchronize()
        assert torch.equal(o, want), name


def test_grouped_skips_modules_without_tokens(bank):
    _, bk, pools = bank
    g = torch.Generator(device="cuda").manual_seed(6)
    spec = [("q", "a", 50), ("up", "b", 0), ("down", "c", 20)]
    xs, ys = _inputs(spec, g)
    slots = torch.tensor([1, 1, 0], dtype=torch.int32, device="cuda")
    before = [y.clone() for y in ys]
    got = _grouped(bk, pools, spec, xs, [y.clone() for y in ys], slots)
    want = _separate(bk, pools, spec, xs, [y.clone() for y in before], slots)
    assert got[1].numel() == 0
    assert rel(got[0].float().cpu().numpy() - before[0].float().cpu().numpy(),
               want[0].float().cpu().numpy() - before[0].float().cpu().numpy()) < 1e-2


def test_grouped_flux_double_block_projections_full_size(monkeypatch):
    """Image q / k / v (4,096 tokens) and text q / k / v (512 tokens) of 14 samples, 3072 wide, in
    one grouped call: bit-identical to the six per-module calls with the same K split."""
    monkeypatch.setenv("LITHE_SHRINK_KS", "1")
    names = ["q", "k", "v", "aq", "ak", "av"]
    ads = [random_adapter([(n, 3072, 3072) for n in names], rank=RANK, seed=800 + s) for s in range(14)]
    bk, words = PackedBank.from_adapters(ads, "cuda")
    for w in words:
        bk.add(w)
    pools = (bk.pool_a.bfloat16(), bk.pool_b.bfloat16())
    g = torch.Generator(device="cuda").manual_seed(9)
    ximg = torch.randn(14, 4096, 3072, device="cuda", generator=g).bfloat16()
    xtxt = torch.randn(14, 512, 3072, device="cuda", generator=g).bfloat16()
    xs = [ximg] * 3 + [xtxt] * 3
    ys = [torch.randn(14, x.shape[1], 3072, device="cuda", generator=g).bfloat16() for x in xs]
    slots = torch.randperm(14, generator=torch.Generator().manual_seed(2)).to(torch.int32).cuda()
    spec = [(n, "", x.shape[1]) for n, x in zip(names, xs)]
    offs = [bk.layout.module(n)[3:5] for n in names]
    ws = shared_workspace("cuda", 64 << 20)
    got = [y.clone() for y in ys]
    prepare_packed_group(xs, got, bk.words, offs, 3, pools, slots, RANK, 1.0, ws)()
    want = [y.clone() for y in ys]
    for n, x, y in zip(names, xs, want):
        _, _, _, a_off, b_off = bk.layout.module(n)
        packed_lora_delta(x, bk.words, a_off, b_off, 3, pools, slots, RANK, 3072, 1.0, out=y, accumulate=True)
    torch.cuda.synchronize()
    for n, o, w in zip(names, got, want):
        assert torch.equal(o, w), n
    assert workspace_errors() == 0


def _per_module_routes(bk, pools, spec, xs, ys, slots, weights, rank, scale=0.75):
    """Per-module lithe_lora_delta calls with a mixture route (the grouped call's reference)."""
    lut_a = _hip.lut_from_pools(pools[0], xs[0].dtype)
    lut_b = _hip.lut_from_pools(pools[1], xs[0].dtype)
    for (name, _, _), x, y in zip(spec, xs, ys):
        _, _, _, a_off, b_off = bk.layout.module(name)
        f = _delta.indexed_factors(_delta.packed_source(bk.words, 3, a_off), _delta.packed_source(bk.words, 3, b_off),
                                   lut_a, lut_b)
        _delta.lora_delta(x, y, rank=rank, factors=f, route=_delta.routes(slots, weights), accumulate=True,
                          out_scale=scale)
    torch.cuda.synchronize()
    return ys


@pytest.mark.parametrize("rank", [32, 64])
def test_grouped_higher_ranks(monkeypatch, rank):
    """Rank 32 and 64 (2 and 4 rank groups per module: the shrink and expand compiled for 2 and 4
    groups) in one grouped call: bit-identical to the per-module calls with the same K split."""
    monkeypatch.setenv("LITHE_SHRINK_KS", "1")
    mods = [("q", 256, 256), ("k", 256, 256), ("aq", 256, 256), ("up", 256, 1024), ("down", 1024, 256)]
    ads = [random_adapter(mods, rank=rank, seed=900 + s) for s in range(3)]
    bk, words = PackedBank.from_adapters(ads, "cuda")
    for w in words:
        bk.add(w)
    pools = (bk.pool_a.bfloat16(), bk.pool_b.bfloat16())
    g = torch.Generator(device="cuda").manual_seed(rank)
    spec = [("q", "img", 96), ("k", "img", 96), ("aq", "txt", 40), ("up", "u", 70), ("down", "d", 33)]
    shape = {n: (di, do) for n, di, do in mods}
    xs_by_key, xs, ys = {}, [], []
    for name, key, seq in spec:
        di, do = shape[name]
        if key not in xs_by_key:
            xs_by_key[key] = torch.randn(3, seq, di, device="cuda", generator=g).bfloat16()
        xs.append(xs_by_key[key])
        ys.append(torch.randn(3, seq, do, device="cuda", generator=g).bfloat16())
    slots = torch.tensor([2, 0, 1], dtype=torch.int32, device="cuda")
    offs = [bk.layout.module(n)[3:5] for n, _, _ in spec]
    got = [y.clone() for y in ys]
    prepare_packed_group(xs, got, bk.words, offs, 3, pools, slots, rank, 0.75, shared_workspace("cuda", 64 << 20))()
    want = [y.clone() for y in ys]
    for (name, _, _), x, y in zip(spec, xs, want):
        _, _, sb, a_off, b_off = bk.layout.module(name)
        packed_lora_delta(x, bk.words, a_off, b_off, 3, pools, slots, rank, sb[0], 0.75, out=y, accumulate=True)
    torch.cuda.synchronize()
    for (name, _, _), o, w in zip(spec, got, want):
        assert torch.equal(o, w), name
    assert workspace_errors() == 0


def test_grouped_three_entry_mixture(bank, monkeypatch):
    """Three route entries at rank 16: three rank groups (the shrink compiled for exactly three,
    the expand for four), one with an empty entry; bit-identical to the per-module calls."""
    _, bk, pools = bank
    monkeypatch.setenv("LITHE_SHRINK_KS", "1")
    g = torch.Generator(device="cuda").manual_seed(13)
    spec = [("q", "img", 120), ("k", "img", 120), ("aq", "txt", 50), ("down", "d", 64)]
    xs, ys = _inputs(spec, g)
    slots = torch.tensor([[0, 3, 4], [2, -1, 1], [4, 1, 0]], dtype=torch.int32, device="cuda")
    w = torch.tensor([[0.5, 0.3, 0.2], [0.6, 0.0, 0.4], [0.2, 0.2, 0.6]], device="cuda").sqrt().contiguous()
    got = _grouped(bk, pools, spec, xs, [y.clone() for y in ys], slots, weights=w)
    want = _per_module_routes(bk, pools, spec, xs, [y.clone() for y in ys], slots, w, RANK)
    for (name, _, _), o, r in zip(spec, got, want):
        assert torch.equal(o, r), name
    assert workspace_errors() == 0


def test_grouped_eight_modules(bank, monkeypatch):
    """The largest grouped call (8 modules, 8 distinct inputs of different lengths and widths)."""
    _, bk, pools = bank
    monkeypatch.setenv("LITHE_SHRINK_KS", "1")
    g = torch.Generator(device="cuda").manual_seed(17)
    spec = [(n, n, seq) for n, seq in zip(["q", "k", "v", "aq", "ak", "av", "up", "down"],
                                          [17, 64, 129, 8, 200, 1, 77, 45])]
    xs, ys = _inputs(spec, g)
    slots = torch.tensor([4, 1, 2], dtype=torch.int32, device="cuda")
    got = _grouped(bk, pools, spec, xs, [y.clone() for y in ys], slots)
    want = _separate(bk, pools, spec, xs, [y.clone() for y in ys], slots)
    for (name, _, _), o, r in zip(spec, got, want):
        assert torch.equal(o, r), name


def test_grouped_fp32_activations(bank, monkeypatch):
    """fp32 activations (no grouped kernel: the call runs its jobs one launch at a time through the
    per-call kernels): bit-identical to the per-module calls."""
    _, bk, _ = bank
    pools = (bk.pool_a.float(), bk.pool_b.float())
    monkeypatch.setenv("LITHE_SHRINK_KS", "1")
    g = torch.Generator(device="cuda").manual_seed(19)
    spec = [("q", "img", 50), ("k", "img", 50), ("up", "u", 30)]
    shape = {n: (di, do) for n, di, do in MODS}
    xs_by_key, xs, ys = {}, [], []
    for name, key, seq in spec:
        di, do = shape[name]
        if key not in xs_by_key:
            xs_by_key[key] = torch.randn(3, seq, di, device="cuda", generator=g)
        xs.append(xs_by_key[key])
        ys.append(torch.randn(3, seq, do, device="cuda", generator=g))
    slots = torch.tensor([1, 3, 0], dtype=torch.int32, device="cuda")
    got = _grouped(bk, pools, spec, xs, [y.clone() for y in ys], slots)
    want = _separate(bk, pools, spec, xs, [y.clone() for y in ys], slots)
    for (name, _, _), o, r in zip(spec, got, want):
        assert torch.equal(o, r), name


def test_grouped_partial_tiles(bank, monkeypatch):
    """Token counts that fill no tile evenly and d_out = 640 (its second 512-output workgroup has
    one wave past the end of the row), in write and accumulate mode: bit-identical to the
    per-module calls."""
    _, bk, pools = bank
    monkeypatch.setenv("LITHE_SHRINK_KS", "1")
    g = torch.Generator(device="cuda").manual_seed(23)
    spec = [("mid", "m", 37), ("q", "q", 45), ("down", "d", 3)]
    xs, ys = _inputs(spec, g)
    slots = torch.tensor([3, 2, 0], dtype=torch.int32, device="cuda")
    for acc in (True, False):
        got = _grouped(bk, pools, spec, xs, [y.clone() for y in ys], slots, accumulate=acc)
        want = _separate(bk, pools, spec, xs, [y.clone() for y in ys], slots, accumulate=acc)
        for (name, _, _), o, r in zip(spec, got, want):
            assert torch.equal(o, r), (name, acc)
    assert workspace_errors() == 0
