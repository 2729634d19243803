"""GPU parity of the delta's launch plans and output paths that the serving shapes reach only at
sizes too large for the oracle, on small shapes with the plan forced through the plan overrides
(LITHE_SHRINK_KS, LITHE_SHRINK_TW, LITHE_EXPAND_BO, LITHE_EXPAND_WO, LITHE_EXPAND_SUBS; the library reads
them on every call):

* the shrink with each token group's K range on 1, 2 or 4 waves (one rank group): 2 waves is the
  plan of the 12288 -> 3072 projections at 1,536 and 4,096 tokens. Results differ only in the fp32
  grouping of the K sum, so each is checked against the oracle;
* the expand with 128- and 256-output waves, 1, 2 or 4 waves along the outputs of a workgroup and
  1 or 2 sub-tiles: the same sums in the same order, so the outputs are bit-identical to each other;
  the same at ranks 32, 64 and 128 (rank groups summed per factor block) over 1 / 2 waves and
  1 / 2 / 4 / 8 sub-tiles;
* the shrink with one or two 16-token groups per wave at 2, 3, 4 and 8 rank groups: bit-identical
  at each K split;
* d_out not a multiple of 8 (the per-element y path), bf16 and fp32 y;
* a bf16 y that is not 16-byte aligned (the per-element path at d_out = 3072): bit-identical to
  the same call into an aligned y.

Tolerance as in tests/test_gpu_delta.py: rel-Frobenius < 2e-3 against the oracle in bf16.
"""
import numpy as np
import pytest
import torch

from lithe_amd.kernels import PackedBank, packed_lora_delta, workspace_errors
from oracle import codebook as ocb
from oracle import delta as odelta

from helpers import random_adapter, rel

pytestmark = pytest.mark.gpu
RANK = 16
REL_BF16 = 2e-3
MODS = [("down", 12288, 3072), ("odd", 256, 100), ("q", 3072, 3072), ("mid", 512, 640)]


@pytest.fixture(scope="module")
def bank():
    ads = [random_adapter(MODS, rank=RANK, seed=500 + s) for s in range(4)]
    bank, words = PackedBank.from_adapters(ads, "cuda")
    for w in words:
        bank.add(w)
    return ads, bank, (bank.pool_a.bfloat16(), bank.pool_b.bfloat16())


def _delta(bank, pools, name, x, assign, scale, out=None, accumulate=False, out_dtype=None):
    _, _, sb, a_off, b_off = bank.layout.module(name)
    return packed_lora_delta(x, bank.words, a_off, b_off, 3, pools, assign, RANK, sb[0], scale, out=out,
                             accumulate=accumulate, out_dtype=out_dtype)


def _oracle(ads, name, x, assign, d_out, scale, out_dtype="bf16"):
    ia = np.stack([a.indices[name]["A"] for a in ads]).astype(np.int64)
    ib = np.stack([a.indices[name]["B"] for a in ads]).astype(np.int64)
    opa, opb = ocb.twin_pools()
    return odelta.shared_delta(x.float().cpu().numpy(), ia, opa, ib, opb, assign.tolist(), RANK, d_out, scale,
                               "bf16", out_dtype)


@pytest.mark.parametrize("ks", [1, 2, 4])
def test_shrink_k_split(bank, monkeypatch, ks):
    ads, bk, pools = bank
    monkeypatch.setenv("LITHE_SHRINK_KS", str(ks))
    g = torch.Generator(device="cuda").manual_seed(ks)
    x = torch.randn(3, 100, 12288, device="cuda", generator=g).bfloat16()      # partial last token tile
    assign = torch.tensor([2, 0, 3], dtype=torch.int32, device="cuda")
    d = _delta(bk, pools, "down", x, assign, 0.75)
    err = rel(d.float().cpu().numpy(), _oracle(ads, "down", x, assign, 3072, 0.75))
    print(f"ks={ks}: rel vs oracle {err:.2e}")
    assert err < REL_BF16
    assert workspace_errors() == 0


@pytest.mark.parametrize("name,d_in,d_out", [("q", 3072, 3072), ("down", 12288, 3072), ("mid", 512, 640)])
def test_expand_tiles_bit_identical(bank, monkeypatch, name, d_in, d_out):
    """Every expand tile (128 / 256 outputs per wave, 1 / 2 / 4 waves along the outputs, 1 / 2
    sub-tiles) computes the same sums in the same order: bit-identical outputs, in accumulate and
    write mode; an empty route writes zeros. d_out = 640 leaves the last workgroup's outer waves
    past the end of the row."""
    ads, bk, pools = bank
    g = torch.Generator(device="cuda").manual_seed(7)
    x = torch.randn(4, 200, d_in, device="cuda", generator=g).bfloat16()
    y0 = torch.randn(4, 200, d_out, device="cuda", generator=g).bfloat16()
    assign = torch.tensor([1, 3, 0, 1], dtype=torch.int32, device="cuda")
    assign_empty = torch.tensor([1, -1, 0, 3], dtype=torch.int32, device="cuda")
    outs, writes = [], []
    for bo in (128, 256):
        for wo in (1, 2, 4):
            for subs in (1, 2):
                monkeypatch.setenv("LITHE_EXPAND_BO", str(bo))
                monkeypatch.setenv("LITHE_EXPAND_WO", str(wo))
                monkeypatch.setenv("LITHE_EXPAND_SUBS", str(subs))
                y = y0.clone()
                _delta(bk, pools, name, x, assign, 1.0, out=y, accumulate=True)
                outs.append(y)
                writes.append(_delta(bk, pools, name, x, assign_empty, 1.0))
    for y in outs[1:]:
        assert torch.equal(y, outs[0])
    for w in writes[1:]:
        assert torch.equal(w, writes[0])
    assert not writes[0][1].any()
    assert workspace_errors() == 0
    want = odelta.index_linear(y0.float().cpu().numpy(), _oracle(ads, name, x, assign, d_out, 1.0), "bf16")
    assert rel(outs[0].float().cpu().numpy() - y0.float().cpu().numpy(), want - y0.float().cpu().numpy()) < 1e-2


@pytest.mark.parametrize("rank", [32, 64, 128])
def test_rank_collapse_tiles_bit_identical(monkeypatch, rank):
    """Rank 32 / 64 / 128 (the expand sums the mid values of 2 / 4 / 4 rank groups per factor
    block): 1 or 2 waves along the outputs and 1, 2, 4 or 8 sub-tiles compute the same sums in the
    same order, bit-identical; the result matches the oracle."""
    mods = [("mid", 512, 640), ("odd", 256, 100)]
    ads = [random_adapter(mods, rank=rank, seed=520 + s) for s in range(3)]
    bk, words = PackedBank.from_adapters(ads, "cuda")
    for w in words:
        bk.add(w)
    pools = (bk.pool_a.bfloat16(), bk.pool_b.bfloat16())
    g = torch.Generator(device="cuda").manual_seed(rank)
    for name, d_in, d_out in mods:
        _, _, sb, a_off, b_off = bk.layout.module(name)
        x = torch.randn(3, 150, d_in, device="cuda", generator=g).bfloat16()
        y0 = torch.randn(3, 150, d_out, device="cuda", generator=g).bfloat16()
        assign = torch.tensor([2, 0, 1], dtype=torch.int32, device="cuda")
        outs = []
        for wo in (1, 2):
            for subs in (1, 2, 4, 8):
                monkeypatch.setenv("LITHE_EXPAND_WO", str(wo))
                monkeypatch.setenv("LITHE_EXPAND_SUBS", str(subs))
                y = y0.clone()
                packed_lora_delta(x, bk.words, a_off, b_off, 3, pools, assign, rank, sb[0], 0.5, out=y,
                                  accumulate=True)
                outs.append(y)
        for y in outs[1:]:
            assert torch.equal(y, outs[0]), name
        assert workspace_errors() == 0
        ia = np.stack([a.indices[name]["A"] for a in ads]).astype(np.int64)
        ib = np.stack([a.indices[name]["B"] for a in ads]).astype(np.int64)
        opa, opb = ocb.twin_pools()
        want = odelta.shared_delta(x.float().cpu().numpy(), ia, opa, ib, opb, assign.tolist(), rank, d_out, 0.5,
                                   "bf16", "bf16")
        y0n = y0.float().cpu().numpy()
        want = odelta.index_linear(y0n, want, "bf16")
        assert rel(outs[0].float().cpu().numpy() - y0n, want - y0n) < 1e-2, name


@pytest.mark.parametrize("rank", [32, 48, 64, 128])
def test_shrink_two_token_groups_per_wave(monkeypatch, rank):
    """With several rank groups each shrink wave takes two 16-token groups (LITHE_SHRINK_TW=2, the
    default there): per token group the same MFMAs in the same order as one group per wave, so the
    outputs are bit-identical at a given K split (1, 2 and 4 waves per token group), including a
    ragged last tile (seq 150 and 7) and ranks of 2, 3, 4 and 8 rank groups."""
    mods = [("mid", 512, 640), ("long", 1536, 256)]
    ads = [random_adapter(mods, rank=rank, seed=540 + s) for s in range(3)]
    bk, words = PackedBank.from_adapters(ads, "cuda")
    for w in words:
        bk.add(w)
    pools = (bk.pool_a.bfloat16(), bk.pool_b.bfloat16())
    g = torch.Generator(device="cuda").manual_seed(rank + 1)
    for name, d_in, d_out in mods:
        _, _, sb, a_off, b_off = bk.layout.module(name)
        for seq in (150, 7):
            x = torch.randn(3, seq, d_in, device="cuda", generator=g).bfloat16()
            assign = torch.tensor([1, 2, 0], dtype=torch.int32, device="cuda")
            for ks in (1, 2, 4):
                outs = []
                for tw in (1, 2):
                    monkeypatch.setenv("LITHE_SHRINK_KS", str(ks))
                    monkeypatch.setenv("LITHE_SHRINK_TW", str(tw))
                    outs.append(packed_lora_delta(x, bk.words, a_off, b_off, 3, pools, assign, rank, sb[0], 0.5,
                                                  out_dtype=torch.float32))
                assert torch.equal(outs[0], outs[1]), (name, seq, ks)
            assert workspace_errors() == 0
            ia = np.stack([a.indices[name]["A"] for a in ads]).astype(np.int64)
            ib = np.stack([a.indices[name]["B"] for a in ads]).astype(np.int64)
            opa, opb = ocb.twin_pools()
            want = odelta.shared_delta(x.float().cpu().numpy(), ia, opa, ib, opb, assign.tolist(), rank, d_out,
                                       0.5, "bf16", "fp32")
            assert rel(outs[1].cpu().numpy(), want) < REL_BF16, (name, seq)


@pytest.mark.parametrize("out_dtype", [torch.bfloat16, torch.float32])
def test_d_out_not_multiple_of_8(bank, out_dtype):
    ads, bk, pools = bank
    g = torch.Generator(device="cuda").manual_seed(3)
    x = torch.randn(4, 70, 256, device="cuda", generator=g).bfloat16()
    assign = torch.tensor([3, 1, 2, 0], dtype=torch.int32, device="cuda")
    od = "bf16" if out_dtype == torch.bfloat16 else "fp32"
    d = _delta(bk, pools, "odd", x, assign, 1.5, out_dtype=out_dtype)
    assert d.shape == (4, 70, 100) and d.dtype == out_dtype
    want = _oracle(ads, "odd", x, assign, 100, 1.5, od)
    assert rel(d.float().cpu().numpy(), want) < REL_BF16
    y0 = torch.randn(4, 70, 100, device="cuda", generator=g).to(out_dtype)
    y = y0.clone()
    _delta(bk, pools, "odd", x, assign, 1.5, out=y, accumulate=True)
    if out_dtype == torch.bfloat16:
        assert torch.equal(y, (y0.float() + d.float()).bfloat16())
    else:
        assert torch.equal(y, y0 + d)


def test_unaligned_y_matches_aligned(bank):
    ads, bk, pools = bank
    g = torch.Generator(device="cuda").manual_seed(4)
    x = torch.randn(2, 130, 3072, device="cuda", generator=g).bfloat16()
    y0 = torch.randn(2, 130, 3072, device="cuda", generator=g).bfloat16()
    assign = torch.tensor([0, 2], dtype=torch.int32, device="cuda")
    n = y0.numel()
    buf = torch.empty(n + 8, dtype=torch.bfloat16, device="cuda")
    y_un = buf[1:1 + n].view(2, 130, 3072)                  # 2 bytes past a 16-byte boundary
    assert y_un.data_ptr() % 16 == 2 and y_un.is_contiguous()
    for acc in (False, True):
        y_al = y0.clone()
        y_un.copy_(y0)
        _delta(bk, pools, "q", x, assign, 0.5, out=y_al, accumulate=acc)
        _delta(bk, pools, "q", x, assign, 0.5, out=y_un, accumulate=acc)
        assert torch.equal(y_un, y_al), acc
