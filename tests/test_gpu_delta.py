"""GPU parity of the fused index-resident delta (shrink + expand) against the oracle.

Tolerances (stated here, used below):
* bf16: the kernel rounds at the reference's points (y_lo to bf16, delta to bf16,
  ``* scaling``, ``out + delta``); only the fp32 accumulation order differs from
  the oracle, which evaluates the products in float64. Required: rel-Frobenius
  error vs the oracle < 2e-3, and vs the unrounded float64 truth < 2e-2 (the
  reference's own bound, tests/test_kernels.py:216 of the reference).
* fp32: rtol 1e-5, atol 1e-5 against the float64-evaluated oracle.
"""
import numpy as np
import pytest
import torch

import lithe_amd
from lithe_amd.kernels import IndexLoRALinear, PackedBank, packed_lora_delta, shared_codebook_lora_delta
from oracle import codebook as ocb
from oracle import decode as odec
from oracle import delta as odelta

from helpers import random_adapter, rel, to_np, ulp_stats

pytestmark = pytest.mark.gpu

REL_BF16 = 2e-3
REL_TRUTH = 2e-2


def _stack(ads, name, side, dtype=np.int32):
    return np.stack([a.indices[name][side].astype(dtype) for a in ads])


def _truth(x, ia, ib, assign, R, d_in, d_out):
    pa, pb = ocb.twin_pools()
    out = []
    for i, j in enumerate(assign):
        a = odec.decode(ia[j], (R, d_in), pa)
        b = odec.decode(ib[j], (d_out, R), pb)
        out.append(odelta.truth_delta(x[i], a, b))
    return np.stack(out)


@pytest.mark.parametrize("seq,d_in,d_out,r", [(256, 3072, 3072, 16), (50, 128, 192, 16), (1, 256, 384, 4),
                                              (77, 512, 640, 8), (130, 12288, 256, 16), (64, 512, 640, 64),
                                              (33, 256, 100, 32), (20, 128, 200, 128), (50, 384, 264, 96)])
def test_shared_delta_matches_oracle(seq, d_in, d_out, r):
    ads = [random_adapter([("l", d_in, d_out)], rank=r, seed=s) for s in range(3)]
    ia, ib = _stack(ads, "l", "A"), _stack(ads, "l", "B")
    g = torch.Generator().manual_seed(seq)
    x = (torch.randn(4, seq, d_in, generator=g) * 0.5).bfloat16()
    assign = [2, 0, 1, 2]
    pa, pb = (p.cuda() for p in lithe_amd.twin_pools())
    got = shared_codebook_lora_delta(x.cuda(), torch.from_numpy(ia).cuda(), pa, torch.from_numpy(ib).cuda(), pb,
                                     torch.tensor(assign, device="cuda", dtype=torch.int32), r, d_out, 1.0)
    assert got.dtype == torch.bfloat16 and got.shape == (4, seq, d_out)
    want = odelta.shared_delta(to_np(x), ia, ocb.twin_pools()[0], ib, ocb.twin_pools()[1], assign, r, d_out,
                               1.0, "bf16")
    g_np = to_np(got)
    err, err_t = rel(g_np, want), rel(g_np, _truth(to_np(x), ia, ib, assign, r, d_in, d_out))
    print(f"shared seq={seq} d_in={d_in} d_out={d_out} r={r}: rel vs oracle {err:.2e}, vs truth {err_t:.2e}, "
          f"ulp/mismatch {ulp_stats(g_np, want)}")
    assert err < REL_BF16 and err_t < REL_TRUTH


def test_shared_delta_scaling_and_fp32_out():
    ads = [random_adapter([("l", 256, 384)], rank=16, seed=s) for s in range(2)]
    ia, ib = _stack(ads, "l", "A"), _stack(ads, "l", "B")
    x = (torch.randn(3, 40, 256, generator=torch.Generator().manual_seed(1))).bfloat16()
    assign = [1, 0, 1]
    pa, pb = (p.cuda() for p in lithe_amd.twin_pools())
    args = (x.cuda(), torch.from_numpy(ia).cuda(), pa, torch.from_numpy(ib).cuda(), pb,
            torch.tensor(assign, device="cuda"), 16, 384)
    opa, opb = ocb.twin_pools()
    for scaling, out_dtype, od in ((0.5, None, "bf16"), (0.3, torch.float32, "fp32"), (2.0, torch.float32, "fp32")):
        got = shared_codebook_lora_delta(*args, scaling, out_dtype=out_dtype)
        want = odelta.shared_delta(to_np(x), ia, opa, ib, opb, assign, 16, 384, scaling, "bf16", od)
        assert rel(to_np(got), want) < REL_BF16, (scaling, out_dtype)


@pytest.mark.parametrize("r,d_out", [(32, 264), (64, 640), (128, 200), (96, 100)])
def test_rank_collapse_matches_per_group_sums(monkeypatch, r, d_out):
    """Ranks that are multiples of 32 sum the mid values of the rank groups sharing a factor block
    before the expand's MFMA (the hi / lo bf16 split of the sum); LITHE_EXPAND_NS=1 runs one MFMA
    per rank group instead. fp32 outputs (no final rounding) agree to 2e-5 relative (fp32
    accumulation order and the 2^-17 split bound), and both match the oracle."""
    ads = [random_adapter([("l", 256, d_out)], rank=r, seed=40 + s) for s in range(3)]
    ia, ib = _stack(ads, "l", "A"), _stack(ads, "l", "B")
    x = (torch.randn(3, 45, 256, generator=torch.Generator().manual_seed(r)) * 0.5).bfloat16()
    assign = [2, 1, 0]
    pa, pb = (p.cuda() for p in lithe_amd.twin_pools())
    args = (x.cuda(), torch.from_numpy(ia).cuda(), pa, torch.from_numpy(ib).cuda(), pb,
            torch.tensor(assign, device="cuda", dtype=torch.int32), r, d_out, 0.5)
    got = shared_codebook_lora_delta(*args, out_dtype=torch.float32)
    monkeypatch.setenv("LITHE_EXPAND_NS", "1")
    ref = shared_codebook_lora_delta(*args, out_dtype=torch.float32)
    err = rel(to_np(got), to_np(ref))
    opa, opb = ocb.twin_pools()
    want = odelta.shared_delta(to_np(x), ia, opa, ib, opb, assign, r, d_out, 0.5, "bf16", "fp32")
    err_o = rel(to_np(got), want)
    print(f"rank {r} d_out {d_out}: collapsed vs per-group {err:.2e}, vs oracle {err_o:.2e}")
    assert err < 2e-5 and err_o < REL_BF16


def test_shared_delta_fp32_activations():
    ads = [random_adapter([("l", 3072, 3072)], rank=16, seed=s) for s in range(4)]
    ia, ib = _stack(ads, "l", "A"), _stack(ads, "l", "B")
    x = torch.randn(4, 64, 3072, generator=torch.Generator().manual_seed(2))
    assign = [0, 1, 2, 3]
    pa, pb = (p.cuda() for p in lithe_amd.twin_pools())
    got = shared_codebook_lora_delta(x.cuda(), torch.from_numpy(ia).cuda(), pa, torch.from_numpy(ib).cuda(), pb,
                                     torch.tensor(assign, device="cuda"), 16, 3072, 1.0)
    opa, opb = ocb.twin_pools()
    want = odelta.shared_delta(x.numpy(), ia, opa, ib, opb, assign, 16, 3072, 1.0, "fp32")
    np.testing.assert_allclose(to_np(got), want, rtol=1e-5, atol=1e-5)


@pytest.mark.parametrize("shape", [(3, 64, 256), (3, 256)])
def test_index_layer_matches_oracle(shape):
    ads = [random_adapter([("l", 256, 384)], rank=16, seed=s) for s in range(2)]
    ia, ib = _stack(ads, "l", "A"), _stack(ads, "l", "B")
    torch.manual_seed(0)
    base = torch.nn.Linear(256, 384).cuda().bfloat16()
    pa, pb = (p.cuda() for p in lithe_amd.twin_pools())
    layer = IndexLoRALinear(base, torch.from_numpy(ia).cuda(), torch.from_numpy(ib).cuda(), pa.bfloat16(),
                            pb.bfloat16(), 16, 1.0)
    layer.assign = torch.tensor([1, 0, 1], device="cuda", dtype=torch.int32)
    x = torch.randn(*shape, generator=torch.Generator().manual_seed(5)).bfloat16()
    with torch.no_grad():
        base_out = to_np(base(x.cuda()))
        got = to_np(layer(x.cuda()))
    x3 = to_np(x).reshape(3, -1, 256)
    opa, opb = ocb.twin_pools()
    delta = odelta.shared_delta(x3, ia, opa, ib, opb, [1, 0, 1], 16, 384, 1.0, "bf16")
    want = odelta.index_linear(base_out.reshape(3, -1, 384), delta, "bf16").reshape(got.shape)
    assert rel(got, want) < REL_BF16
    layer.assign = None      # default: slot 0 for every sample
    with torch.no_grad():
        got0 = to_np(layer(x.cuda()))
    delta0 = odelta.shared_delta(x3, ia, opa, ib, opb, [0, 0, 0], 16, 384, 1.0, "bf16")
    assert rel(got0, odelta.index_linear(base_out.reshape(3, -1, 384), delta0, "bf16").reshape(got.shape)) < REL_BF16


def test_packed_bank_delta_accumulates_into_base_output():
    """North-star path: factors read straight from the 9-bit packed bank, delta added into y."""
    mods = [("q", 3072, 3072), ("up", 3072, 12288), ("down", 12288, 3072)]
    ads = [random_adapter(mods, rank=16, seed=20 + s) for s in range(6)]
    bank, words = PackedBank.from_adapters(ads, "cuda")
    for w in words:
        bank.add(w)
    assign = [5, 2, 0]
    seq = 96
    opa, opb = ocb.twin_pools()
    for name, d_in, d_out in mods:
        _, sa, sb, a_off, b_off = bank.layout.module(name)
        x = torch.randn(3, seq, d_in, generator=torch.Generator().manual_seed(d_out)).bfloat16()
        y0 = torch.randn(3, seq, d_out, generator=torch.Generator().manual_seed(d_in)).bfloat16()
        y = y0.cuda()
        pools = (bank.pool_a.bfloat16(), bank.pool_b.bfloat16())
        packed_lora_delta(x.cuda(), bank.words, a_off, b_off, 3, pools, torch.tensor(assign, device="cuda"),
                          16, d_out, 1.0, out=y, accumulate=True)
        ia = _stack(ads, name, "A")
        ib = _stack(ads, name, "B")
        delta = odelta.shared_delta(to_np(x), ia, opa, ib, opb, assign, 16, d_out, 1.0, "bf16")
        want = odelta.index_linear(to_np(y0), delta, "bf16")
        got = to_np(y)
        print(f"packed {name}: rel {rel(got, want):.2e} ulp/mismatch {ulp_stats(got, want)}")
        assert rel(got, want) < REL_BF16
        assert rel(got - to_np(y0), want - to_np(y0)) < 2e-2


def test_bank_backed_index_layer():
    mods = [("l", 256, 384)]
    ads = [random_adapter(mods, rank=16, seed=s) for s in range(3)]
    bank, words = PackedBank.from_adapters(ads, "cuda")
    for w in words:
        bank.add(w)
    torch.manual_seed(1)
    base = torch.nn.Linear(256, 384).cuda().bfloat16()
    layer = IndexLoRALinear.from_bank(base, bank, "l")
    layer.assign = torch.tensor([2, 1], device="cuda")
    x = torch.randn(2, 33, 256, generator=torch.Generator().manual_seed(3)).bfloat16()
    with torch.no_grad():
        base_out = to_np(base(x.cuda()))
        got = to_np(layer(x.cuda()))
    opa, opb = ocb.twin_pools()
    delta = odelta.shared_delta(to_np(x), _stack(ads, "l", "A"), opa, _stack(ads, "l", "B"), opb, [2, 1], 16, 384,
                                1.0, "bf16")
    assert rel(got, odelta.index_linear(base_out, delta, "bf16")) < REL_BF16


def test_bank_backed_layer_sees_slots_added_after_a_call():
    """A slot added to the bank within its capacity (same storage, one more slot) after the layer
    ran is routable by the next call: the layer's kept call descriptors follow the slot count."""
    mods = [("l", 256, 384)]
    ads = [random_adapter(mods, rank=16, seed=40 + s) for s in range(3)]
    bank, words = PackedBank.from_adapters(ads, "cuda")       # capacity 3
    bank.add(words[0])
    bank.add(words[1])
    base = torch.nn.Linear(256, 384).cuda().bfloat16()
    layer = IndexLoRALinear.from_bank(base, bank, "l")
    x = torch.randn(2, 40, 256, generator=torch.Generator().manual_seed(4)).bfloat16().cuda()
    opa, opb = ocb.twin_pools()
    ia, ib = _stack(ads, "l", "A"), _stack(ads, "l", "B")
    lithe_amd.kernels.workspace_errors()                       # clears what earlier calls left
    with torch.no_grad():
        base_out = to_np(base(x))
        layer.assign = torch.tensor([1, 0], device="cuda")
        first = to_np(layer(x))
        ptr = bank.words.data_ptr()
        bank.add(words[2])
        assert bank.words.data_ptr() == ptr and bank.num_slots == 3
        layer.assign = torch.tensor([2, 1], device="cuda")
        second = to_np(layer(x))
    assert lithe_amd.kernels.workspace_errors() == 0
    for got, assign in ((first, [1, 0]), (second, [2, 1])):
        delta = odelta.shared_delta(to_np(x), ia, opa, ib, opb, assign, 16, 384, 1.0, "bf16")
        assert rel(got, odelta.index_linear(base_out, delta, "bf16")) < REL_BF16, assign
