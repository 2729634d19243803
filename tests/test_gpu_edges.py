"""GPU edge cases of the public wrappers: empty batches and empty token dimensions (every entry
point returns a correctly shaped result and launches nothing; an accumulate leaves the base
output alone), and the largest batch the delta accepts (65,535 samples), checked against the
oracle with the tokens of each slot gathered into one sample (a token's result depends only on
its own x row and its slot's factors).
"""
import numpy as np
import pytest
import torch

import lithe_amd
from lithe_amd.kernels import (IndexLoRALinear, PackedBank, decode_packed_slots, packed_lora_delta,
                               per_sample_lora_delta, shared_codebook_lora_delta)
from oracle import codebook as ocb
from oracle import delta as odelta

from helpers import random_adapter, rel

pytestmark = pytest.mark.gpu
D_IN, D_OUT, R = 128, 192, 16


@pytest.fixture(scope="module")
def small():
    ads = [random_adapter([("l", D_IN, D_OUT)], rank=R, seed=s) for s in range(3)]
    ia = torch.from_numpy(np.stack([a.indices["l"]["A"].astype(np.int32) for a in ads])).cuda()
    ib = torch.from_numpy(np.stack([a.indices["l"]["B"].astype(np.int32) for a in ads])).cuda()
    pa, pb = (p.cuda() for p in lithe_amd.twin_pools())
    bank, words = PackedBank.from_adapters(ads, "cuda")
    for w in words:
        bank.add(w)
    return ads, ia, ib, pa, pb, bank


@pytest.mark.parametrize("bsz,seq", [(0, 5), (3, 0), (0, 0)])
def test_empty_shared_and_packed_delta(small, bsz, seq):
    _, ia, ib, pa, pb, bank = small
    x = torch.randn(bsz, seq, D_IN, device="cuda").bfloat16()
    assign = torch.zeros(bsz, dtype=torch.int32, device="cuda")
    d = shared_codebook_lora_delta(x, ia, pa, ib, pb, assign, R, D_OUT, 0.5)
    assert d.shape == (bsz, seq, D_OUT) and d.dtype == torch.bfloat16
    _, _, _, a_off, b_off = bank.layout.module("l")
    pools = (bank.pool_a.bfloat16(), bank.pool_b.bfloat16())
    d2 = packed_lora_delta(x, bank.words, a_off, b_off, 3, pools, assign, R, D_OUT, 0.5)
    assert d2.shape == (bsz, seq, D_OUT)
    y = torch.empty(bsz, seq, D_OUT, device="cuda", dtype=torch.bfloat16)
    assert packed_lora_delta(x, bank.words, a_off, b_off, 3, pools, assign, R, D_OUT, 0.5, out=y,
                             accumulate=True) is y
    sA = torch.randn(bsz, R, D_IN, device="cuda").bfloat16()
    sB = torch.randn(bsz, D_OUT, R, device="cuda").bfloat16()
    d3 = per_sample_lora_delta(x, sA, sB, torch.ones(bsz, device="cuda"))
    assert d3.shape == (bsz, seq, D_OUT)
    torch.cuda.synchronize()
    assert lithe_amd.kernels._hip.workspace_errors() == 0


def test_empty_rows_through_index_layer_and_decode(small):
    _, ia, ib, pa, pb, bank = small
    base = torch.nn.Linear(D_IN, D_OUT).cuda().bfloat16()
    layer = IndexLoRALinear(base, ia, ib, pa.bfloat16(), pb.bfloat16(), R, 1.0)
    x = torch.zeros(0, D_IN, device="cuda", dtype=torch.bfloat16)
    layer.assign = torch.zeros(0, dtype=torch.int32, device="cuda")
    assert layer(x).shape == (0, D_OUT)
    out = decode_packed_slots(bank.words, torch.zeros(0, dtype=torch.int32, device="cuda"), bank.layout,
                              bank.pool_a, bank.pool_b)
    assert out.shape == (0, bank.layout.total_blocks, 64)


def test_largest_batch_matches_oracle(small):
    """65,535 samples of one token each (the most the delta accepts), routed over the 3 slots."""
    ads, ia, ib, pa, pb, _ = small
    bsz = 65535
    g = torch.Generator(device="cuda").manual_seed(11)
    x = torch.randn(bsz, 1, D_IN, device="cuda", generator=g).bfloat16()
    assign = torch.randint(0, 3, (bsz,), device="cuda", generator=g, dtype=torch.int32)
    got = shared_codebook_lora_delta(x, ia, pa, ib, pb, assign, R, D_OUT, 0.75).float().cpu().numpy()
    xs, a_np = x.float().cpu().numpy(), assign.cpu().numpy()
    opa, opb = ocb.twin_pools()
    ia_np, ib_np = ia.cpu().numpy(), ib.cpu().numpy()
    for s in range(3):
        rows = np.nonzero(a_np == s)[0]
        want = odelta.shared_delta(xs[rows][None, :, 0], ia_np, opa, ib_np, opb, [s], R, D_OUT, 0.75)
        assert rel(got[rows][:, 0], want[0]) < 2e-3, s
    with pytest.raises(ValueError):
        shared_codebook_lora_delta(torch.zeros(bsz + 1, 1, D_IN, device="cuda").bfloat16(), ia, pa, ib, pb,
                                   torch.zeros(bsz + 1, dtype=torch.int32, device="cuda"), R, D_OUT, 1.0)
