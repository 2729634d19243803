"""GPU checks of the delta at the headline workload's real shapes, where the oracle is too slow
to run whole: B = 14 samples routed to 14 distinct slots of a packed bank, with the shapes of the
342-linear FLUX sweep, all seven (d_in, d_out, tokens) classes: 3072 -> 3072 at 4,608 (single-block
q / k / v), 4,096 (image attention) and 512 (text attention) tokens; 3072 -> 12288 at 4,096 and 512;
12288 -> 3072 at 4,096 (planned with K split over 2 waves, one rank group) and 512 (K split over 4
waves).

Size-independent properties, bit-exact (each token's result depends only on its own x row, its
slot's factors and the plan, which is the same for every sample):

* accumulate = the write-mode delta added to the base output with one bf16 rounding;
* permuting the samples together with their slots permutes the outputs;
* routing a sample to a copy of its slot changes nothing;
* changing one sample's x leaves every other sample's output unchanged;

and, on a few token rows of two samples, agreement with the oracle within the bf16 tolerance of
tests/test_gpu_delta.py.
"""
import numpy as np
import pytest
import torch

from lithe_amd.kernels import PackedBank, packed_lora_delta
from oracle import codebook as ocb
from oracle import delta as odelta

from helpers import random_adapter, rel

pytestmark = pytest.mark.gpu
MODS = [("single.q", 3072, 3072), ("img.q", 3072, 3072), ("txt.q", 3072, 3072), ("ff.up", 3072, 12288),
        ("ffc.up", 3072, 12288), ("ff.down", 12288, 3072), ("ffc.down", 12288, 3072)]
TOKENS = {"single.q": 4608, "img.q": 4096, "txt.q": 512, "ff.up": 4096, "ffc.up": 512, "ff.down": 4096,
          "ffc.down": 512}
B, RANK, SCALE = 14, 16, 0.75


@pytest.fixture(scope="module")
def setup():
    ads = [random_adapter(MODS, rank=RANK, seed=300 + s) for s in range(B + 2)]
    bank, words = PackedBank.from_adapters(ads, "cuda")
    for w in words:
        bank.add(w)
    bank.add(words[5])                                  # slot 16: a copy of slot 5
    assign = torch.tensor([5, 0, 9, 2, 14, 7, 1, 12, 3, 15, 8, 11, 4, 6], dtype=torch.int32, device="cuda")
    pools = (bank.pool_a.bfloat16(), bank.pool_b.bfloat16())
    return ads, bank, assign, pools


def _delta(bank, pools, name, x, assign, out=None, accumulate=False):
    _, sa, sb, a_off, b_off = bank.layout.module(name)
    return packed_lora_delta(x, bank.words, a_off, b_off, 3, pools, assign, RANK, sb[0], SCALE, out=out,
                             accumulate=accumulate)


@pytest.mark.parametrize("name,d_in,d_out", MODS)
def test_fullsize_exact_properties(setup, name, d_in, d_out):
    ads, bank, assign, pools = setup
    m = TOKENS[name]
    g = torch.Generator(device="cuda").manual_seed(sum(map(ord, name)))
    x = torch.randn(B, m, d_in, device="cuda", generator=g).bfloat16()
    y0 = torch.randn(B, m, d_out, device="cuda", generator=g).bfloat16()
    d = _delta(bank, pools, name, x, assign)
    # accumulate == write-mode delta added with one rounding
    y = y0.clone()
    _delta(bank, pools, name, x, assign, out=y, accumulate=True)
    assert torch.equal(y, (y0.float() + d.float()).bfloat16())
    # permutation equivariance
    perm = torch.randperm(B, generator=torch.Generator().manual_seed(1)).cuda()
    dp = _delta(bank, pools, name, x[perm].contiguous(), assign[perm].contiguous())
    assert torch.equal(dp, d[perm])
    # a copy of a slot gives the same output
    a2 = assign.clone()
    a2[0] = 16                                          # slot 16 holds slot 5's words
    assert torch.equal(_delta(bank, pools, name, x, a2), d)
    # sample independence
    x2 = x.clone()
    x2[3] = torch.randn(m, d_in, device="cuda", generator=g).bfloat16()
    d2 = _delta(bank, pools, name, x2, assign)
    keep = [i for i in range(B) if i != 3]
    assert torch.equal(d2[keep], d[keep]) and not torch.equal(d2[3], d[3])
    # oracle on 8 token rows of two samples
    opa, opb = ocb.twin_pools()
    for smp in (0, B - 1):
        rows = x[smp:smp + 1, :8].float().cpu().numpy()
        j = int(assign[smp])
        ia = ads[j].indices[name]["A"][None].astype(np.int64)
        ib = ads[j].indices[name]["B"][None].astype(np.int64)
        want = odelta.shared_delta(rows, ia, opa, ib, opb, [0], RANK, d_out, SCALE)
        got = d[smp:smp + 1, :8].float().cpu().numpy()
        assert rel(got, want) < 2e-3, (name, smp)


def test_fullsize_encode_round_trip():
    """A whole 342-linear rank-16 adapter (700,416 blocks) decoded to dense factors and encoded
    back into a bank slot (PackedBank.encode_factors): every B index comes back (pool B's level
    scales are separable), and every A factor decodes to within 1e-7 of the original (equal A
    scales admit other index triples with the same sum; tests/test_module.py:115-127 of the
    reference)."""
    import lithe_amd
    from lithe_amd.kernels import pack_adapter, split_decoded
    from helpers import flux_modules
    ad = random_adapter(flux_modules(), rank=16, seed=77)
    words, layout = pack_adapter(ad)
    bank = PackedBank(layout, "cuda", capacity=2)
    bank.add(words)
    factors = lithe_amd.decode_factors(ad)                       # fp32 on the GPU
    slot = bank.encode_factors(factors)
    assert slot == 1 and bank.ingest_errors() == 0
    got = bank.decode_slots(torch.tensor([slot], dtype=torch.int32, device="cuda"), dtype=torch.float32)[0]
    got = split_decoded(got, layout)
    from lithe_amd.kernels import unpack_indices
    idx = unpack_indices(bank.words[slot], layout.num_indices).view(-1, 3).cpu().numpy()
    for name, sa, sb, a_off, b_off in zip(layout.names, layout.shapes_a, layout.shapes_b, layout.a_off, layout.b_off):
        nb = -(-sb[0] * sb[1] // 64)
        assert np.array_equal(idx[b_off:b_off + nb].T, ad.indices[name]["B"].astype(np.int64)), name
        a, _ = factors[name]
        assert torch.allclose(got[name][0], a, atol=1e-7), name
