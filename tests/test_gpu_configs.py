"""GPU checks of the delta on two whole serving workloads, read from a bank of the 342-linear FLUX
layout with uniformly random 9-bit fields:

* the 512^2 FFN pair: up 3072 -> 12288 and down 12288 -> 3072 at B = 14 samples x 1,536 tokens,
  each sample routed to a distinct slot of a 1,000-slot bank (drawn uniformly, seeded). The down
  projection is planned with one rank group and K split over 2 waves per token group;
* the 256^2 high-batch sweep: the seven (d_in, d_out, tokens) classes of the 342 linears at
  B = 96 samples (256 image, 512 text, 768 single-block tokens), the 96 slots drawn from a
  Zipf(1.1) law over a 10,000-slot bank (24 GB resident), so adapters repeat within the batch.

Bit-exact, size-independent properties (each token's result depends only on its own x row, its
slot's factors and the plan, which is the same for every sample of a call): accumulate = the
write-mode delta added with one bf16 rounding; permuting the samples with their slots permutes
the outputs; a copy of a slot in another slot gives the same output; changing one sample's x
leaves every other sample's output alone; two samples routed to one slot with the same x get the
same output. Plus the oracle on the first and last token rows of a few samples (one of them a
repeated slot), within the bf16 tolerance of tests/test_gpu_delta.py.
"""
import numpy as np
import pytest
import torch

from lithe_amd.kernels import PackedBank, PackedLayout, packed_lora_delta, unpack_indices, workspace_errors
from oracle import codebook as ocb
from oracle import delta as odelta

from helpers import flux_modules, rel

pytestmark = pytest.mark.gpu
RANK = 16
REL_BF16 = 2e-3


def _bank(n_slots, seed):
    layout = PackedLayout.from_modules(
        [{"name": n, "shape_a": [RANK, di], "shape_b": [do, RANK]} for n, di, do in flux_modules()],
        num_levels=3, block_size=64, scaling=1.0)
    bank = PackedBank(layout, "cuda", capacity=n_slots)
    bank.fill_random(n_slots, generator=torch.Generator(device="cuda").manual_seed(seed))
    return bank


def _slot_indices(bank, slot, name):
    """Level-major (3, n_blocks) A and B indices of module ``name`` in ``slot``, unpacked from the
    slot's words (residency order: (block, level)-major, A blocks at a_off, B blocks at b_off)."""
    _, sa, sb, a_off, b_off = bank.layout.module(name)
    idx = unpack_indices(bank.words[slot], bank.layout.num_indices).view(-1, 3).cpu().numpy()
    na, nb = sa[0] * sa[1] // 64, sb[0] * sb[1] // 64
    return idx[a_off:a_off + na].T.copy(), idx[b_off:b_off + nb].T.copy()


class Case:
    def __init__(self, bank, assign, copy_slot, scale):
        self.bank, self.assign, self.copy_slot, self.scale = bank, assign, copy_slot, scale
        self.pools = (bank.pool_a.bfloat16(), bank.pool_b.bfloat16())
        # the copy slot holds the words of the first sample's slot
        bank.words[copy_slot].copy_(bank.words[int(assign[0])])

    def delta(self, name, x, assign=None, out=None, accumulate=False):
        _, _, sb, a_off, b_off = self.bank.layout.module(name)
        return packed_lora_delta(x, self.bank.words, a_off, b_off, 3, self.pools,
                                 self.assign if assign is None else assign, RANK, sb[0], self.scale, out=out,
                                 accumulate=accumulate)


def _check(case, name, d_in, d_out, m, oracle_samples):
    assign = case.assign
    B = assign.numel()
    g = torch.Generator(device="cuda").manual_seed(sum(map(ord, name)) + m)
    x = torch.randn(B, m, d_in, device="cuda", generator=g).bfloat16()
    # samples routed to an already-used slot repeat that sample's x
    first = {}
    rep = []
    for i, s in enumerate(assign.tolist()):
        if s in first:
            x[i] = x[first[s]]
            rep.append((first[s], i))
        else:
            first[s] = i
    y0 = torch.randn(B, m, d_out, device="cuda", generator=g).bfloat16()
    d = case.delta(name, x)
    for i, j in rep:
        assert torch.equal(d[i], d[j]), (name, i, j)
    y = y0.clone()
    case.delta(name, x, out=y, accumulate=True)
    assert torch.equal(y, (y0.float() + d.float()).bfloat16())
    del y, y0
    perm = torch.randperm(B, generator=torch.Generator().manual_seed(1)).cuda()
    assert torch.equal(case.delta(name, x[perm].contiguous(), assign[perm].contiguous()), d[perm])
    a2 = assign.clone()
    a2[0] = case.copy_slot
    assert torch.equal(case.delta(name, x, a2), d)
    x2 = x.clone()
    k = B // 2
    x2[k] = torch.randn(m, d_in, device="cuda", generator=g).bfloat16()
    d2 = case.delta(name, x2)
    keep = [i for i in range(B) if i != k]
    assert torch.equal(d2[keep], d[keep]) and not torch.equal(d2[k], d[k])
    del x2, d2
    assert workspace_errors() == 0
    opa, opb = ocb.twin_pools()
    rows = np.r_[0:4, m - 4:m]
    for smp in oracle_samples:
        ia, ib = _slot_indices(case.bank, int(assign[smp]), name)
        xr = x[smp:smp + 1, rows].float().cpu().numpy()
        want = odelta.shared_delta(xr, ia[None], opa, ib[None], opb, [0], RANK, d_out, case.scale)
        got = d[smp:smp + 1, rows].float().cpu().numpy()
        assert rel(got, want) < REL_BF16, (name, m, smp, rel(got, want))


# ------------------------------------------------------------------ 512^2 FFN pair, 1,000-slot bank
@pytest.fixture(scope="module")
def ffn():
    bank = _bank(1000, seed=21)
    rng = np.random.default_rng(1234)
    assign = rng.choice(999, 14, replace=False)           # slot 999 is the copy slot
    case = Case(bank, torch.tensor(assign, dtype=torch.int32, device="cuda"), 999, 1.0)
    yield case
    del case, bank
    torch.cuda.empty_cache()


@pytest.mark.parametrize("name,d_in,d_out", [("transformer_blocks.0.ff.net.0.proj", 3072, 12288),
                                             ("transformer_blocks.0.ff.net.2", 12288, 3072)])
def test_ffn_pair_b14x1536(ffn, name, d_in, d_out):
    _check(ffn, name, d_in, d_out, 1536, oracle_samples=(0, 13))


# ------------------------------------------------------------------ 256^2 sweep, B = 96, Zipf(1.1) over 10,000 slots
@pytest.fixture(scope="module")
def high_batch():
    n_slots = 10_000
    bank = _bank(n_slots, seed=22)
    rng = np.random.default_rng(4321)
    ranks = np.arange(1, n_slots + 1, dtype=np.float64)
    p = ranks ** -1.1
    p /= p.sum()
    perm = rng.permutation(n_slots)
    assign = perm[rng.choice(n_slots, 96, p=p)]
    assert len(set(assign.tolist())) < 96                 # Zipf routing repeats adapters
    copy_slot = int(next(s for s in range(n_slots - 1, 0, -1) if s not in set(assign.tolist())))
    case = Case(bank, torch.tensor(assign, dtype=torch.int32, device="cuda"), copy_slot, 1.0)
    yield case
    del case, bank
    torch.cuda.empty_cache()


HB_CLASSES = [("transformer_blocks.18.attn.to_q", 3072, 3072, 256),
              ("transformer_blocks.18.attn.add_k_proj", 3072, 3072, 512),
              ("transformer_blocks.18.ff.net.0.proj", 3072, 12288, 256),
              ("transformer_blocks.18.ff.net.2", 12288, 3072, 256),
              ("transformer_blocks.18.ff_context.net.0.proj", 3072, 12288, 512),
              ("transformer_blocks.18.ff_context.net.2", 12288, 3072, 512),
              ("single_transformer_blocks.37.attn.to_v", 3072, 3072, 768)]


@pytest.mark.parametrize("name,d_in,d_out,m", HB_CLASSES)
def test_high_batch_b96_zipf(high_batch, name, d_in, d_out, m):
    assign = high_batch.assign.tolist()
    seen, repeated = set(), None
    for i, s in enumerate(assign):
        if s in seen and repeated is None:
            repeated = i
        seen.add(s)
    _check(high_batch, name, d_in, d_out, m, oracle_samples=(0, repeated, 95))
