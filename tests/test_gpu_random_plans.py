"""Seeded random sweep of the index-resident delta against the oracle: ranks 16-128 (one to eight
rank groups; the rank collapse at 32, 64, 96 and 128), per-call and grouped launches of one to three
modules with their own token counts or all reading one x (the shared-input shrink), bf16 and fp32
outputs, write and accumulate mode, and random
plan overrides (waves along the outputs, expand sub-tiles, the shrink's K split and token groups
per wave, the rank collapse off, the shared-input shrink form). Every plan computes the same delta up to the fp32 summation
order, so each case must meet the bf16 tolerance of tests/test_gpu_delta.py (rel-Frobenius 2e-3
against the oracle; 1e-2 on the change of an accumulated bf16 output, which includes the rounding
of y + delta). A second sweep runs serve.py's mixture routing."""
import math

import numpy as np
import pytest
import torch
from torch import nn

from lithe_amd import serve

from lithe_amd.kernels import PackedBank, packed_lora_delta, workspace_errors
from lithe_amd.kernels.prepared import group_workspace_bytes, prepare_packed_group, shared_workspace
from oracle import codebook as ocb
from oracle import delta as odelta

from helpers import random_adapter, rel

pytestmark = pytest.mark.gpu

KNOBS = {"LITHE_EXPAND_WO": ["1", "2", "4"], "LITHE_EXPAND_SUBS": ["1", "2", "4", "8"],
         "LITHE_SHRINK_KS": ["1", "2", "4"], "LITHE_SHRINK_TW": ["1", "2"], "LITHE_EXPAND_NS": ["1"],
         "LITHE_SHARED_X_STACKED": ["0", "1"]}


def _case(rng, monkeypatch):
    rank = int(rng.choice([16, 32, 48, 64, 96, 128]))
    grouped = bool(rng.integers(0, 2))
    n_mod = int(rng.integers(1, 4)) if grouped else 1
    shapes = [(f"m{m}", int(rng.integers(1, 33)) * 64, int(rng.integers(2, 400)) * 4) for m in range(n_mod)]
    n_ad, batch = int(rng.integers(1, 5)), int(rng.integers(1, 5))
    seqs = [int(rng.integers(1, 300)) for _ in range(n_mod)]
    share = grouped and n_mod > 1 and bool(rng.integers(0, 2))    # every module reads one x
    if share:
        shapes = [(nm, shapes[0][1], do) for nm, _, do in shapes]
        seqs = [seqs[0]] * n_mod
    out_dt = torch.bfloat16 if rng.integers(0, 3) else torch.float32
    acc, scale = bool(rng.integers(0, 2)), float(rng.choice([1.0, 0.5, 2.0]))
    for k, v in KNOBS.items():
        if rng.integers(0, 2):
            monkeypatch.setenv(k, v[int(rng.integers(0, len(v)))])
        else:
            monkeypatch.delenv(k, raising=False)
    desc = (rank, grouped, share, shapes, seqs, batch, n_ad, out_dt, acc, scale)
    ads = [random_adapter(shapes, rank=rank, seed=int(rng.integers(0, 1 << 30))) for _ in range(n_ad)]
    bk, words = PackedBank.from_adapters(ads, "cuda")
    for w in words:
        bk.add(w)
    pools = (bk.pool_a.bfloat16(), bk.pool_b.bfloat16())
    assign = torch.tensor(rng.integers(0, n_ad, batch), dtype=torch.int32, device="cuda")
    gen = torch.Generator(device="cuda").manual_seed(int(rng.integers(0, 1 << 30)))
    xs = [torch.randn(batch, s, di, device="cuda", generator=gen).bfloat16() for (_, di, _), s in zip(shapes, seqs)]
    if share:
        xs = [xs[0]] * n_mod
    if grouped:
        acc = True
        y0s = [(torch.randn(batch, s, do, device="cuda", generator=gen) if out_dt == torch.bfloat16
                else torch.zeros(batch, s, do, device="cuda")).to(out_dt) for (_, _, do), s in zip(shapes, seqs)]
        outs = [y.clone() for y in y0s]
        offs = [bk.layout.module(nm)[3:5] for nm, _, _ in shapes]
        need = group_workspace_bytes([(s, di, do) for (_, di, do), s in zip(shapes, seqs)],
                                     [0] * n_mod if share else list(range(n_mod)), batch, rank, 1, torch.bfloat16)
        prepare_packed_group(xs, outs, bk.words, offs, 3, pools, assign, rank, scale, shared_workspace("cuda", need),
                             accumulate=True)()
    else:
        _, _, sb, a_off, b_off = bk.layout.module(shapes[0][0])
        do = shapes[0][2]
        y0s = [torch.randn(batch, seqs[0], do, device="cuda", generator=gen).to(out_dt)]
        if acc:
            outs = [y0s[0].clone()]
            packed_lora_delta(xs[0], bk.words, a_off, b_off, 3, pools, assign, rank, sb[0], scale, out=outs[0],
                              accumulate=True)
        else:
            outs = [packed_lora_delta(xs[0], bk.words, a_off, b_off, 3, pools, assign, rank, sb[0], scale,
                                      out_dtype=out_dt)]
    torch.cuda.synchronize()
    assert workspace_errors() == 0, desc
    opa, opb = ocb.twin_pools()
    od = "bf16" if out_dt == torch.bfloat16 else "fp32"
    for m, ((nm, _, do), _) in enumerate(zip(shapes, seqs)):
        ia = np.stack([a.indices[nm]["A"] for a in ads]).astype(np.int64)
        ib = np.stack([a.indices[nm]["B"] for a in ads]).astype(np.int64)
        want = odelta.shared_delta(xs[m].float().cpu().numpy(), ia, opa, ib, opb, assign.tolist(), rank, do, scale,
                                   "bf16", od)
        got = outs[m].float().cpu().numpy()
        if acc:
            y0 = y0s[m].float().cpu().numpy()
            want = odelta.index_linear(y0, want, od) if od == "bf16" else y0 + want
            err, tol = rel(got - y0, want - y0), (1e-2 if od == "bf16" else 2e-3)
        else:
            err, tol = rel(got, want), 2e-3
        assert err < tol, (desc, m, err)


@pytest.mark.parametrize("seed", [11, 12, 13])
def test_random_plans_match_oracle(monkeypatch, seed):
    rng = np.random.default_rng(seed)
    for _ in range(50):
        _case(rng, monkeypatch)


class _One(nn.Module):
    def __init__(self, d_in, d_out):
        super().__init__()
        self.fc = nn.Linear(d_in, d_out)

    def forward(self, x):
        return self.fc(x)


def test_random_mixtures_match_serve_oracle(monkeypatch):
    """serve.py mixture routing (0 to 8 / ceil(rank / 16) weighted route entries per sample, ranks
    8-128, bf16 and fp32 activations) under random plan overrides against the oracle's
    serve_forward: rtol / atol 1e-5 in fp32, rel-Frobenius 2e-3 in bf16 (tests/test_gpu_serve.py)."""
    rng = np.random.default_rng(21)
    pa, pb = ocb.twin_pools()
    for n in range(60):
        rank = int(rng.choice([8, 16, 32, 48, 64, 128]))
        n_routes = int(rng.integers(1, max(1, 8 // ((rank + 15) // 16)) + 1))
        n_ad = n_routes + int(rng.integers(0, 3))
        d_in = int(rng.integers(1, 25)) * 64
        d_out = int(rng.integers(2, 300)) * (64 // math.gcd(64, rank))
        batch, seq = int(rng.integers(1, 5)), int(rng.integers(1, 200))
        dtype = torch.bfloat16 if rng.integers(0, 3) else torch.float32
        for k, v in KNOBS.items():
            if rng.integers(0, 2):
                monkeypatch.setenv(k, v[int(rng.integers(0, len(v)))])
            else:
                monkeypatch.delenv(k, raising=False)
        routes = []
        for _ in range(batch):
            ids = rng.choice(n_ad, int(rng.integers(0, n_routes + 1)), replace=False)
            w = rng.uniform(0.2, 1.0, len(ids))
            w = w / max(w.sum(), 1e-6)
            routes.append([(int(a), float(v)) for a, v in zip(ids, w)])
        ads = [random_adapter([("fc", d_in, d_out)], rank=rank, seed=int(rng.integers(0, 1 << 30))) for _ in range(n_ad)]
        for a in ads:
            a.alpha = float(rng.choice([rank, 2 * rank]))
        torch.manual_seed(n)
        model = _One(d_in, d_out).cuda().to(dtype)
        router, layers = serve.attach_adapters(model, ads)
        router.set(routes)
        x = torch.randn(batch, seq, d_in, generator=torch.Generator().manual_seed(n)).to(dtype)
        with torch.no_grad():
            base_out = layers["fc"].base(x.cuda()).float().cpu().numpy()
            y = model(x.cuda()).float().cpu().numpy()
        ia = np.stack([a.indices["fc"]["A"] for a in ads])
        ib = np.stack([a.indices["fc"]["B"] for a in ads])
        scales = np.array([a.alpha / a.rank for a in ads], np.float32)
        want = odelta.serve_forward(x.float().numpy(), base_out, router.ids.numpy(), router.weights.numpy(), ia, ib,
                                    scales, pa, pb, rank, "fp32" if dtype == torch.float32 else "bf16")
        case = (rank, n_routes, d_in, d_out, batch, seq, dtype, routes)
        if dtype == torch.float32:
            np.testing.assert_allclose(y, want, rtol=1e-5, atol=1e-5, err_msg=str(case))
        else:
            assert rel(y, want) < 2e-3, case
