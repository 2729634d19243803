"""GPU parity of serve.py routing, the decoded-factor SGMV and LitheLinear against the oracle.

Tolerances: fp32 activations rtol 1e-5 / atol 1e-5 against the float64-evaluated
oracle (the reference's own serve test uses atol 1e-6 at d=128,
tests/test_serve.py:46 of the reference; at d=3072 fp32 accumulation order alone
moves results by ~1e-6). bf16 activations: rel-Frobenius < 2e-3 vs the oracle
with the reference's rounding steps.
"""
import numpy as np
import pytest
import torch
from torch import nn

import lithe_amd
from lithe_amd import serve
from lithe_amd.kernels import PerSampleLoRALinear, per_sample_lora_delta
from oracle import codebook as ocb
from oracle import decode as odec
from oracle import delta as odelta

from helpers import random_adapter, rel, to_np

pytestmark = pytest.mark.gpu


class One(nn.Module):
    def __init__(self, d_in, d_out):
        super().__init__()
        self.fc = nn.Linear(d_in, d_out)

    def forward(self, x):
        return self.fc(x)


def _serve_case(d_in, d_out, rank, n_ad, routes, x, alpha=None, dtype=torch.float32):
    ads = [random_adapter([("fc", d_in, d_out)], rank=rank, seed=100 + s) for s in range(n_ad)]
    for a in ads:
        a.alpha = float(alpha if alpha is not None else rank)
    torch.manual_seed(0)
    model = One(d_in, d_out).cuda().to(dtype)
    router, layers = serve.attach_adapters(model, ads)
    router.set(routes)
    with torch.no_grad():
        base_out = to_np(layers["fc"].base(x.cuda()))
        y = to_np(model(x.cuda()))
    ids, w = router.ids.numpy(), router.weights.numpy()
    ia = np.stack([a.indices["fc"]["A"] for a in ads])
    ib = np.stack([a.indices["fc"]["B"] for a in ads])
    scales = np.array([a.alpha / a.rank for a in ads], np.float32)
    pa, pb = ocb.twin_pools()
    want = odelta.serve_forward(to_np(x), base_out, ids, w, ia, ib, scales, pa, pb, rank,
                                "fp32" if dtype == torch.float32 else "bf16")
    return y, want, ads


def test_config1_serve_fp32():
    """One 3072->3072 layer, rank 16, 4 adapters, 4 x 256 tokens fp32, sample i -> adapter i."""
    x = torch.randn(4, 256, 3072, generator=torch.Generator().manual_seed(0))
    y, want, _ = _serve_case(3072, 3072, 16, 4, [[(i, 1.0)] for i in range(4)], x)
    np.testing.assert_allclose(y, want, rtol=1e-5, atol=1e-5)


def test_serve_mixture_empty_and_alpha():
    x = torch.randn(5, 10, 128, generator=torch.Generator().manual_seed(1))
    routes = [[(0, 1.0)], [(2, 1.0)], [], [(1, 0.6), (2, 0.4)], [(0, 1.0)]]
    y, want, ads = _serve_case(128, 64, 4, 3, routes, x, alpha=8.0)
    np.testing.assert_allclose(y, want, rtol=1e-5, atol=1e-6)
    # closed form: base + sum_a w_a (x A_a^T B_a^T) alpha / r (tests/test_serve.py:28-46 of the reference)
    pa, pb = ocb.twin_pools()
    base_minus = y - want      # ~0; the closed form below checks the oracle itself
    assert np.abs(base_minus).max() < 1e-5
    for i, r in enumerate(routes):
        d = np.zeros((10, 64))
        for a_id, wt in r:
            a = odec.decode(ads[a_id].indices["fc"]["A"], (4, 128), pa)
            b = odec.decode(ads[a_id].indices["fc"]["B"], (64, 4), pb)
            d += wt * odelta.truth_delta(to_np(x)[i], a, b) * 2.0
        assert np.abs(want[i] - (want[i] - d) - d).max() < 1e-12


def test_serve_bf16_and_three_way_mixture():
    x = torch.randn(3, 40, 256, generator=torch.Generator().manual_seed(2)).bfloat16()
    routes = [[(0, 0.5), (1, 0.3), (2, 0.2)], [(1, 1.0)], [(2, 0.7), (0, 0.3)]]
    y, want, _ = _serve_case(256, 192, 16, 3, routes, x, dtype=torch.bfloat16)
    assert rel(y, want) < 2e-3


def test_serve_all_empty_returns_base_and_errors():
    x = torch.randn(2, 8, 128, generator=torch.Generator().manual_seed(3))
    y, want, _ = _serve_case(128, 64, 4, 2, [[], []], x)
    assert np.array_equal(y, want)
    ads = [random_adapter([("fc", 128, 64)], rank=4, seed=1)]
    model = One(128, 64).cuda()
    router, _ = serve.attach_adapters(model, ads)
    router.set([[(0, 1.0)]])
    with pytest.raises(ValueError):
        model(torch.randn(2, 8, 128, device="cuda"))
    router.set([[(3, 1.0)]])
    with pytest.raises(IndexError):
        model(torch.randn(1, 8, 128, device="cuda"))


@pytest.mark.parametrize("seq,d_in,d_out,r", [(256, 3072, 9216, 16), (77, 512, 640, 16), (10, 256, 128, 4)])
def test_per_sample_sgmv_matches_oracle(seq, d_in, d_out, r):
    g = torch.Generator().manual_seed(seq)
    x = (torch.randn(3, seq, d_in, generator=g) * 0.5).bfloat16()
    a = (torch.randn(3, r, d_in, generator=g) * 0.02).bfloat16()
    b = (torch.randn(3, d_out, r, generator=g) * 0.02).bfloat16()
    s = torch.tensor([0.5, 1.0, 2.0]).bfloat16()
    got = per_sample_lora_delta(x.cuda(), a.cuda(), b.cuda(), s.cuda())
    assert got.dtype == torch.bfloat16 and got.shape == (3, seq, d_out)
    want = odelta.per_sample_delta(to_np(x), to_np(a), to_np(b), to_np(s), "bf16")
    x64, a64, b64 = (to_np(t).astype(np.float64) for t in (x, a, b))
    truth = np.stack([x64[i] @ a64[i].T @ b64[i].T for i in range(3)]) * to_np(s)[:, None, None]
    assert rel(to_np(got), want) < 2e-3 and rel(to_np(got), truth) < 1e-2


def test_per_sample_layer_and_fp32():
    torch.manual_seed(0)
    base = nn.Linear(128, 64).cuda()
    facs = [(torch.randn(4, 128, device="cuda"), torch.randn(64, 4, device="cuda"), 0.5),
            (torch.randn(4, 128, device="cuda"), torch.randn(64, 4, device="cuda"), 2.0)]
    layer = PerSampleLoRALinear(base, "sgmv")
    layer.set_factors(facs)
    for x in (torch.randn(3, 6, 128, device="cuda"), torch.randn(3, 128, device="cuda")):
        with torch.no_grad():
            got = layer(x)
            want = base(x) + torch.stack([
                torch.nn.functional.linear(torch.nn.functional.linear(x[i], facs[i % 2][0]), facs[i % 2][1])
                * facs[i % 2][2] for i in range(3)])
        np.testing.assert_allclose(to_np(got), to_np(want), rtol=1e-4, atol=1e-4)


def test_lithe_linear_inference():
    ad = random_adapter([("fc", 256, 384)], rank=16, seed=9)
    ad.alpha = 8.0
    torch.manual_seed(0)
    model = One(256, 384).cuda().bfloat16()
    layers = lithe_amd.inject_lithe(model, ["fc"], rank=16, alpha=8.0)
    layer = layers["fc"]
    layer.load_indices(torch.from_numpy(ad.indices["fc"]["A"].astype(np.int64)),
                       torch.from_numpy(ad.indices["fc"]["B"].astype(np.int64)))
    pa, pb = ocb.twin_pools()
    a_hat = odec.decode(ad.indices["fc"]["A"], (16, 256), pa)
    b_hat = odec.decode(ad.indices["fc"]["B"], (384, 16), pb)
    ah, bh = layer.decoded_factors()
    assert np.array_equal(to_np(ah).view(np.uint32), a_hat.view(np.uint32))
    assert np.array_equal(to_np(bh).view(np.uint32), b_hat.view(np.uint32))
    x = torch.randn(2, 50, 256, generator=torch.Generator().manual_seed(4)).bfloat16()
    with torch.no_grad():
        base_out = to_np(layer.base(x.cuda()))
        got = to_np(model(x.cuda()))
    want = odelta.lithe_linear(to_np(x), base_out, a_hat, b_hat, 0.5, "bf16")
    assert rel(got, want) < 2e-3
    # the codebook's GPU encode returns every B index of the decoded factor (pool B's level scales
    # are separable) and reconstructs it exactly
    idx_b, b_rec = layer.codebook.encode(bh, "B")
    assert np.array_equal(idx_b.cpu().numpy(), ad.indices["fc"]["B"].astype(np.int64))
    assert torch.equal(b_rec, bh)


@pytest.mark.parametrize("n_routes,rank,d_out", [(2, 16, 200), (6, 16, 200), (8, 16, 328), (2, 32, 264), (5, 8, 96),
                                                 (3, 32, 200), (4, 32, 264), (2, 64, 136)])
def test_serve_bf16_rank_group_tiles(n_routes, rank, d_out):
    """bf16 mixtures over 2..8 rank groups: every output-tile width of the expand (256, 128
    and 64 outputs), partial last tiles, a ragged token count and a sample with one route
    entry fewer than the others (an empty rank group). Ranks 32 and 64 sum the rank groups of a
    route before the expand's MFMA (2 to 4 such sums per token, one of them empty for 3 routes)."""
    rng = np.random.default_rng(n_routes * 100 + rank)
    n_ad = n_routes + 1
    routes = []
    for i in range(3):
        k = n_routes if i != 1 else n_routes - 1
        ids = rng.choice(n_ad, k, replace=False)
        w = rng.uniform(0.2, 1.0, k)
        w = w / w.sum()
        routes.append([(int(a), float(v)) for a, v in zip(ids, w)])
    x = torch.randn(3, 37, 192, generator=torch.Generator().manual_seed(n_routes)).bfloat16()
    y, want, _ = _serve_case(192, d_out, rank, n_ad, routes, x, alpha=2.0 * rank, dtype=torch.bfloat16)
    err = rel(y, want)
    print(f"serve bf16 routes={n_routes} rank={rank} d_out={d_out}: rel vs oracle {err:.2e}")
    assert err < 2e-3
