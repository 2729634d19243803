"""CPU pins of the oracle's nearest-codeword search and greedy encode (lithe/quant.py:46-71):
brute force over all 512 codewords, exact round trips of lattice points, and the exact
per-coordinate error recursion of the nine orthogonal Hadamard directions
(tests/test_quant.py:17-74 of the reference, restated)."""
import numpy as np
import pytest

from oracle import codebook as ocb
from oracle import decode as odec
from oracle import search as osr


def test_closed_form_equals_brute_force():
    rng = np.random.default_rng(0)
    pa, pb = ocb.twin_pools()
    for pools, scale in ((pa, 0.08), (pb, 0.003)):
        x = (scale * rng.standard_normal((4096, 64))).astype(np.float32)
        idx, _ = osr.nearest_index(x)
        assert np.array_equal(idx, osr.cdist_nearest(x, pools[0]))


def test_planted_wrong_hyperplanes_fail_the_pin():
    rng = np.random.default_rng(1)
    pa, _ = ocb.twin_pools()
    x = (0.08 * rng.standard_normal((2048, 64))).astype(np.float32)
    wrong = ocb.hadamard(64)[:, 1:10].astype(np.float64)        # columns 1..9 instead of 0..8
    idx, _ = osr.nearest_index(x, wrong)
    assert (idx != osr.cdist_nearest(x, pa[0])).mean() > 0.5


def test_lattice_points_round_trip_exactly():
    rng = np.random.default_rng(2)
    _, pb = ocb.twin_pools()
    true_idx = rng.integers(0, 512, (3, 2048))
    x = odec.rvq_decode(true_idx, pb)
    idx, rec, _ = osr.rvq_encode_blocks(x, pb)
    assert np.array_equal(idx, true_idx)
    assert np.array_equal(rec.view(np.uint32), x.view(np.uint32))


def test_error_follows_the_per_coordinate_recursion():
    rng = np.random.default_rng(3)
    pa, pb = ocb.twin_pools()
    u = osr.projection_matrix() / 8.0                           # orthonormal basis of col(U)
    for pools, sigmas, scale in ((pa, (0.06,) * 3, 0.06), (pb, (0.0025, 0.001, 0.0005), 0.0025)):
        x = scale * rng.standard_normal((4096, 64))
        _, rec, _ = osr.rvq_encode_blocks(x.astype(np.float32), pools)
        err = x.astype(np.float32).astype(np.float64) - rec.astype(np.float64)
        perp = x.astype(np.float32).astype(np.float64)
        perp = perp - perp @ u @ u.T
        assert np.allclose(err - err @ u @ u.T, perp, atol=1e-6)
        e = x.astype(np.float32).astype(np.float64) @ u
        for s in sigmas:
            e = e - np.where(e > 0, 1.0, -1.0) * (8.0 * s / 3.0)
        assert np.allclose(err @ u, e, atol=1e-6)


def test_blockify_factors_places_every_factor_at_its_offset():
    """The encoder's input: every factor row-major blockified (zero-padded) at its layout offset,
    A blocks before B blocks per module, as the oracle's per-factor blockify lays them out."""
    import torch

    from lithe_amd.kernels import PackedLayout, blockify_factors
    from oracle import packing as opk
    mods = [("q", 16, 256, 384), ("pad", 16, 90, 41), ("odd", 5, 7, 3), ("up", 16, 128, 512)]
    lay = PackedLayout.from_modules([{"name": n, "shape_a": [r, di], "shape_b": [do, r]} for n, r, di, do in mods])
    g = torch.Generator().manual_seed(5)
    factors = {n: (torch.randn(r, di, generator=g), torch.randn(do, r, generator=g).bfloat16())
               for n, r, di, do in mods}
    got = blockify_factors(lay, factors, "cpu").numpy()
    want = np.concatenate([opk.blockify(f.float().numpy()) for n, *_ in mods for f in factors[n]])
    assert got.shape == want.shape == (lay.total_blocks, 64)
    assert np.array_equal(got.view(np.uint32), want.astype(np.float32).view(np.uint32))
    with pytest.raises(ValueError, match="missing factors"):
        blockify_factors(lay, {k: v for k, v in factors.items() if k != "pad"}, "cpu")
    with pytest.raises(ValueError, match="layout"):
        blockify_factors(lay, {**factors, "odd": (factors["odd"][1], factors["odd"][0])}, "cpu")


def test_encode_refuses_cpu_tensors():
    """The encode runs only on the GPU: a CPU factor raises RuntimeError, nothing is computed
    on the host."""
    import torch

    from lithe_amd import codebook as cb
    from lithe_amd import quant
    pa, _ = cb.twin_pools()
    with pytest.raises(RuntimeError):
        quant.encode(torch.zeros(4, 64), pa, cb.projection_matrix())
