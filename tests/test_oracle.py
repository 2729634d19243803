"""Pinning the oracle: every restated function is checked against a fixture of the
reference's own tests, a library routine, a closed form or brute force, chosen so
that a plausible mistake (transposed operand, wrong bit order, dropped level,
wrong summation order, wrong side) fails at least one check."""
import hashlib

import numpy as np
import pytest
import scipy.linalg
import torch

from oracle import codebook as ocb
from oracle import decode as odec
from oracle import delta as odelta
from oracle import native
from oracle import packing as opk

from helpers import SMALL, random_adapter


# ------------------------------------------------------------------ codebook
def test_codebook_sha256_pin():
    # digest from the reference's tests/test_codebook.py:9
    table = ocb.integer_table()
    assert table.shape == (512, 64) and table.dtype == np.int8
    assert hashlib.sha256(table.tobytes()).hexdigest() == ocb.INT_TABLE_SHA256


def test_hadamard_equals_scipy_and_is_orthogonal():
    h = ocb.hadamard(64).astype(np.int64)
    assert np.array_equal(h, scipy.linalg.hadamard(64))
    assert (h @ h.T == 64 * np.eye(64, dtype=np.int64)).all()
    for t in (0, 1, 5, 33, 63):
        for j in (0, 3, 8, 62):
            assert h[t, j] == (-1) ** bin(t & j).count("1")


def test_sign_bit_order_and_table_values():
    s = ocb.signs()
    assert (s[0] == -1).all() and (s[511] == 1).all()
    assert s[1, 0] == 1 and (s[1, 1:] == -1).all()          # bit 0 is the LSB
    assert s[256, 8] == 1 and (s[256, :8] == -1).all()
    t = ocb.integer_table()
    assert len({row.tobytes() for row in t}) == 512
    assert set(np.unique(t).tolist()) <= {-9, -7, -5, -3, -1, 1, 3, 5, 7, 9}
    assert (t[511] == ocb.generator().astype(np.int64).sum(axis=1)).all()   # all +1 signs: row sums of U


def test_planted_codebook_mistakes_break_the_pin():
    u = ocb.generator().astype(np.int64)
    s = ocb.signs().astype(np.int64)
    # LSB/MSB swap of the sign bits, and relabelling k -> 511 - k, both change the digest
    wrong = (s[:, ::-1] @ u.T).astype(np.int8)
    assert hashlib.sha256(wrong.tobytes()).hexdigest() != ocb.INT_TABLE_SHA256
    wrong = ((-s) @ u.T).astype(np.int8)
    assert hashlib.sha256(wrong.tobytes()).hexdigest() != ocb.INT_TABLE_SHA256


def test_pools_scales_and_float64_order():
    pa, pb = ocb.twin_pools()
    c = ocb.integer_table().astype(np.float64) / 3.0
    for level, sig in enumerate(ocb.SIGMA_A):
        assert np.array_equal(pa[level], (sig * c).astype(np.float32))
    for level, sig in enumerate(ocb.SIGMA_B):
        assert np.array_equal(pb[level], (sig * c).astype(np.float32))
        np.testing.assert_allclose(pb[level], sig * c, rtol=1e-6, atol=0)
    assert abs((c ** 2).mean() - 1.0) < 1e-12                  # unit per-coordinate variance
    assert np.allclose(np.linalg.norm(c, axis=1), 8.0)


def test_codeword_period_16_and_popcount_closed_form():
    """3c_k[t] = 9 - 2 popcount((k ^ m_t) & 511), m_t depends on t mod 16 (the kernels' decode)."""
    t = ocb.integer_table().astype(np.int64)
    assert np.array_equal(t[:, :16], t[:, 16:32]) and np.array_equal(t[:, :16], t[:, 48:64])
    for tt in range(64):
        m = sum(((bin(tt & q).count("1") + 1) & 1) << q for q in range(9))
        k = np.arange(512)
        pc = np.array([bin((kk ^ m) & 511).count("1") for kk in k])
        assert np.array_equal(t[:, tt], 9 - 2 * pc)


@pytest.mark.parametrize("rank,collapses", [(32, True), (64, True), (128, True), (48, False)])
def test_rank_groups_sharing_a_factor_block_have_equal_columns(rank, collapses):
    """The expand's rank collapse: B (d_out x r) is the flat factor o * r + j cut into 64-value
    blocks, each four copies of a 16-value period, so when r is a multiple of 32 the 16-rank groups
    of an output that fall in one block have equal columns and (sum of their mid values) . P equals
    mid . B^T. At r = 48 an output's groups straddle blocks: the columns differ."""
    d_out = 40
    ad = random_adapter([("l", 64, d_out)], rank=rank, seed=rank)
    pa, pb = ocb.twin_pools()
    b = odec.decode(np.asarray(ad.indices["l"]["B"]).astype(np.int64), (d_out, rank), pb).astype(np.float64)
    ns = 4 if rank % 64 == 0 else 2
    same = all(np.array_equal(b[:, 16 * (ns * e):16 * (ns * e + 1)], b[:, 16 * (ns * e + q):16 * (ns * e + q + 1)])
               for e in range(rank // (16 * ns)) for q in range(ns))
    assert same == collapses
    if collapses:
        mid = np.random.default_rng(rank).standard_normal((9, rank))
        z = mid.reshape(9, rank // (16 * ns), ns, 16).sum(axis=2)                     # the summed fragments
        p = b.reshape(d_out, rank // (16 * ns), ns, 16)[:, :, 0, :]                    # one period per set
        np.testing.assert_allclose(np.einsum("tec,oec->to", z, p), mid @ b.T, rtol=1e-12, atol=1e-15)


# ------------------------------------------------------------------ packing
def test_pack_roundtrip_sizes_and_range():
    rng = np.random.default_rng(1)
    for n in (1, 6, 7, 8, 700, 1001):        # sizes of the reference's test_pack_roundtrip
        v = rng.integers(0, 512, n)
        w = opk.pack(v)
        assert w.dtype == np.uint64 and w.size == -(-n // 7)
        assert np.array_equal(opk.unpack(w, n), v)
    with pytest.raises(ValueError):
        opk.pack([512])


def test_pack_hand_computed_words():
    assert opk.pack([1]).tolist() == [1]
    assert opk.pack([0, 1]).tolist() == [1 << 9]
    assert opk.pack([0] * 6 + [511]).tolist() == [511 << 54]
    assert opk.pack([511] * 7).tolist() == [(1 << 63) - 1]          # bit 63 stays 0
    assert opk.pack([3] * 8).tolist() == [sum(3 << (9 * j) for j in range(7)), 3]
    assert opk.pack([5, 0, 0, 0, 0, 0, 0, 0, 7]).tolist() == [5, 7 << 9]


def test_kohya_304_size_kat():
    # reference tests/test_kernels.py:57-64: 3,589,632 indices -> 512,805 words = 4,102,440 B
    shapes = ([(3072, 9216)] * 76 + [(3072, 18432)] * 38 + [(3072, 3072)] * 38 + [(3072, 12288)] * 38
              + [(12288, 3072)] * 38 + [(3072, 21504)] * 38 + [(15360, 3072)] * 38)
    mods = [{"name": f"m{i}", "shape_a": [16, a], "shape_b": [b, 16]} for i, (a, b) in enumerate(shapes)]
    lay = opk.layout_of({"modules": mods, "rank": 16, "alpha": 16.0, "num_levels": 3, "block_size": 64})
    assert lay.num_indices == 3_589_632
    assert lay.num_words * 8 == 4_102_440


def test_flux_342_size():
    from helpers import flux_modules
    mods = [{"name": n, "shape_a": [16, a], "shape_b": [b, 16]} for n, a, b in flux_modules()]
    lay = opk.layout_of({"modules": mods, "rank": 16, "alpha": 16.0, "num_levels": 3, "block_size": 64})
    assert len(mods) == 342 and lay.total_blocks == 700_416 and lay.num_indices == 2_101_248
    assert lay.num_words == 300_179 and lay.num_words * 8 == 2_401_432


def test_layout_and_stream_order_closed_form():
    ad = random_adapter(SMALL, rank=16, seed=2)
    lay = opk.layout_of(ad)
    # odd: A (16, 96) = 24 blocks, B (40, 16) = 10 blocks; offsets accumulate A then B per module
    sizes = [(16 * d_in // 64, -(-d_out * 16 // 64)) for _, d_in, d_out in SMALL]
    cursor = 0
    for i, (na, nb) in enumerate(sizes):
        assert lay.a_off[i] == cursor and lay.b_off[i] == cursor + na
        assert (lay.sides[cursor:cursor + na] == 0).all() and (lay.sides[cursor + na:cursor + na + nb] == 1).all()
        cursor += na + nb
    flat = opk.stream_order(ad, lay)
    for i, name in enumerate(lay.names):
        a = ad.indices[name]["A"]
        for blk in (0, 5, a.shape[1] - 1):
            for lev in range(3):
                assert flat[(lay.a_off[i] + blk) * 3 + lev] == a[lev, blk]
    words = opk.pack(flat)
    got_a, got_b = opk.module_levels(words, lay, "odd")
    assert np.array_equal(got_a, ad.indices["odd"]["A"]) and np.array_equal(got_b, ad.indices["odd"]["B"])


def test_numpy_and_c_restatements_agree():
    rng = np.random.default_rng(5)
    for n in (1, 7, 8, 9999):
        v = rng.integers(0, 512, n)
        assert np.array_equal(native.pack(v), opk.pack(v))
        assert np.array_equal(native.unpack(opk.pack(v), n), v)
    with pytest.raises(ValueError):
        native.pack([600])


# ------------------------------------------------------------------ decode
def test_bf16_rounding_matches_torch():
    rng = np.random.default_rng(0)
    x = np.concatenate([rng.standard_normal(100_000).astype(np.float32) * 3,
                        np.array([0.0, -0.0, 1e-40, 3.0e38, 1.00390625, 1.01171875], np.float32)])
    want = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(odec.bf16_bits(x), want)
    assert np.array_equal(native.bf16_bits(x), want)


def test_decode_brute_force_float64():
    """Decode = sum_l sigma_l * (U s_{k_l}) / 3 evaluated from the Hadamard matrix in float64."""
    rng = np.random.default_rng(3)
    idx = rng.integers(0, 512, (3, 64))
    pa, pb = ocb.twin_pools()
    got = odec.rvq_decode(idx, pb)
    u = scipy.linalg.hadamard(64)[:, :9].astype(np.float64)
    for n in range(idx.shape[1]):
        want = np.zeros(64)
        for lev, sig in enumerate(ocb.SIGMA_B):
            s = np.array([1.0 if (idx[lev, n] >> q) & 1 else -1.0 for q in range(9)])
            want += sig * (u @ s) / 3.0
        np.testing.assert_allclose(got[n], want, rtol=0, atol=1e-8)


def test_decode_all_levels_same_index_special_case():
    pa, _ = ocb.twin_pools()
    for k in (0, 1, 255, 511):
        idx = np.full((3, 1), k)
        got = odec.rvq_decode(idx, pa)[0]
        want = 0.18 * ocb.integer_table()[k].astype(np.float64) / 3.0
        np.testing.assert_allclose(got, want, rtol=1e-6)


def test_decode_level_order_is_pinned():
    """(p0 + p1) + p2 in fp32: the reversed order differs in some elements (so order is observable)."""
    rng = np.random.default_rng(9)
    idx = rng.integers(0, 512, (3, 4096))
    _, pb = ocb.twin_pools()
    fwd = odec.rvq_decode(idx, pb)
    rev = (pb[2][idx[2]] + pb[1][idx[1]]) + pb[0][idx[0]]
    assert not np.array_equal(fwd.view(np.uint32), rev.view(np.uint32))
    ref = (pb[0][idx[0]] + pb[1][idx[1]]) + pb[2][idx[2]]
    assert np.array_equal(fwd.view(np.uint32), ref.view(np.uint32))


def test_decode_packed_numpy_vs_c_and_sides():
    ad = random_adapter(SMALL, rank=16, seed=4)
    words, lay = opk.pack_adapter(ad)
    pa, pb = ocb.twin_pools()
    f32 = odec.decode_packed(words, lay, pa, pb)
    c32 = native.decode(words, lay.total_blocks, 3, lay.sides, pa, pb, want="f32")
    assert np.array_equal(f32.view(np.uint32), c32.view(np.uint32))
    assert np.array_equal(odec.bf16_bits(f32), native.decode(words, lay.total_blocks, 3, lay.sides, pa, pb, "bf16"))
    views = odec.split_decoded(f32, lay)
    for m in ad.modules:
        a = odec.decode(ad.indices[m["name"]]["A"], m["shape_a"], pa)
        b = odec.decode(ad.indices[m["name"]]["B"], m["shape_b"], pb)
        assert np.array_equal(views[m["name"]][0], a) and np.array_equal(views[m["name"]][1], b)
    # a wrong side (A pool for a B block) is caught
    wrong = native.decode(words, lay.total_blocks, 3, None, pa, pb, want="f32")
    assert not np.array_equal(wrong, f32)


# ------------------------------------------------------------------ deltas
def _factors(ad, name, d_in, d_out, r):
    pa, pb = ocb.twin_pools()
    return (odec.decode(ad.indices[name]["A"], (r, d_in), pa), odec.decode(ad.indices[name]["B"], (d_out, r), pb))


def test_shared_delta_fp32_equals_decode_then_matmul():
    # reference tests/test_kernels.py:125-136: fp32 path vs decode-then-matmul, rtol 1e-4 / atol 1e-6
    ads = [random_adapter([("l", 128, 64)], rank=16, seed=s) for s in (2, 9)]
    ia = np.stack([a.indices["l"]["A"] for a in ads]).astype(np.int64)
    ib = np.stack([a.indices["l"]["B"] for a in ads]).astype(np.int64)
    x = np.random.default_rng(0).standard_normal((3, 7, 128)).astype(np.float32)
    assign = [1, 0, 1]
    pa, pb = ocb.twin_pools()
    got = odelta.shared_delta(x, ia, pa, ib, pb, assign, 16, 64, 0.5, "fp32")
    facs = [_factors(a, "l", 128, 64, 16) for a in ads]
    want = np.stack([odelta.truth_delta(x[i], *facs[j]) for i, j in enumerate(assign)]) * 0.5
    np.testing.assert_allclose(got, want, rtol=1e-4, atol=1e-6)


def test_shared_delta_bf16_steps_and_planted_transpose():
    ads = [random_adapter([("l", 256, 384)], rank=16, seed=s) for s in range(2)]
    ia = np.stack([a.indices["l"]["A"] for a in ads]).astype(np.int64)
    ib = np.stack([a.indices["l"]["B"] for a in ads]).astype(np.int64)
    x = odec.round_bf16(np.random.default_rng(1).standard_normal((2, 20, 256)).astype(np.float32))
    pa, pb = ocb.twin_pools()
    got = odelta.shared_delta(x, ia, pa, ib, pb, [1, 0], 16, 384, 1.0, "bf16")
    assert np.array_equal(got, odec.round_bf16(got))                       # output is bf16-valued
    facs = [_factors(a, "l", 256, 384, 16) for a in ads]
    truth = np.stack([odelta.truth_delta(x[i], *facs[j]) for i, j in enumerate([1, 0])])
    assert np.linalg.norm(got - truth) / np.linalg.norm(truth) < 2e-2     # the reference's truth bound
    # swapping the adapters (a routing mistake) is far outside that bound
    bad = np.stack([odelta.truth_delta(x[i], *facs[j]) for i, j in enumerate([0, 1])])
    assert np.linalg.norm(bad - truth) / np.linalg.norm(truth) > 0.5


def test_serve_forward_closed_form_with_mixture_and_empty():
    # reference tests/test_serve.py:28-46 with the same routes
    ads = [random_adapter([("fc", 128, 64)], rank=4, seed=s) for s in range(3)]
    for a in ads:
        a.alpha = 8.0
    x = np.random.default_rng(0).standard_normal((5, 10, 128)).astype(np.float32)
    base = np.random.default_rng(1).standard_normal((5, 10, 64)).astype(np.float32)
    routes = [[(0, 1.0)], [(2, 1.0)], [], [(1, 0.6), (2, 0.4)], [(0, 1.0)]]
    ids = np.full((5, 2), -1)
    w = np.zeros((5, 2), np.float32)
    for i, r in enumerate(routes):
        for j, (a, wt) in enumerate(r):
            ids[i, j], w[i, j] = a, wt
    ia = np.stack([a.indices["fc"]["A"] for a in ads])
    ib = np.stack([a.indices["fc"]["B"] for a in ads])
    pa, pb = ocb.twin_pools()
    got = odelta.serve_forward(x, base, ids, w, ia, ib, np.full(3, 2.0, np.float32), pa, pb, 4, "fp32")
    facs = [_factors(a, "fc", 128, 64, 4) for a in ads]
    for i, r in enumerate(routes):
        want = base[i].astype(np.float64)
        for a_id, wt in r:
            want = want + wt * odelta.truth_delta(x[i], *facs[a_id]) * 2.0
        np.testing.assert_allclose(got[i], want, atol=1e-6)
    # dropping the sqrt (weighting each factor by w instead of sqrt(w)) breaks the mixture sample
    a1, b1 = facs[1]
    a2, b2 = facs[2]
    wrong = base[3] + (0.36 * odelta.truth_delta(x[3], a1, b1) + 0.16 * odelta.truth_delta(x[3], a2, b2)) * 2.0
    assert np.abs(got[3] - wrong).max() > 1e-3


def test_per_sample_delta_matches_einsum():
    # reference tests/test_kernels.py:116-122
    rng = np.random.default_rng(0)
    x, a, b = rng.standard_normal((3, 5, 32)), rng.standard_normal((3, 4, 32)), rng.standard_normal((3, 24, 4))
    s = np.array([0.5, 1.0, 2.0])
    want = np.einsum("bsd,brd,bor->bso", x, a, b) * s[:, None, None]
    np.testing.assert_allclose(odelta.per_sample_delta(x, a, b, s, "fp32"), want, rtol=1e-5, atol=1e-5)
    got16 = odelta.per_sample_delta(odec.round_bf16(x * 0.5), a * 0.02, b * 0.02, s, "bf16")
    truth = np.einsum("bsd,brd,bor->bso", odec.round_bf16(x * 0.5), odec.round_bf16(a * 0.02),
                      odec.round_bf16(b * 0.02)) * s[:, None, None]
    assert np.linalg.norm(got16 - truth) / np.linalg.norm(truth) < 1e-2


def _lithe_linear_case(scaling):
    rng = np.random.default_rng(11)
    d_in, d_out, r = 192, 320, 16
    ad = random_adapter([("l", d_in, d_out)], rank=r, seed=6)
    a, b = _factors(ad, "l", d_in, d_out, r)
    x = odec.round_bf16(rng.standard_normal((3, 40, d_in)).astype(np.float32))
    base = odec.round_bf16(rng.standard_normal((3, 40, d_out)).astype(np.float32) * 0.01)
    return x, base, a, b


def test_lithe_linear_fp32_closed_form_and_planted_mistakes():
    """lithe/module.py:154-156 in fp32: base + (x A^T) B^T * scaling, against the float64 closed form.
    A dropped scaling, a doubled scaling and B read as an (r, d_out) matrix all fail the check."""
    s = 1.5                                              # alpha / r = 24 / 16
    x, base, a, b = _lithe_linear_case(s)
    truth = base.astype(np.float64) + s * odelta.truth_delta(x, a, b)
    got = odelta.lithe_linear(x, base, a, b, s, "fp32")
    np.testing.assert_allclose(got, truth, rtol=0, atol=1e-6)
    r, d_out = a.shape[0], b.shape[0]
    for wrong in (odelta.lithe_linear(x, base, a, b, 1.0, "fp32"),
                  odelta.lithe_linear(x, base, a, b, s * s, "fp32"),
                  odelta.lithe_linear(x, base, a, b.reshape(r, d_out).T.copy(), s, "fp32")):
        assert np.abs(wrong - truth).max() > 1e-3


def test_lithe_linear_bf16_equals_torch_cpu_ops_and_truth_bound():
    """lithe/module.py:154-156 in bf16, evaluated by torch's own CPU ops (F.linear twice, the
    bf16 multiply by the scaling, the bf16 add): the oracle's rounding points give the same bits.
    With a zero base the delta stays within the reference's 2e-2 truth bound
    (tests/test_kernels.py:216 of the reference). An oracle that kept x A^T unrounded, or
    skipped the rounding of delta * scaling, would differ in more than a fifth of the outputs."""
    import torch.nn.functional as F
    s = 1.5
    x, base, a, b = _lithe_linear_case(s)
    tx, ta, tb, tbase = (torch.from_numpy(np.ascontiguousarray(v)).bfloat16() for v in (x, a, b, base))
    want = (tbase + F.linear(F.linear(tx, ta), tb) * s).float().numpy()
    got = odelta.lithe_linear(x, base, a, b, s, "bf16")
    differ = got != want
    assert differ.mean() < 1e-3                          # torch's fp32 accumulation order may flip a rare tie
    if differ.any():
        from helpers import bf16_ulp
        assert (np.abs(got - want) <= bf16_ulp(want)).all()
    zero = np.zeros_like(base)
    d = odelta.lithe_linear(x, zero, a, b, s, "bf16")
    truth = s * odelta.truth_delta(x, a, b)
    assert np.linalg.norm(d - truth) / np.linalg.norm(truth) < 2e-2
    ar, br = odec.round_bf16(a).astype(np.float64), odec.round_bf16(b).astype(np.float64)
    mid_unrounded = odec.round_bf16(odec.round_bf16((x.astype(np.float64) @ ar.T) @ br.T) * np.float32(s))
    mid = odec.round_bf16(x.astype(np.float64) @ ar.T).astype(np.float64)
    scale_unrounded = odec.round_bf16(mid @ br.T) * np.float32(s)
    for wrong in (odec.round_bf16(base + mid_unrounded), odec.round_bf16(base + scale_unrounded)):
        assert (wrong != want).mean() > 0.2


def test_index_linear_bit_exact_with_torch_add():
    """lithe/kernels/layers.py:131: ``out + delta`` with both in the activation dtype is torch's
    bf16 (or fp32) add; the oracle gives the same bits. Leaving the sum unrounded fails."""
    rng = np.random.default_rng(12)
    base = odec.round_bf16(rng.standard_normal((4, 33, 96)).astype(np.float32))
    delta = odec.round_bf16(rng.standard_normal((4, 33, 96)).astype(np.float32) * 0.02)
    want = (torch.from_numpy(base).bfloat16() + torch.from_numpy(delta).bfloat16()).float().numpy()
    got = odelta.index_linear(base, delta, "bf16")
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    assert (base + delta != want).mean() > 0.2
    b32 = rng.standard_normal((4, 33, 96)).astype(np.float32)
    d32 = rng.standard_normal((4, 33, 96)).astype(np.float32) * 0.02
    want32 = (torch.from_numpy(b32) + torch.from_numpy(d32)).numpy()
    assert np.array_equal(odelta.index_linear(b32, d32, "fp32").view(np.uint32), want32.view(np.uint32))


def test_torch_cpu_serving_path_equals_serve_forward():
    """oracle.torch_cpu (the CPU baseline: the reference's serve.py forward in torch CPU ops) gives
    the pinned numpy restatement's numbers: fp32 to accumulation-order precision, bf16 to within
    one bf16 ulp in a small fraction of the outputs (torch's bmm accumulates in fp32)."""
    from oracle import torch_cpu
    from helpers import ulp_stats
    ads = [random_adapter([("fc", 192, 128)], rank=8, seed=s) for s in range(3)]
    routes = [[(0, 1.0)], [(2, 1.0)], [], [(1, 0.6), (2, 0.4)], [(0, 1.0)]]
    ids = np.full((5, 2), -1)
    w = np.zeros((5, 2), np.float32)
    for i, r in enumerate(routes):
        for j, (a, wt) in enumerate(r):
            ids[i, j], w[i, j] = a, wt
    ia = np.stack([a.indices["fc"]["A"] for a in ads])
    ib = np.stack([a.indices["fc"]["B"] for a in ads])
    scales = np.array([2.0, 0.5, 1.5], np.float32)
    pa, pb = ocb.twin_pools()
    rng = np.random.default_rng(2)
    x = odec.round_bf16(rng.standard_normal((5, 12, 192)).astype(np.float32))
    base = odec.round_bf16(rng.standard_normal((5, 12, 128)).astype(np.float32) * 0.05)
    args = (torch.from_numpy(ids), torch.from_numpy(w), [torch.from_numpy(v.astype(np.int64)) for v in ia],
            [torch.from_numpy(v.astype(np.int64)) for v in ib], torch.from_numpy(scales), torch.from_numpy(pa),
            torch.from_numpy(pb), 8)
    got32 = torch_cpu.routed_add(torch.from_numpy(x), torch.from_numpy(base), *args).numpy()
    want32 = odelta.serve_forward(x, base, ids, w, ia, ib, scales, pa, pb, 8, "fp32")
    np.testing.assert_allclose(got32, want32, rtol=0, atol=1e-6)
    got16 = torch_cpu.routed_add(torch.from_numpy(x).bfloat16(), torch.from_numpy(base).bfloat16(), *args)
    want16 = odelta.serve_forward(x, base, ids, w, ia, ib, scales, pa, pb, 8, "bf16")
    max_ulp, frac = ulp_stats(got16.float().numpy(), want16)
    assert max_ulp <= 1.0 and frac < 0.02, (max_ulp, frac)
    assert np.array_equal(got16[2].float().numpy(), base[2])           # the empty route
