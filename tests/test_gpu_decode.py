"""GPU parity of the 9-bit unpack / pack and the bulk decode against the oracle (bit-exact)."""
import numpy as np
import pytest
import torch

import lithe_amd
from lithe_amd import quant
from lithe_amd.kernels import (PackedBank, decode_int16, decode_packed, decode_packed_slots, flat_indices,
                               pack_adapter, pack_indices, split_decoded, unpack_indices)
from oracle import codebook as ocb
from oracle import decode as odec
from oracle import native
from oracle import packing as opk

from helpers import SMALL, flux_modules, random_adapter

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("n", [1, 6, 7, 8, 700, 1001, 2_101_248])
def test_unpack_bit_exact(n):
    v = np.random.default_rng(n).integers(0, 512, n)
    words = opk.pack(v)
    w = torch.from_numpy(words.view(np.int64)).cuda()
    got = unpack_indices(w, n).cpu().numpy()
    assert np.array_equal(got, v)
    for dt in (torch.int32, torch.int16):
        assert np.array_equal(unpack_indices(w, n, dtype=dt).cpu().numpy().astype(np.int64), v)


def test_device_pack_matches_oracle_and_rejects_512():
    v = np.random.default_rng(3).integers(0, 512, 12345)
    for dt in (torch.int16, torch.int32, torch.int64):
        got = pack_indices(torch.from_numpy(v).to(dt).cuda())
        assert np.array_equal(got.view(torch.int64).cpu().numpy().view(np.uint64), opk.pack(v))
    with pytest.raises(ValueError):
        pack_indices(torch.tensor([3, 512, 1], device="cuda"))
    with pytest.raises(ValueError):
        pack_indices(torch.tensor([-1], device="cuda"))


def _oracle_decode_bits(ad):
    words, lay = opk.pack_adapter(ad)
    pa, pb = ocb.twin_pools()
    f32 = odec.decode_packed(words, lay, pa, pb)
    return f32, odec.bf16_bits(f32), lay


@pytest.mark.parametrize("mods,rank,seed", [(SMALL, 16, 4), (SMALL + [("wide", 3072, 9216)], 16, 4),
                                            (SMALL, 8, 3), (SMALL, 4, 1)])
def test_decode_packed_bit_exact(mods, rank, seed):
    ad = random_adapter(mods, rank=rank, seed=seed)
    f32, bits, _ = _oracle_decode_bits(ad)
    words, layout = pack_adapter(ad)
    pa, pb = (p.cuda() for p in lithe_amd.twin_pools())
    w = words.cuda()
    out = decode_packed(w, layout, pa, pb)
    assert out.dtype == torch.bfloat16 and out.shape == (layout.total_blocks, 64)
    assert np.array_equal(out.view(torch.int16).cpu().numpy().view(np.uint16), bits)
    out32 = decode_packed(w, layout, pa, pb, dtype=torch.float32)
    assert np.array_equal(out32.cpu().numpy().view(np.uint32), f32.view(np.uint32))
    # int16 block-major source decodes identically (the reference's residency A/B check)
    idx16 = torch.from_numpy(flat_indices(ad, layout).astype(np.int16)).view(-1, layout.num_levels).cuda()
    assert torch.equal(decode_int16(idx16, layout, pa, pb), out)
    # per-module views equal quant.decode -> bf16 (tests/test_kernels.py:166-179 of the reference)
    got = split_decoded(out, layout)
    pa_np, pb_np = ocb.twin_pools()
    for m in ad.modules:
        a = odec.decode(ad.indices[m["name"]]["A"], m["shape_a"], pa_np)
        b = odec.decode(ad.indices[m["name"]]["B"], m["shape_b"], pb_np)
        assert np.array_equal(got[m["name"]][0].view(torch.int16).cpu().numpy().view(np.uint16), odec.bf16_bits(a))
        assert np.array_equal(got[m["name"]][1].view(torch.int16).cpu().numpy().view(np.uint16), odec.bf16_bits(b))


def test_decode_full_flux_layout_matches_c_oracle():
    """All 342 FLUX linears of one rank-16 adapter (700,416 blocks), against the C restatement."""
    ad = random_adapter(flux_modules(), rank=16, seed=11)
    words, layout = pack_adapter(ad)
    assert layout.total_blocks == 700_416 and layout.num_words == 300_179
    pa, pb = ocb.twin_pools()
    ref_bits = native.decode(words.view(torch.int64).numpy().view(np.uint64), layout.total_blocks, 3,
                             layout.sides.numpy(), pa, pb, want="bf16")
    out = decode_packed(words.cuda(), layout, *(p.cuda() for p in lithe_amd.twin_pools()))
    assert np.array_equal(out.view(torch.int16).cpu().numpy().view(np.uint16), ref_bits)


def test_quant_decode_fp32_exact_and_levels():
    rng = np.random.default_rng(7)
    for L in (1, 2, 3, 4):
        scales = [0.06, 0.03, 0.01, 0.005][:L]
        pools = ocb.pools(scales)
        idx = rng.integers(0, 512, (L, 777))
        want = odec.rvq_decode(idx, pools)
        got = quant.rvq_decode_blocks(torch.from_numpy(idx).cuda(), torch.from_numpy(pools).cuda())
        assert np.array_equal(got.cpu().numpy().view(np.uint32), want.view(np.uint32)), L
        # 7 x 7103 = 49,721 values: 777 blocks, the last one zero-padded
        w = quant.decode(torch.from_numpy(idx).cuda(), (7, 7103), torch.from_numpy(pools).cuda())
        assert w.shape == (7, 7103)
        assert np.array_equal(w.cpu().numpy().view(np.uint32),
                              odec.decode(idx, (7, 7103), pools).view(np.uint32))


def test_bank_multi_slot_decode():
    ads = [random_adapter(SMALL, rank=16, seed=s) for s in range(5)]
    bank, words = PackedBank.from_adapters(ads, "cuda")
    for w in words:
        bank.add(w)
    slots = torch.tensor([4, 0, 2, 2], dtype=torch.int32, device="cuda")
    out = bank.decode_slots(slots)
    for i, s in enumerate([4, 0, 2, 2]):
        _, bits, _ = _oracle_decode_bits(ads[s])
        assert np.array_equal(out[i].view(torch.int16).cpu().numpy().view(np.uint16), bits)
    dec = bank.decode(1)
    want = split_decoded(decode_packed(words[1].cuda(), bank.layout, bank.pool_a, bank.pool_b), bank.layout)
    for name in want:
        assert torch.equal(dec[name][0], want[name][0]) and torch.equal(dec[name][1], want[name][1])


def test_bank_random_fill_fields_in_range():
    ad = random_adapter(SMALL, rank=16, seed=1)
    bank, words = PackedBank.from_adapters([ad], "cuda")
    bank.add(words[0])
    bank.fill_random(7, generator=torch.Generator(device="cuda").manual_seed(0))
    assert bank.num_slots == 7
    w = bank.words.cpu().numpy().view(np.uint64)
    assert (w >> np.uint64(63) == 0).all()
    n = bank.layout.num_indices
    fields = opk.unpack(w[3], bank.layout.num_words * 7)
    assert (fields[n:] == 0).all() and fields[:n].max() <= 511


def test_decode_bad_slot_zero_fills_and_flags():
    """lithe_decode through the C ABI: a slot id outside the bank decodes to zeros and sets
    bit 1 of the error word; the valid selections beside it stay bit-exact."""
    import ctypes

    from lithe_amd.kernels import _delta, _hip
    ads = [random_adapter(SMALL, rank=16, seed=s) for s in range(3)]
    bank, words = PackedBank.from_adapters(ads, "cuda")
    for w in words:
        bank.add(w)
    lay = bank.layout
    sel = [2, 7, -1, 0]
    out = torch.full((len(sel), lay.total_blocks, 64), 3.0, dtype=torch.bfloat16, device="cuda")
    err = torch.zeros(1, dtype=torch.int32, device="cuda")
    src = _delta.packed_source(bank.words, lay.num_levels, 0)
    lut_a = _hip.lut_from_pools(bank.pool_a, torch.float32)
    lut_b = _hip.lut_from_pools(bank.pool_b, torch.float32)
    slots = torch.tensor(sel, dtype=torch.int32, device="cuda")
    rc = _hip.load().lithe_decode(ctypes.byref(src), _hip.ptr(slots), len(sel), lay.total_blocks,
                                  _hip.ptr(lay.sides_on("cuda")), ctypes.byref(lut_a), ctypes.byref(lut_b),
                                  _hip.ptr(out), _hip.dtype_code(out.dtype), lay.total_blocks * 64, _hip.ptr(err),
                                  _hip.stream_of(out.device))
    assert rc == 0
    torch.cuda.synchronize()
    assert int(err.item()) & 1
    for i, s in enumerate(sel):
        got = out[i].view(torch.int16).cpu().numpy().view(np.uint16)
        if 0 <= s < 3:
            _, bits, _ = _oracle_decode_bits(ads[s])
            assert np.array_equal(got, bits), i
        else:
            assert not got.any(), i      # bf16 +0.0 everywhere


def test_decode_side_table_unaligned_and_tail():
    """The packed decode reads a workgroup's 3,072 side bytes with 4-byte loads where it can; a
    side table at an odd address and the partial last workgroup take the byte path. Both forms
    give the oracle's bits: a layout of 3,082 blocks (one whole workgroup and a tail) at an
    aligned and an odd address here; the rank-64 FLUX layout in the next test."""
    from lithe_amd.kernels import _delta
    from lithe_amd.kernels.packed import _decode
    ad = random_adapter([("m0", 1024, 1024), ("m1", 1024, 2048), ("m2", 512, 2600), ("m3", 2048, 2048)], rank=16,
                        seed=4)
    _, bits, _ = _oracle_decode_bits(ad)
    words, layout = pack_adapter(ad)
    n = layout.total_blocks
    assert n % 3072 != 0 and n > 3072
    pa, pb = (p.cuda() for p in lithe_amd.twin_pools())
    w = words.cuda()
    aligned = decode_packed(w, layout, pa, pb)
    assert np.array_equal(aligned.view(torch.int16).cpu().numpy().view(np.uint16), bits)
    buf = torch.zeros(n + 1, dtype=torch.int8, device="cuda")
    buf[1:].copy_(layout.sides.cuda())
    odd = buf[1:]
    assert odd.data_ptr() % 4 != 0
    s = _delta.packed_source(w.view(1, -1), layout.num_levels, 0)
    out = torch.empty((n, 64), dtype=torch.bfloat16, device="cuda")
    _decode(s, n, odd, pa, pb, out)
    assert torch.equal(out, aligned)


def test_decode_rank64_flux_layout_staged_sides():
    """The rank-64 FLUX layout plus one small module (2,801,768 blocks, a partial last
    workgroup) against the C restatement, aligned and at an odd side-table address."""
    from lithe_amd.kernels import _delta
    from lithe_amd.kernels.packed import _decode
    ad = random_adapter(flux_modules() + [("extra", 64, 40)], rank=64, seed=12)
    words, layout = pack_adapter(ad)
    n = layout.total_blocks
    assert n == 2_801_768 and n % 3072 != 0
    pa, pb = ocb.twin_pools()
    ref_bits = native.decode(words.view(torch.int64).numpy().view(np.uint64), n, 3,
                             layout.sides.numpy(), pa, pb, want="bf16")
    pa_t, pb_t = (p.cuda() for p in lithe_amd.twin_pools())
    w = words.cuda()
    out = decode_packed(w, layout, pa_t, pb_t)
    assert np.array_equal(out.view(torch.int16).cpu().numpy().view(np.uint16), ref_bits)
    buf = torch.zeros(n + 1, dtype=torch.int8, device="cuda")
    buf[1:].copy_(layout.sides.cuda())
    out2 = torch.empty_like(out)
    _decode(_delta.packed_source(w.view(1, -1), layout.num_levels, 0), n, buf[1:], pa_t, pb_t, out2)
    assert torch.equal(out2, out)


def test_decode_factors_equals_oracle_decode():
    """lithe_amd.decode_factors (one packed decode of the whole adapter, split into per-module
    views) gives every factor of the oracle's fp32 level-order decode bit for bit, the
    non-multiple-of-64 module included."""
    import lithe_amd
    from helpers import SMALL, random_adapter
    ad = random_adapter(SMALL, rank=16, seed=31)
    got = lithe_amd.decode_factors(ad)
    pa, pb = ocb.twin_pools()
    for m in ad.modules:
        a, b = got[m["name"]]
        want_a = odec.decode(ad.indices[m["name"]]["A"], m["shape_a"], pa)
        want_b = odec.decode(ad.indices[m["name"]]["B"], m["shape_b"], pb)
        assert a.dtype == torch.float32 and tuple(a.shape) == tuple(m["shape_a"])
        assert np.array_equal(a.cpu().numpy().view(np.uint32), want_a.view(np.uint32)), m["name"]
        assert np.array_equal(b.cpu().numpy().view(np.uint32), want_b.view(np.uint32)), m["name"]
