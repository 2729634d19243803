"""GPU checks of bank ingest (cold swap): .lithe file or raw index blob -> resident slot, packed
on the GPU straight into the bank (lithe_ingest / lithe_pack9), bit-exact against the oracle's
split + residency order + packer; the slot allocator; a delta served from an ingested slot."""
import ctypes

import numpy as np
import pytest
import torch

from lithe_amd import fileio
from lithe_amd.kernels import PackedBank, PackedLayout, _hip, packed_lora_delta
from oracle import packing as opk

from helpers import SMALL, flux_modules, random_adapter

pytestmark = pytest.mark.gpu


def _want_words(ad):
    stream = np.frombuffer(ad.raw_stream(), "<u2")
    return opk.pack(opk.residency_from_file_stream(stream, ad.modules, ad.num_levels))


def _slot_words(bank, slot):
    return bank.words[slot].cpu().numpy().view(np.uint64)


@pytest.mark.parametrize("mods", [SMALL, flux_modules()])
def test_load_lithe_device_and_host_match_oracle(tmp_path, mods):
    ads = [random_adapter(mods, rank=16, seed=20 + s) for s in range(3)]
    paths = []
    for i, ad in enumerate(ads):
        paths.append(tmp_path / f"a{i}.lithe")
        fileio.save_lithe(paths[-1], ad)
    bank = PackedBank(PackedLayout.from_adapter(ads[0]), "cuda", capacity=4)
    s0 = bank.load_lithe(paths[0])                       # device reorder + pack
    s1 = bank.load_lithe(paths[1], on_device=False)      # host packer
    s2 = bank.load_lithe(paths[2])
    torch.cuda.synchronize()
    assert (s0, s1, s2) == (0, 1, 2) and bank.ingest_errors() == 0
    for s, ad in zip((s0, s1, s2), ads):
        assert np.array_equal(_slot_words(bank, s), _want_words(ad)), s
    # reload into an occupied slot: overwritten in place
    assert bank.load_lithe(paths[2], slot=0) == 0
    torch.cuda.synchronize()
    assert np.array_equal(_slot_words(bank, 0), _want_words(ads[2]))


def test_load_blob_matches_oracle(tmp_path):
    ad = random_adapter(flux_modules()[:20], rank=16, seed=7)
    lay = PackedLayout.from_adapter(ad)
    blob = tmp_path / "a.int16.bin"
    opk.stream_order(ad, opk.layout_of(ad)).astype(np.int16).tofile(blob)   # serving/bench_hotswap.py:100-104
    bank = PackedBank(lay, "cuda", capacity=2)
    s = bank.load_blob(blob)
    torch.cuda.synchronize()
    assert np.array_equal(_slot_words(bank, s), _want_words(ad))


def test_slot_allocator_reuses_freed_slots(tmp_path):
    ads = [random_adapter(SMALL, rank=16, seed=30 + s) for s in range(4)]
    bank = PackedBank(PackedLayout.from_adapter(ads[0]), "cuda", capacity=2)
    slots = [bank.load_stream(np.frombuffer(ad.raw_stream(), "<u2")) for ad in ads[:3]]
    assert slots == [0, 1, 2] and bank.num_slots == 3          # grew past the initial capacity
    bank.free(1)
    assert bank.num_free == 1
    with pytest.raises(ValueError):
        bank.free(1)
    with pytest.raises(IndexError):
        bank.free(7)
    assert bank.load_stream(np.frombuffer(ads[3].raw_stream(), "<u2")) == 1    # the freed slot
    torch.cuda.synchronize()
    for s, ad in zip((0, 1, 2), (ads[0], ads[3], ads[2])):
        assert np.array_equal(_slot_words(bank, s), _want_words(ad)), s
    with pytest.raises(ValueError):
        bank.load_stream(np.zeros(5, np.uint16))
    bad = np.frombuffer(ads[0].raw_stream(), "<u2").copy()
    bad[3] = 600
    with pytest.raises(ValueError):
        bank.load_stream(bad, slot=0)


def test_device_ingest_flags_a_table_outside_the_stream():
    """A table whose offsets point past the stream: the kernel reads nothing out of range,
    packs index 0 there and sets bit 2 of the error word."""
    ad = random_adapter(SMALL, rank=16, seed=9)
    lay = PackedLayout.from_adapter(ad)
    stream = torch.from_numpy(np.frombuffer(ad.raw_stream(), "<u2").view(np.int16).copy()).cuda()
    table = lay.ingest_table().clone()
    table[-1, 2] += 10_000                      # last factor starts past the end of the stream
    tdev = table.cuda()
    words = torch.zeros(lay.num_words, dtype=torch.int64, device="cuda")
    err = torch.zeros(1, dtype=torch.int32, device="cuda")
    rc = _hip.load().lithe_ingest(_hip.ptr(stream), stream.numel(), 3, table.shape[0], _hip.ptr(tdev),
                                  _hip.ptr(words), lay.num_words, _hip.ptr(err), _hip.stream_of(stream.device))
    assert rc == 0
    torch.cuda.synchronize()
    assert int(err.item()) == 2
    want = _want_words(ad)
    got = words.cpu().numpy().view(np.uint64)
    first_bad = (lay.b_off[-1] * 3) // 7     # words before the last factor are untouched by the bad row
    assert np.array_equal(got[:first_bad], want[:first_bad])


def test_delta_from_ingested_slot_matches_prebuilt_slot(tmp_path):
    mods = [("q", 3072, 3072), ("up", 3072, 12288)]
    ads = [random_adapter(mods, rank=16, seed=40 + s) for s in range(2)]
    bank, words = PackedBank.from_adapters(ads, "cuda")
    for w in words:
        bank.add(w)
    path = tmp_path / "b.lithe"
    fileio.save_lithe(path, ads[1])
    s = bank.load_lithe(path)                # slot 2: same adapter as slot 1, ingested from disk
    assert s == 2
    _, _, _, a_off, b_off = bank.layout.module("up")
    x = torch.randn(2, 40, 3072, generator=torch.Generator().manual_seed(0)).bfloat16().cuda()
    pools = (bank.pool_a.bfloat16(), bank.pool_b.bfloat16())
    outs = []
    for slot in (1, 2):
        y = torch.zeros(2, 40, 12288, dtype=torch.bfloat16, device="cuda")
        packed_lora_delta(x, bank.words, a_off, b_off, 3, pools, torch.tensor([slot, slot], device="cuda"), 16,
                          12288, 1.0, out=y, accumulate=True)
        outs.append(y)
    torch.cuda.synchronize()
    assert torch.equal(outs[0], outs[1])
