"""CPU checks of the bank-ingest path: the oracle's .lithe stream split, the segment table
and the host reorder-and-pack of the C ABI (lithe_ingest_table / lithe_ingest_host), bit-exact
against the oracle's residency order and packer."""
import ctypes

import numpy as np
import pytest

from lithe_amd import fileio
from lithe_amd.kernels import PackedLayout, _hip
from oracle import packing as opk

from helpers import SMALL, flux_modules, random_adapter


def _p(a):
    return a.ctypes.data_as(ctypes.c_void_p)


def _table(modules, levels):
    ba = np.array([opk.num_blocks(m["shape_a"]) for m in modules], np.int64)
    bb = np.array([opk.num_blocks(m["shape_b"]) for m in modules], np.int64)
    t = np.zeros((2 * len(modules), 3), np.int64)
    assert _hip.load().lithe_ingest_table(len(modules), _p(ba), _p(bb), levels, _p(t)) == 0
    return t


def _host_ingest(stream, modules, levels):
    s = np.ascontiguousarray(stream, np.uint16)
    t = _table(modules, levels)
    nw = -(-s.size // 7)
    words = np.full(nw + 2, 0xDEAD, np.uint64)      # two extra words: zero-padded by the call
    rc = _hip.load().lithe_ingest_host(_p(s), s.size, levels, t.shape[0], _p(t), _p(words), nw + 2)
    return rc, words


def test_oracle_split_inverts_the_file_stream():
    """The oracle split of a .lithe stream gives back the per-module matrices the stream was made
    of (lithe/fileio.py:53-56 builds the stream, :136-150 splits it) and, reordered, the
    residency order of pack_adapter; a tiny hand case pins the order itself."""
    ad = random_adapter(SMALL, rank=16, seed=3)
    stream = np.frombuffer(ad.raw_stream(), "<u2")
    parts = opk.split_file_stream(stream, ad.modules, 3)
    for m in ad.modules:
        for side in "AB":
            assert np.array_equal(parts[m["name"]][side], ad.indices[m["name"]][side])
    assert np.array_equal(opk.residency_from_file_stream(stream, ad.modules, 3),
                          opk.stream_order(ad, opk.layout_of(ad)))
    # hand case: one module, A = 1 block, B = 2 blocks, L = 2. Stream: A(L=2, n=1) then B(L=2, n=2).
    mods = [{"name": "m", "shape_a": [1, 64], "shape_b": [2, 64]}]
    stream = np.array([10, 11,            # A level 0, level 1
                       20, 21, 30, 31],   # B level 0 (blocks 0, 1), level 1 (blocks 0, 1)
                      np.uint16)
    # residency: block-major, level inside: A0(l0, l1), B0(l0, l1), B1(l0, l1)
    assert opk.residency_from_file_stream(stream, mods, 2).tolist() == [10, 11, 20, 30, 21, 31]
    with pytest.raises(ValueError):
        opk.split_file_stream(stream[:-1], mods, 2)


def test_ingest_table_matches_layout():
    ad = random_adapter(SMALL, rank=16, seed=1)
    lay = PackedLayout.from_adapter(ad)
    t = _table(ad.modules, 3)
    total_a = sum(opk.num_blocks(m["shape_a"]) for m in ad.modules)
    off_a, off_b = 0, 3 * total_a
    for i, m in enumerate(ad.modules):
        na, nb = opk.num_blocks(m["shape_a"]), opk.num_blocks(m["shape_b"])
        assert t[2 * i].tolist() == [lay.a_off[i], na, off_a]
        assert t[2 * i + 1].tolist() == [lay.b_off[i], nb, off_b]
        off_a += 3 * na
        off_b += 3 * nb
    assert np.array_equal(lay.ingest_table().numpy(), t)


@pytest.mark.parametrize("mods,rank,levels,seed", [(SMALL, 16, 3, 0), (SMALL, 4, 2, 1), (SMALL, 8, 4, 2),
                                                   (flux_modules()[:14], 16, 3, 3), (flux_modules(), 16, 3, 4)])
def test_host_ingest_matches_oracle(mods, rank, levels, seed):
    ad = random_adapter(mods, rank=rank, seed=seed, levels=levels)
    stream = np.frombuffer(ad.raw_stream(), "<u2")
    rc, words = _host_ingest(stream, ad.modules, levels)
    assert rc == 0
    want = opk.pack(opk.residency_from_file_stream(stream, ad.modules, levels))
    assert np.array_equal(words[:want.size], want)
    assert (words[want.size:] == 0).all()


def test_host_ingest_rejects_bad_streams():
    ad = random_adapter(SMALL, rank=16, seed=5)
    stream = np.frombuffer(ad.raw_stream(), "<u2").copy()
    stream[123] = 512
    rc, words = _host_ingest(stream, ad.modules, 3)
    assert rc == _hip.ERR_RANGE and (words == 0xDEAD).all()      # nothing written
    t = _table(ad.modules, 3)
    s = np.frombuffer(ad.raw_stream(), "<u2").copy()
    w = np.zeros(-(-s.size // 7), np.uint64)
    lib = _hip.load()
    assert lib.lithe_ingest_host(_p(s), s.size - 1, 3, t.shape[0], _p(t), _p(w), w.size) == _hip.ERR_SHAPE
    bad = t.copy()
    bad[3, 0] += 1                                               # a gap in the residency order
    assert lib.lithe_ingest_host(_p(s), s.size, 3, t.shape[0], _p(bad), _p(w), w.size) == _hip.ERR_SHAPE
    assert lib.lithe_ingest_host(_p(s), s.size, 3, t.shape[0], _p(t), _p(w), w.size - 1) == _hip.ERR_SHAPE
    assert lib.lithe_ingest_host(_p(s), s.size, 5, t.shape[0], _p(t), _p(w), w.size) == _hip.ERR_LEVELS


def test_read_stream_round_trip(tmp_path):
    ad = random_adapter(SMALL, rank=16, seed=6)
    path = tmp_path / "a.lithe"
    fileio.save_lithe(path, ad)
    header, stream = fileio.read_stream(path)
    assert stream.tobytes() == ad.raw_stream()
    lay = PackedLayout.from_adapter(ad)
    assert lay.matches_modules(header["modules"], header["codebook"]["num_levels"], header["codebook"]["block_size"])
    assert not lay.matches_modules(header["modules"][:-1], 3, 64)
