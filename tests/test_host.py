"""CPU checks of the host logic around the kernels: layout / stream order / packing against
the oracle, .lithe file I/O, routing tables, value tables from pools, and the reference's
own host-side known answers (parse_route cases, FLUX target count, codebook hash)."""
import numpy as np
import pytest
import torch

import lithe_amd
from lithe_amd import codebook as cb
from lithe_amd import fileio, module, quant, serve
from lithe_amd.kernels import _hip
from lithe_amd.kernels.packed import PackedLayout, flat_indices, pack_adapter
from oracle import codebook as ocb
from oracle import packing as opk

from helpers import SMALL, flux_modules, random_adapter


@pytest.mark.parametrize("mods,rank", [(SMALL, 16), (SMALL, 4), (flux_modules(), 16)])
def test_layout_matches_oracle(mods, rank):
    ad = random_adapter(mods, rank=rank, seed=2)
    lay = PackedLayout.from_adapter(ad)
    ref = opk.layout_of(ad)
    assert lay.names == ref.names and lay.a_off == ref.a_off and lay.b_off == ref.b_off
    assert lay.shapes_a == ref.shapes_a and lay.shapes_b == ref.shapes_b
    assert np.array_equal(lay.sides.numpy(), ref.sides)
    assert lay.num_words == ref.num_words and lay.scaling == ref.scaling
    assert lay.matches(ad)


def test_stream_order_and_words_match_oracle():
    ad = random_adapter(SMALL + [("wide", 3072, 9216)], rank=16, seed=5)
    lay = PackedLayout.from_adapter(ad)
    assert np.array_equal(flat_indices(ad, lay).astype(np.int64), opk.stream_order(ad, opk.layout_of(ad)))
    words, lay2 = pack_adapter(ad)
    ref_words, _ = opk.pack_adapter(ad)
    assert words.dtype == torch.uint64 and words.device.type == "cpu"   # reference: CPU uint64 tensor
    assert np.array_equal(words.view(torch.int64).numpy().view(np.uint64), ref_words)
    # a layout from another adapter with the same modules packs identically
    words3, _ = pack_adapter(ad, lay2)
    assert torch.equal(words3.view(torch.int64), words.view(torch.int64))


def test_flux_342_layout_sizes():
    """700,416 blocks = 2,101,248 indices = 300,179 words = 2,401,432 B per rank-16 adapter."""
    lay = PackedLayout.from_modules([{"name": n, "shape_a": [16, di], "shape_b": [do, 16]}
                                     for n, di, do in flux_modules()], num_levels=3)
    assert lay.total_blocks == 700_416 and lay.num_indices == 2_101_248
    assert lay.num_words == 300_179 and lay.num_words * 8 == 2_401_432


def test_quant_blockify_matches_oracle():
    rng = np.random.default_rng(0)
    for shape in ((16, 128), (40, 96), (7, 7103), (3, 5)):
        w = rng.standard_normal(shape).astype(np.float32)
        assert quant.num_blocks(shape) == opk.num_blocks(shape)
        b = quant.blockify(torch.from_numpy(w))
        assert np.array_equal(b.numpy(), opk.blockify(w))
        assert np.array_equal(quant.unblockify(b, shape).numpy(), w)


def test_codebook_pin_and_pools():
    assert cb.codebook_sha256() == ocb.INT_TABLE_SHA256
    pa, pb = lithe_amd.twin_pools()
    ra, rb = ocb.twin_pools()
    assert np.array_equal(pa.numpy().view(np.uint32), ra.view(np.uint32))
    assert np.array_equal(pb.numpy().view(np.uint32), rb.view(np.uint32))


def test_value_tables_from_pools():
    pa, pb = lithe_amd.twin_pools()
    cls = _hip._popcount_classes(64, 9)
    for pools, dt in ((pa, torch.float32), (pb, torch.float32), (pa, torch.bfloat16), (pb, torch.bfloat16)):
        lut = _hip.lut_from_pools(pools, dt)
        host = pools.to(dt).float().numpy()
        for level in range(3):
            vals = np.array([lut.value[level][p] for p in range(10)], dtype=np.float32)
            assert np.array_equal(vals[cls].view(np.uint32), host[level].view(np.uint32))
    # pools that are not twin Hadamard pools are refused
    bad = pa.clone()
    bad[1, 7, 3] += 1e-3
    with pytest.raises(ValueError):
        _hip.lut_from_pools(bad)
    with pytest.raises(ValueError):
        _hip.lut_from_pools(torch.zeros(3, 256, 64))
    # an in-place change of the pools invalidates the cached table
    p = pa.clone()
    before = _hip.lut_from_pools(p).value[0][0]
    p.mul_(2.0)
    assert _hip.lut_from_pools(p).value[0][0] == 2 * before


def test_lithe_file_round_trip_and_corruption(tmp_path):
    ad = random_adapter(SMALL, rank=16, seed=9)
    ad.metadata = {"instance_prompt": "a photo of a <v_sub_001> cat"}
    path = tmp_path / "a.lithe"
    size = fileio.save_lithe(path, ad)
    assert size == path.stat().st_size
    ad2 = fileio.load_lithe(path)
    assert ad2.modules == ad.modules and ad2.rank == ad.rank and ad2.alpha == ad.alpha
    assert ad2.metadata == ad.metadata
    for m in ad.modules:
        for side in ("A", "B"):
            assert ad2.indices[m["name"]][side].dtype == np.uint16
            assert np.array_equal(ad2.indices[m["name"]][side], ad.indices[m["name"]][side])
    assert ad2.raw_stream() == ad.raw_stream()
    assert fileio.read_header(path)["codebook"]["sha256"] == cb.codebook_sha256()
    # stream layout: all A blocks of every module, then all B
    raw = np.frombuffer(ad.raw_stream(), dtype="<u2")
    names = [m["name"] for m in ad.modules]
    expect = np.concatenate([ad.indices[n]["A"].ravel() for n in names] + [ad.indices[n]["B"].ravel() for n in names])
    assert np.array_equal(raw, expect)
    blob = bytearray(path.read_bytes())
    blob[-5] ^= 0xFF
    bad = tmp_path / "bad.lithe"
    bad.write_bytes(bytes(blob))
    with pytest.raises(Exception):
        fileio.load_lithe(bad)


def test_parse_route_reference_cases():
    # tests/test_serve.py:49-52 of the reference
    assert serve.parse_route("1") == [(1, 1.0)]
    assert serve.parse_route("0:0.6,2:0.4") == [(0, 0.6), (2, 0.4)]
    assert serve.parse_route("none") == []


def test_router_tables():
    r = serve.Router()
    r.set([[(2, 0.25), (0, 1.0)], [], [(1, 4.0)]])
    slot, w = r.device_tables("cpu")
    assert slot.dtype == torch.int32 and slot.tolist() == [[2, 0], [-1, -1], [1, -1]]
    assert np.array_equal(w.numpy(), np.sqrt(np.array([[0.25, 1.0], [0, 0], [4.0, 0]], np.float32)))
    with pytest.raises(ValueError):
        r.set([[(0, -1.0)]])


def test_flux_target_count():
    # tests/test_module.py:42-51 of the reference: 19 x 12 + 38 x 3 = 342 targets; proj_mlp,
    # proj_out and norm.linear of the single blocks are not matched
    names = []
    for i in range(19):
        names += [f"transformer_blocks.{i}.{t}" for t in module.FLUX_TARGET_MODULES]
    for i in range(38):
        names += [f"single_transformer_blocks.{i}.attn.{t}" for t in ("to_q", "to_k", "to_v")]
        names += [f"single_transformer_blocks.{i}.{t}" for t in ("proj_mlp", "proj_out", "norm.linear")]
    assert sum(module._match(n, module.FLUX_TARGET_MODULES) for n in names) == 342


def test_split_views_equal_per_module_slices():
    """split_decoded / split_stacked (one cached split of the flat buffer) give the same views as
    slicing every factor at its layout offset, aliasing the buffer; stacked views refuse factors
    that leave block padding."""
    import pytest
    import torch

    from helpers import random_adapter
    from lithe_amd.kernels import pack_adapter, split_decoded, split_stacked
    ad = random_adapter([("a", 96, 40), ("odd", 7, 5), ("b", 128, 64)], rank=5, seed=1)
    _, lay = pack_adapter(ad)
    out = torch.arange(lay.total_blocks * 64, dtype=torch.float32).view(-1, 64)
    flat = out.reshape(-1)
    for _ in range(2):                                   # second call: the cached plan
        got = split_decoded(out, lay)
        for name, sa, sb, ao, bo in zip(lay.names, lay.shapes_a, lay.shapes_b, lay.a_off, lay.b_off):
            na, nb = sa[0] * sa[1], sb[0] * sb[1]
            assert torch.equal(got[name][0], flat[ao * 64: ao * 64 + na].view(*sa)), name
            assert torch.equal(got[name][1], flat[bo * 64: bo * 64 + nb].view(*sb)), name
            assert got[name][0].data_ptr() == flat[ao * 64:].data_ptr()
    with pytest.raises(ValueError, match="whole blocks"):
        split_stacked(out, lay, 2)
    ad2 = random_adapter([("a", 128, 64), ("b", 256, 128)], rank=16, seed=2)
    _, lay2 = pack_adapter(ad2)
    n_sel = 3
    buf = torch.arange(n_sel * lay2.total_blocks * 64, dtype=torch.float32)
    st = split_stacked(buf, lay2, n_sel)
    for name, sa, sb, ao, bo in zip(lay2.names, lay2.shapes_a, lay2.shapes_b, lay2.a_off, lay2.b_off):
        na, nb = sa[0] * sa[1], sb[0] * sb[1]
        assert torch.equal(st[name][0], buf[n_sel * ao * 64: n_sel * ao * 64 + n_sel * na].view(n_sel, *sa)), name
        assert torch.equal(st[name][1], buf[n_sel * bo * 64: n_sel * bo * 64 + n_sel * nb].view(n_sel, *sb)), name


def test_attach_adapters_loads_every_adapter_in_order():
    """attach_adapters on a CPU model: each layer's int16 stacks hold adapter i's indices at row i
    (the stores grow past their capacity), scales are alpha / r; mismatched adapters are refused."""
    from torch import nn

    from helpers import random_adapter

    class Two(nn.Module):
        def __init__(self):
            super().__init__()
            self.a = nn.Linear(128, 64)
            self.b = nn.Linear(64, 192)

    ads = [random_adapter([("a", 128, 64), ("b", 64, 192)], rank=4, seed=s) for s in range(5)]
    for i, ad in enumerate(ads):
        ad.alpha = float(2 * i + 1)
    model = Two()
    router, layers = serve.attach_adapters(model, ads)
    assert set(layers) == {"a", "b"} and model.a is layers["a"] and layers["a"].router is router
    for name in ("a", "b"):
        lay = layers[name]
        assert lay.idx_a.shape[0] == lay.idx_b.shape[0] == 5 and lay.idx_a.dtype == torch.int16
        for i, ad in enumerate(ads):
            assert np.array_equal(lay.idx_a[i].numpy(), ad.indices[name]["A"].astype(np.int16))
            assert np.array_equal(lay.idx_b[i].numpy(), ad.indices[name]["B"].astype(np.int16))
        assert lay.scales.tolist() == [(2 * i + 1) / 4 for i in range(5)]
    with pytest.raises(ValueError):
        layers["a"].add_adapter(ads[0].indices["b"]["A"], ads[0].indices["b"]["B"], 1.0)
    other = random_adapter([("a", 128, 64)], rank=4, seed=9)
    with pytest.raises(ValueError):
        serve.attach_adapters(Two(), [ads[0], other])
    with pytest.raises(ValueError):
        serve.attach_adapters(Two(), [])


def test_target_match_is_a_whole_component_suffix():
    """module._match: a path matches a target when it equals it or ends with '.' + target
    (lithe/module.py:159-160), never inside a path component."""
    t = ["attn.to_q", "ff.net.2"]
    for path, want in [("attn.to_q", True), ("transformer_blocks.3.attn.to_q", True), ("xattn.to_q", False),
                       ("to_q", False), ("single.attn.to_q.lora", False), ("blk.ff.net.2", True),
                       ("blk.ff.net.20", False), ("blk.ff_context.net.2", False)]:
        assert module._match(path, t) == want, path
        assert module._match(path, t) == any(path == s or path.endswith("." + s) for s in t), path
