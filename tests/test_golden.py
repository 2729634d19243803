"""The fixtures of tests/golden: the reference tests' known answers (as data), and the
oracle's seeded regression vectors (tests/golden/make_fixtures.py writes both)."""
import json
import os

import numpy as np
import torch

from lithe_amd import codebook as cb
from lithe_amd import module, serve
from lithe_amd.fileio import LitheAdapter
from lithe_amd.kernels.packed import PackedLayout, pack_indices
from oracle import codebook as ocb
from oracle import decode as odec
from oracle import delta as odelta
from oracle import packing as opk

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
KNOWN = json.load(open(os.path.join(GOLD, "known_answers.json")))
VEC = np.load(os.path.join(GOLD, "oracle_vectors.npz"))


def _small_adapter():
    mods = [{"name": n, "shape_a": [16, di], "shape_b": [do, 16]} for n, di, do in KNOWN["small_modules"]["value"]]
    return mods


def test_known_answers_codebook_and_layouts():
    assert cb.codebook_sha256() == KNOWN["codebook_int_table_sha256"]["value"] == ocb.table_sha256()
    k = KNOWN["kohya304"]
    mods = []
    for di, do, count in k["modules"]:
        mods += [{"name": f"m{len(mods) + i}", "shape_a": [k["rank"], di], "shape_b": [do, k["rank"]]} for i in range(count)]
    lay = PackedLayout.from_adapter(LitheAdapter(modules=mods, indices={}, rank=16, alpha=16.0))
    assert lay.num_indices == k["num_indices"] and lay.num_words * 8 == k["packed_bytes"]
    f = KNOWN["flux342"]
    from helpers import flux_modules
    lay = PackedLayout.from_modules([{"name": n, "shape_a": [16, di], "shape_b": [do, 16]} for n, di, do in flux_modules()])
    assert (lay.total_blocks, lay.num_indices, lay.num_words, lay.num_words * 8) == (
        f["blocks"], f["num_indices"], f["words"], f["packed_bytes"])


def test_known_answers_pack_roundtrip_route_and_targets():
    rng = np.random.default_rng(1)
    for n in KNOWN["pack_roundtrip_sizes"]["value"]:
        v = rng.integers(0, 512, n)
        words = pack_indices(v)
        assert words.dtype == torch.uint64 and words.numel() == -(-n // 7)
        assert np.array_equal(words.view(torch.int64).numpy().view(np.uint64), opk.pack(v))
        assert np.array_equal(opk.unpack(opk.pack(v), n), v)
    for spec, want in KNOWN["parse_route"]["value"]:
        assert serve.parse_route(spec) == [tuple(p) for p in want]
    names = []
    for i in range(19):
        names += [f"transformer_blocks.{i}.{t}" for t in module.FLUX_TARGET_MODULES]
    for i in range(38):
        names += [f"single_transformer_blocks.{i}.attn.{t}" for t in ("to_q", "to_k", "to_v")]
        names += [f"single_transformer_blocks.{i}.{t}" for t in ("proj_mlp", "proj_out", "norm.linear")]
    assert sum(module._match(n, module.FLUX_TARGET_MODULES) for n in names) == KNOWN["flux_target_count"]["value"]


def test_oracle_regression_vectors():
    mods = _small_adapter()
    stream = VEC["small_indices"].astype(np.int64)
    words = opk.pack(stream)
    assert np.array_equal(words, VEC["small_words"])
    lay = opk.layout_of({"modules": mods, "rank": 16, "alpha": 16.0, "num_levels": 3, "block_size": 64})
    pa, pb = ocb.twin_pools()
    assert np.array_equal(odec.bf16_bits(odec.decode_packed(words, lay, pa, pb)), VEC["small_decode_bf16"])
    delta = odelta.shared_delta(VEC["delta_x"], VEC["delta_ia"], pa, VEC["delta_ib"], pb, [1, 0], 16, 192, 0.5, "bf16")
    assert np.array_equal(odec.bf16_bits(delta), VEC["delta_bf16"])
    # the product's host packer gives the same words
    assert np.array_equal(pack_indices(stream.astype(np.uint16)).view(torch.int64).numpy().view(np.uint64), words)
