"""Writes the fixtures of tests/golden (run from the repository root: python tests/golden/make_fixtures.py).

* known_answers.json — the known-answer values the reference's own tests hold for this path,
  restated as data with the file:line they come from (the reference stores no fixture files).
* oracle_vectors.npz — small seeded vectors produced by the oracle (packed words, bf16 bits
  of a bulk decode, a bf16 shared-codebook delta). They pin nothing by themselves; they guard
  the oracle against accidental change between the runs that pinned it (tests/test_oracle.py).
"""
import json
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

from oracle import codebook as ocb  # noqa: E402
from oracle import decode as odec  # noqa: E402
from oracle import delta as odelta  # noqa: E402
from oracle import packing as opk  # noqa: E402

KNOWN = {
    "codebook_int_table_sha256": {
        "value": "eb1f4de0d64df9980436232299238e56ff04efa9ab075ded3f72c2a821ad0301",
        "source": "tests/test_codebook.py:9"},
    "kohya304": {
        "modules": [[3072, 9216, 76], [3072, 18432, 38], [3072, 3072, 38], [3072, 12288, 38],
                    [12288, 3072, 38], [3072, 21504, 38], [15360, 3072, 38]],
        "rank": 16, "num_indices": 3_589_632, "packed_bytes": 4_102_440,
        "source": "tests/test_kernels.py:57-64"},
    "flux342": {
        "rank": 16, "blocks": 700_416, "num_indices": 2_101_248, "words": 300_179, "packed_bytes": 2_401_432,
        "source": "README.md:146; module.py:13-28"},
    "pack_roundtrip_sizes": {"value": [1, 6, 7, 8, 700, 1001], "source": "tests/test_kernels.py:46-54"},
    "small_modules": {"value": [["blk.0.q", 128, 192], ["blk.0.mlp", 128, 320], ["blk.0.out", 320, 128],
                                ["odd", 96, 40]], "source": "tests/test_kernels.py:42"},
    "delta_shapes": {"value": [[256, 3072, 3072, 16], [50, 128, 192, 16], [1, 256, 384, 4]],
                     "source": "tests/test_kernels.py:203"},
    "parse_route": {"value": [["1", [[1, 1.0]]], ["0:0.6,2:0.4", [[0, 0.6], [2, 0.4]]], ["none", []]],
                    "source": "tests/test_serve.py:49-52"},
    "flux_target_count": {"value": 342, "source": "tests/test_module.py:42-51"},
}


def random_levels(rng, shape, levels=3):
    return rng.integers(0, 512, (levels, opk.num_blocks(shape)))


def main():
    with open(os.path.join(HERE, "known_answers.json"), "w") as fh:
        json.dump(KNOWN, fh, indent=1)
        fh.write("\n")
    rng = np.random.default_rng(20241201)
    # one small adapter of the reference's SMALL shapes (seeded generator of tests/test_kernels.py:20-28)
    mods = [{"name": n, "shape_a": [16, di], "shape_b": [do, 16]} for n, di, do in KNOWN["small_modules"]["value"]]
    indices = {m["name"]: {"A": random_levels(rng, m["shape_a"]).astype(np.uint16),
                           "B": random_levels(rng, m["shape_b"]).astype(np.uint16)} for m in mods}
    ad = {"modules": mods, "indices": indices, "rank": 16, "alpha": 16.0, "num_levels": 3, "block_size": 64}
    words, layout = opk.pack_adapter(ad)
    pa, pb = ocb.twin_pools()
    dec = odec.decode_packed(words, layout, pa, pb)
    # a bf16 shared-codebook delta: B=2 samples x 5 tokens, 128 -> 192, two adapters
    ia = rng.integers(0, 512, (2, 3, opk.num_blocks((16, 128))))
    ib = rng.integers(0, 512, (2, 3, opk.num_blocks((192, 16))))
    x = odec.round_bf16(rng.standard_normal((2, 5, 128)).astype(np.float32))
    delta = odelta.shared_delta(x, ia, pa, ib, pb, [1, 0], 16, 192, 0.5, "bf16")
    np.savez_compressed(os.path.join(HERE, "oracle_vectors.npz"),
                        small_indices=opk.stream_order(ad, layout), small_words=words,
                        small_decode_bf16=odec.bf16_bits(dec), delta_x=x, delta_ia=ia, delta_ib=ib,
                        delta_bf16=odec.bf16_bits(delta))


if __name__ == "__main__":
    main()
