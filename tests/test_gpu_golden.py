"""GPU checks against the fixtures of tests/golden: the bulk decode of the small packed
adapter (bit-exact) and the bf16 shared-codebook delta (within the bf16 tolerance of
tests/test_gpu_delta.py)."""
import os

import numpy as np
import pytest
import torch

import lithe_amd
from lithe_amd.kernels import PackedLayout, decode_packed, shared_codebook_lora_delta
from oracle import decode as odec

from helpers import rel

pytestmark = pytest.mark.gpu
VEC = np.load(os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "oracle_vectors.npz"))
SMALL = [("blk.0.q", 128, 192), ("blk.0.mlp", 128, 320), ("blk.0.out", 320, 128), ("odd", 96, 40)]


def test_golden_decode_bit_exact():
    layout = PackedLayout.from_modules([{"name": n, "shape_a": [16, di], "shape_b": [do, 16]} for n, di, do in SMALL])
    words = torch.from_numpy(VEC["small_words"].view(np.int64)).cuda()
    pa, pb = (p.cuda() for p in lithe_amd.twin_pools())
    out = decode_packed(words, layout, pa, pb)
    assert np.array_equal(out.view(torch.int16).cpu().numpy().view(np.uint16), VEC["small_decode_bf16"])


def test_golden_shared_delta():
    pa, pb = (p.cuda() for p in lithe_amd.twin_pools())
    x = torch.from_numpy(VEC["delta_x"]).cuda().bfloat16()
    ia = torch.from_numpy(VEC["delta_ia"]).cuda().int()
    ib = torch.from_numpy(VEC["delta_ib"]).cuda().int()
    got = shared_codebook_lora_delta(x, ia, pa.bfloat16(), ib, pb.bfloat16(), torch.tensor([1, 0], device="cuda"),
                                     16, 192, 0.5)
    want = odec.bf16_value(VEC["delta_bf16"])
    assert rel(got.float().cpu().numpy(), want) < 2e-3
