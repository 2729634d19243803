"""CPU checks of the C ABI: the library loads, exports every function include/lithe_amd.h
declares with the signature the ctypes binding uses, and rejects bad arguments before any
GPU work (no call here reaches a kernel launch).
"""
import ctypes
import os
import re

import numpy as np
import pytest
import torch

from lithe_amd.kernels import _hip
from oracle import packing as opk

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "lithe_amd.h")


def _declared():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(lithe_[a-z0-9_]+)\s*\(", text)))


def _defines():
    return {m.group(1): int(m.group(2)) for m in re.finditer(r"#define\s+(LITHE_\w+)\s+(-?\d+)", open(HEADER).read())}


def test_library_loads_and_exports_every_declared_symbol():
    lib = _hip.load()
    names = _declared()
    assert len(names) >= 9, names
    for n in names:
        assert hasattr(lib, n), f"{n} declared in lithe_amd.h but not exported"
        assert n in _hip.SIGNATURES, f"{n} has no ctypes signature in _hip.SIGNATURES"
    assert sorted(_hip.SIGNATURES) == names


def test_constants_match_header():
    d = _defines()
    assert d["LITHE_OK"] == _hip.OK
    for n in ("NULL", "SHAPE", "ALIGN", "DTYPE", "RANGE", "WORKSPACE", "HIP", "LEVELS", "UNSUPPORTED", "OVERLAP"):
        assert d[f"LITHE_ERR_{n}"] == getattr(_hip, f"ERR_{n}"), n
    for n in ("BF16", "F32", "F16", "I16", "I32", "I64", "U16"):
        assert d[f"LITHE_DT_{n}"] == getattr(_hip, f"DT_{n}"), n
    for n in ("PACKED9", "LEVEL_I32", "LEVEL_I16", "BLOCK_I16"):
        assert d[f"LITHE_IDX_{n}"] == getattr(_hip, f"IDX_{n}"), n
    assert d["LITHE_FACTOR_INDEXED"] == _hip.FACTOR_INDEXED and d["LITHE_FACTOR_DENSE"] == _hip.FACTOR_DENSE


def test_struct_layouts_match_header_sizes():
    # lithe_index_src: ptr, 2 x int32, 4 x int64 ; lithe_lut: int32 + 40 floats ; routes: 3 ptrs + int32
    assert ctypes.sizeof(_hip.IndexSrc) == 8 + 4 + 4 + 4 * 8
    assert ctypes.sizeof(_hip.Lut) == 4 + 40 * 4
    assert ctypes.sizeof(_hip.Routes) == 3 * 8 + 8
    assert _hip.Factors.a_idx.offset == 8 and _hip.Factors.dense_a.offset % 8 == 0


def test_version_and_status_strings():
    lib = _hip.load()
    assert lib.lithe_abi_version() == 1
    for code in range(0, -11, -1):
        s = lib.lithe_status_string(code).decode()
        assert s and "unknown" not in s.lower(), (code, s)
    assert "unknown" in lib.lithe_status_string(-99).decode().lower()


@pytest.mark.parametrize("n", [0, 1, 6, 7, 8, 700, 1001, 100_003])
def test_host_pack_matches_oracle(n):
    lib = _hip.load()
    v = np.random.default_rng(n).integers(0, 512, n).astype(np.uint16)
    words = np.zeros(max(1, -(-n // 7)), dtype=np.uint64)
    rc = lib.lithe_pack9_host(v.ctypes.data, n, words.ctypes.data)
    assert rc == _hip.OK
    assert np.array_equal(words[: -(-n // 7)], opk.pack(v))


def test_host_pack_rejects_512():
    lib = _hip.load()
    v = np.array([1, 2, 512, 3], dtype=np.uint16)
    words = np.zeros(1, dtype=np.uint64)
    assert lib.lithe_pack9_host(v.ctypes.data, 4, words.ctypes.data) == _hip.ERR_RANGE
    assert lib.lithe_pack9_host(None, 4, words.ctypes.data) == _hip.ERR_NULL


def test_workspace_bytes():
    lib = _hip.load()
    ws = lib.lithe_lora_workspace_bytes
    # head + mid (rows x 16 x 2 B), 256-aligned
    n = ws(14, 4608, 3072, 3072, 16, 1, _hip.DT_BF16)
    assert n == 256 + ((14 * 4608 * 16 * 2 + 255) // 256) * 256
    assert ws(2, 3, 64, 64, 16, 1, _hip.DT_F32) >= 256 + 2 * 3 * 16 * 4
    # two rank groups per route entry, four entries
    assert ws(1, 10, 128, 64, 32, 4, _hip.DT_BF16) >= 256 + 10 * 128 * 2
    assert ws(1, 10, 128, 64, 16, 9, _hip.DT_BF16) == _hip.ERR_SHAPE     # 9 groups > 8
    assert ws(1, 10, 32, 64, 16, 1, _hip.DT_BF16) == _hip.ERR_SHAPE      # d_in < 64
    assert ws(1, 10, 128, 64, 16, 1, _hip.DT_F16) == _hip.ERR_DTYPE


def _indexed(levels=3, n_slots=4, d_in=128, d_out=64, rank=16):
    nb = rank * d_in // 64 + d_out * rank // 64
    words = np.zeros((n_slots, -(-nb * levels // 7)), dtype=np.uint64)
    src = _hip.IndexSrc(base=words.ctypes.data, kind=_hip.IDX_PACKED9, num_levels=levels,
                        slot_stride=words.shape[1], level_stride=0, block_off=0, n_slots=n_slots)
    srcb = _hip.IndexSrc(base=words.ctypes.data, kind=_hip.IDX_PACKED9, num_levels=levels,
                         slot_stride=words.shape[1], level_stride=0, block_off=rank * d_in // 64, n_slots=n_slots)
    f = _hip.Factors()
    f.kind = _hip.FACTOR_INDEXED
    f.a_idx, f.b_idx = src, srcb
    f.lut_a.num_levels = f.lut_b.num_levels = levels
    return f, words


def _delta(lib, f, route, *, x=1 << 12, y=1 << 12, ws=1 << 12, x_dt=None, y_dt=None, n_batch=2, seq=8,
           d_in=128, d_out=64, rank=16, wsb=1 << 20, dense=False):
    return lib.lithe_lora_delta(ctypes.c_void_p(x), x_dt or _hip.DT_BF16, n_batch, seq, d_in, ctypes.c_void_p(y),
                                y_dt or _hip.DT_BF16, d_out, 1, rank, ctypes.byref(f) if f else None,
                                ctypes.byref(route) if route else None, None, ctypes.c_float(1.0), None,
                                ctypes.c_void_p(ws), wsb, None)


def test_delta_argument_errors_before_any_launch():
    """Every case fails validation on the host; fake (aligned, never dereferenced) pointers suffice."""
    lib = _hip.load()
    f, words = _indexed()
    slot = np.zeros(2, dtype=np.int32)
    route = _hip.Routes(slot=slot.ctypes.data, weight_sqrt=None, slot_scale=None, n_route=1)
    assert _delta(lib, None, route) == _hip.ERR_NULL
    assert _delta(lib, f, None) == _hip.ERR_NULL
    assert _delta(lib, f, route, x_dt=_hip.DT_F16) == _hip.ERR_DTYPE
    assert _delta(lib, f, route, y_dt=_hip.DT_I32) == _hip.ERR_DTYPE
    assert _delta(lib, f, route, d_in=100) == _hip.ERR_ALIGN                # d_in % 64
    assert _delta(lib, f, route, d_out=60, rank=1) == _hip.ERR_ALIGN        # d_out * rank % 64
    assert _delta(lib, f, route, n_batch=-1) == _hip.ERR_SHAPE
    assert _delta(lib, f, route, rank=0) == _hip.ERR_SHAPE
    assert _delta(lib, f, route, n_batch=0) == _hip.OK                      # empty batch: nothing to do
    assert _delta(lib, f, route, x=0) == _hip.ERR_NULL
    assert _delta(lib, f, route, ws=0) == _hip.ERR_WORKSPACE
    assert _delta(lib, f, route, x=(1 << 12) + 8) == _hip.ERR_ALIGN         # x not 16-byte aligned
    assert _delta(lib, f, route, ws=(1 << 12) + 16) == _hip.ERR_ALIGN       # workspace not 256-aligned
    assert _delta(lib, f, route, wsb=256) == _hip.ERR_WORKSPACE             # too small
    # index sources: levels must agree, and cover the factor
    f2, _ = _indexed()
    f2.lut_b.num_levels = 2
    assert _delta(lib, f2, route) == _hip.ERR_LEVELS
    assert _delta(lib, f, route, d_in=256) == _hip.ERR_SHAPE                # A extends past the slot
    f3, _ = _indexed()
    f3.a_idx.num_levels = 5
    assert _delta(lib, f3, route) == _hip.ERR_LEVELS
    f4, _ = _indexed()
    f4.a_idx.kind = 9
    assert _delta(lib, f4, route) == _hip.ERR_DTYPE
    # route weights are for indexed factors only
    a = np.zeros(16, dtype=np.uint16)
    fd = _hip.Factors()
    fd.kind = _hip.FACTOR_DENSE
    fd.dense_dtype = _hip.DT_BF16
    fd.dense_a, fd.dense_b, fd.n_dense = 1 << 12, 1 << 13, 2
    w = np.ones(2, dtype=np.float32)
    rw = _hip.Routes(slot=slot.ctypes.data, weight_sqrt=w.ctypes.data, slot_scale=None, n_route=1)
    assert _delta(lib, fd, rw) == _hip.ERR_UNSUPPORTED
    fd.dense_dtype = _hip.DT_F32
    assert _delta(lib, fd, route) == _hip.ERR_DTYPE                          # dense dtype != x dtype
    del a, words


def test_unpack_decode_argument_errors():
    lib = _hip.load()
    assert lib.lithe_unpack9(None, 5, ctypes.c_void_p(1 << 12), _hip.DT_I64, None) == _hip.ERR_NULL
    assert lib.lithe_unpack9(ctypes.c_void_p(1 << 12), 5, ctypes.c_void_p(1 << 12), _hip.DT_BF16, None) == _hip.ERR_DTYPE
    assert lib.lithe_unpack9(ctypes.c_void_p(1 << 12), -1, ctypes.c_void_p(1 << 12), _hip.DT_I64, None) == _hip.ERR_SHAPE
    assert lib.lithe_unpack9(None, 0, None, _hip.DT_I64, None) == _hip.OK
    lut = _hip.Lut(num_levels=3)
    src = _hip.IndexSrc(base=1 << 12, kind=_hip.IDX_PACKED9, num_levels=3, slot_stride=10, level_stride=0,
                        block_off=0, n_slots=1)
    dec = lib.lithe_decode
    assert dec(None, None, 1, 4, None, ctypes.byref(lut), ctypes.byref(lut), ctypes.c_void_p(1 << 12),
               _hip.DT_BF16, 0, None, None) == _hip.ERR_NULL
    assert dec(ctypes.byref(src), None, 1, 4, None, ctypes.byref(lut), ctypes.byref(lut), ctypes.c_void_p(1 << 12),
               _hip.DT_I32, 0, None, None) == _hip.ERR_DTYPE
    assert dec(ctypes.byref(src), None, 1, 1000, None, ctypes.byref(lut), ctypes.byref(lut),
               ctypes.c_void_p(1 << 12), _hip.DT_BF16, 0, None, None) == _hip.ERR_SHAPE   # 1000 blocks > slot


def test_product_entry_points_refuse_cpu_tensors():
    import lithe_amd
    from lithe_amd.kernels import decode_packed, pack_adapter, unpack_indices
    from helpers import SMALL, random_adapter
    ad = random_adapter(SMALL, rank=16, seed=0)
    words, layout = pack_adapter(ad)
    pa, pb = lithe_amd.twin_pools()
    with pytest.raises(RuntimeError):
        decode_packed(words, layout, pa, pb)
    with pytest.raises(RuntimeError):
        unpack_indices(words.view(torch.int64), 7)


def test_shared_x_argument_errors_before_any_launch():
    """lithe_lora_delta_shared_x: host arrays, one shared A source, group-count limit."""
    lib = _hip.load()
    f0, words = _indexed()
    slot = np.zeros(2, dtype=np.int32)
    route = _hip.Routes(slot=slot.ctypes.data, weight_sqrt=None, slot_scale=None, n_route=1)

    def call(fs, n_mod=None, d_outs=None, ys=None, scales=None, n_batch=2, wsb=1 << 20, rte=route):
        n = len(fs) if n_mod is None else n_mod
        fa = (_hip.Factors * max(1, len(fs)))(*fs) if fs else None
        ya = (ctypes.c_void_p * max(1, n))(*(ys or [1 << 12] * n))
        da = (ctypes.c_int64 * max(1, n))(*(d_outs or [64] * n))
        sa = (ctypes.c_float * max(1, n))(*(scales or [1.0] * n))
        return lib.lithe_lora_delta_shared_x(ctypes.c_void_p(1 << 12), _hip.DT_BF16, n_batch, 8, 128, n, ya,
                                             _hip.DT_BF16, da, 1, 16, fa, ctypes.byref(rte) if rte else None,
                                             None, sa, ctypes.c_void_p(1 << 12), wsb, None)

    fq, fk, fv = _indexed()[0], _indexed()[0], _indexed()[0]
    for f in (fq, fk, fv):
        f.a_idx.base = f0.a_idx.base
        f.b_idx.base = f0.b_idx.base
    assert call([]) == _hip.ERR_NULL                                          # no factors
    assert call([fq, fk, fv], rte=None) == _hip.ERR_NULL
    assert call([fq, fk, fv], n_mod=0) == _hip.ERR_SHAPE
    assert call([fq] * 9) == _hip.ERR_SHAPE                                   # 9 rank groups > 8
    assert call([fq, fk, fv], d_outs=[64, 0, 64]) == _hip.ERR_SHAPE
    assert call([fq, fk, fv], ys=[1 << 12, 0, 1 << 12]) == _hip.ERR_NULL
    assert call([fq, fk, fv], ys=[1 << 12, (1 << 12) + 1, 1 << 12]) == _hip.ERR_ALIGN
    other = _indexed()[0]                                                     # A in another bank
    other.a_idx.base = f0.a_idx.base + 4096
    assert call([fq, other, fv]) == _hip.ERR_UNSUPPORTED
    lut2 = _indexed()[0]
    lut2.a_idx.base, lut2.b_idx.base = f0.a_idx.base, f0.b_idx.base
    lut2.lut_a.value[0][3] = 0.5                                              # another A value table
    assert call([fq, lut2, fv]) == _hip.ERR_UNSUPPORTED
    dense = _hip.Factors()
    dense.kind = _hip.FACTOR_DENSE
    assert call([fq, dense, fv]) == _hip.ERR_UNSUPPORTED
    assert call([fq, fk, fv], wsb=256) == _hip.ERR_WORKSPACE
    assert call([fq, fk, fv], n_batch=0) == _hip.OK                           # empty batch: nothing to do
    del words


def test_encode_decode_stacked_ingest_argument_errors():
    lib = _hip.load()
    lut = _hip.Lut(num_levels=3)
    P = ctypes.c_void_p(1 << 12)
    enc = lib.lithe_encode
    assert enc(P, -1, None, ctypes.byref(lut), None, P, _hip.DT_I16, 5, 1, None, None) == _hip.ERR_SHAPE
    assert enc(P, 5, None, None, None, P, _hip.DT_I16, 5, 1, None, None) == _hip.ERR_NULL
    assert enc(P, 5, P, ctypes.byref(lut), None, P, _hip.DT_I16, 5, 1, None, None) == _hip.ERR_NULL  # sides, no lut_b
    bad = _hip.Lut(num_levels=5)
    assert enc(P, 5, None, ctypes.byref(bad), None, P, _hip.DT_I16, 5, 1, None, None) == _hip.ERR_LEVELS
    assert enc(P, 5, None, ctypes.byref(lut), None, P, _hip.DT_BF16, 5, 1, None, None) == _hip.ERR_DTYPE
    assert enc(P, 0, None, ctypes.byref(lut), None, None, _hip.DT_I16, 0, 1, None, None) == _hip.OK
    assert enc(None, 5, None, ctypes.byref(lut), None, P, _hip.DT_I16, 5, 1, None, None) == _hip.ERR_NULL
    assert enc(P, 5, None, ctypes.byref(lut), None, P, _hip.DT_I16, 2, 1, None, None) == _hip.ERR_SHAPE  # overlap
    assert enc(P, 5, None, ctypes.byref(lut), None, P, _hip.DT_I16, 1, 2, None, None) == _hip.ERR_SHAPE
    assert enc(ctypes.c_void_p((1 << 12) + 4), 5, None, ctypes.byref(lut), None, P, _hip.DT_I16, 5, 1, None,
               None) == _hip.ERR_ALIGN
    src = _hip.IndexSrc(base=1 << 12, kind=_hip.IDX_PACKED9, num_levels=3, slot_stride=10, level_stride=0,
                        block_off=0, n_slots=1)
    ds = lib.lithe_decode_stacked
    assert ds(ctypes.byref(src), None, 1, 4, 2, None, None, ctypes.byref(lut), ctypes.byref(lut), P, _hip.DT_BF16,
              None, None) == _hip.ERR_NULL                                    # no segment table
    assert ds(ctypes.byref(src), None, 1, 4, 0, P, None, ctypes.byref(lut), ctypes.byref(lut), P, _hip.DT_BF16,
              None, None) == _hip.ERR_SHAPE
    ing = lib.lithe_ingest
    assert ing(P, -1, 3, 2, P, P, 10, None, None) == _hip.ERR_SHAPE
    assert ing(P, 7, 3, 0, P, P, 10, None, None) == _hip.ERR_SHAPE
    assert ing(P, 7, 0, 2, P, P, 10, None, None) == _hip.ERR_LEVELS
    assert ing(P, 70, 3, 2, P, P, 9, None, None) == _hip.ERR_SHAPE             # 70 indices need 10 words
    assert ing(None, 0, 3, 2, None, None, 0, None, None) == _hip.OK
    assert ing(None, 7, 3, 2, P, P, 1, None, None) == _hip.ERR_NULL


def test_launch_grid_limits():
    """Problems whose workgroup count would not fit a launch are rejected before any launch."""
    lib = _hip.load()
    f, words = _indexed(d_in=128, d_out=64)
    slot = np.zeros(65535, dtype=np.int32)
    route = _hip.Routes(slot=slot.ctypes.data, weight_sqrt=None, slot_scale=None, n_route=1)
    # 65,535 samples of 2**30 tokens: far more than 2**31 - 1 workgroups
    assert _delta(lib, f, route, n_batch=65535, seq=1 << 30, wsb=1 << 62) == _hip.ERR_SHAPE
    lut = _hip.Lut(num_levels=3)
    P = ctypes.c_void_p(1 << 12)
    assert lib.lithe_encode(P, 1 << 40, None, ctypes.byref(lut), None, P, _hip.DT_I16, 1 << 41, 1, None,
                            None) == _hip.ERR_SHAPE
    src = _hip.IndexSrc(base=1 << 12, kind=_hip.IDX_PACKED9, num_levels=3, slot_stride=10, level_stride=0,
                        block_off=0, n_slots=1)
    assert lib.lithe_decode(ctypes.byref(src), P, 70000, 4, None, ctypes.byref(lut), ctypes.byref(lut), P,
                            _hip.DT_BF16, 256, None, None) == _hip.ERR_SHAPE       # 70,000 selections > 65,535
    assert lib.lithe_unpack9(P, 1 << 45, P, _hip.DT_I64, None) == _hip.ERR_SHAPE
    del words


def test_noalloc_delta_argument_errors_before_any_launch():
    """lithe_lora_delta_noalloc: the checks of lithe_lora_delta, then the static-scratch limit; a call
    that passes every check on a machine without a GPU fails to find the device (LITHE_ERR_HIP)."""
    lib = _hip.load()
    f, words = _indexed(d_in=3072, d_out=3072)
    slot = np.zeros(14, dtype=np.int32)
    route = _hip.Routes(slot=slot.ctypes.data, weight_sqrt=None, slot_scale=None, n_route=1)

    def call(fa=f, rt=route, x=1 << 12, n_batch=2, seq=8, rank=16):
        return lib.lithe_lora_delta_noalloc(ctypes.c_void_p(x), _hip.DT_BF16, n_batch, seq, 3072,
                                            ctypes.c_void_p(1 << 12), _hip.DT_BF16, 3072, 1, rank,
                                            ctypes.byref(fa) if fa else None, ctypes.byref(rt) if rt else None, None,
                                            ctypes.c_float(1.0), None, None, None)

    assert call(fa=None) == _hip.ERR_NULL
    assert call(rt=None) == _hip.ERR_NULL
    assert call(x=0) == _hip.ERR_NULL
    assert call(x=(1 << 12) + 8) == _hip.ERR_ALIGN
    assert call(n_batch=0) == _hip.OK
    # 14 x 40,000 tokens x 16 ranks x 2 bytes = 17.9 MB of intermediate > the 16 MiB scratch
    assert call(n_batch=14, seq=40_000) == _hip.ERR_WORKSPACE
    assert lib.lithe_lora_workspace_bytes(14, 40_000, 3072, 3072, 16, 1, _hip.DT_BF16) - 256 > _hip.STATIC_SCRATCH_BYTES
    # 14 x 37,449 tokens fit exactly below the limit: every check passes, then the device lookup
    assert lib.lithe_lora_workspace_bytes(14, 37_449, 3072, 3072, 16, 1, _hip.DT_BF16) - 256 <= _hip.STATIC_SCRATCH_BYTES
    if not torch.cuda.is_available():
        assert call(n_batch=14, seq=37_449) == _hip.ERR_HIP
    del words


def test_grouped_argument_errors_and_workspace_bytes():
    """lithe_lora_delta_grouped: per-module checks of lithe_lora_delta, the module limit, the checks
    of dense (stacked) factors, the workspace of one intermediate per distinct input; no call
    reaches a launch."""
    lib = _hip.load()
    f, words = _indexed(n_slots=4, d_in=128, d_out=64)
    slot = np.zeros(2, dtype=np.int32)
    route = _hip.Routes(slot=slot.ctypes.data, weight_sqrt=None, slot_scale=None, n_route=1)

    def mods(n, **kw):
        arr = (_hip.Module * max(1, n))()
        for i in range(n):
            arr[i].x, arr[i].y = kw.get("x", 1 << 12), kw.get("y", 1 << 13)
            if kw.get("distinct", False) and arr[i].y:
                arr[i].y += i << 16
            arr[i].seq, arr[i].d_in, arr[i].d_out = kw.get("seq", 8), 128, kw.get("d_out", 64)
            arr[i].a_block_off, arr[i].b_block_off, arr[i].out_scale = 0, 32, 1.0
        return arr

    def call(arr, n, fa=f, wsb=1 << 20, n_batch=2, ws=1 << 12, rt=route):
        return lib.lithe_lora_delta_grouped(n, arr, _hip.DT_BF16, _hip.DT_BF16, n_batch, 1, 16,
                                            ctypes.byref(fa) if fa else None, ctypes.byref(rt),
                                            ctypes.c_void_p(ws), wsb, None)

    assert call(None, 2) == _hip.ERR_NULL
    assert call(mods(2), 2, fa=None) == _hip.ERR_NULL
    assert call(mods(1), 0) == _hip.ERR_SHAPE
    assert call(mods(9), 9) == _hip.ERR_SHAPE                                 # more than 8 modules
    dense = _hip.Factors()                                                    # stacked dense factors
    dense.kind, dense.dense_dtype, dense.n_dense = _hip.FACTOR_DENSE, _hip.DT_BF16, 4
    assert call(mods(2, distinct=True), 2, fa=dense) == _hip.ERR_NULL         # no factor buffers
    dense.dense_a = dense.dense_b = 1 << 14
    dense.dense_dtype = _hip.DT_F32
    assert call(mods(2, distinct=True), 2, fa=dense) == _hip.ERR_DTYPE        # not the activation dtype
    dense.dense_dtype, dense.n_dense = _hip.DT_BF16, 0
    assert call(mods(2, distinct=True), 2, fa=dense) == _hip.ERR_SHAPE
    dense.n_dense, dense.dense_a = 4, (1 << 14) + 8
    assert call(mods(2, distinct=True), 2, fa=dense) == _hip.ERR_ALIGN
    dense.dense_a = 1 << 14
    w = np.ones(2, dtype=np.float32)
    weighted = _hip.Routes(slot=slot.ctypes.data, weight_sqrt=w.ctypes.data, slot_scale=None, n_route=1)
    assert call(mods(2, distinct=True), 2, fa=dense, rt=weighted) == _hip.ERR_UNSUPPORTED
    neg = mods(2, distinct=True)
    neg[1].a_block_off = -1
    assert call(neg, 2, fa=dense) == _hip.ERR_SHAPE
    assert call(mods(2), 2, fa=dense) == _hip.ERR_OVERLAP
    assert call(mods(2, x=(1 << 12) + 8), 2) == _hip.ERR_ALIGN               # x not 16-byte aligned
    assert call(mods(2, d_out=6), 2) == _hip.ERR_ALIGN                       # d_out * rank % 64
    assert call(mods(2, y=0), 2) == _hip.ERR_NULL
    assert call(mods(2, distinct=True), 2, wsb=256) == _hip.ERR_WORKSPACE
    assert call(mods(2), 2, ws=0) == _hip.ERR_WORKSPACE
    assert call(mods(2, seq=0), 2) == _hip.OK                                # nothing to do
    assert call(mods(2), 2, n_batch=0) == _hip.OK
    same_y = mods(2)                                                          # both write one output
    assert call(same_y, 2) == _hip.ERR_OVERLAP
    part = mods(2)
    part[1].y = (1 << 13) + 2 * 8 * 64 * 2 - 16                               # the last 16 bytes overlap
    assert call(part, 2) == _hip.ERR_OVERLAP
    far = mods(1)
    far[0].b_block_off = 10_000                                               # B past the end of a slot
    assert call(far, 1) == _hip.ERR_SHAPE
    # two modules over one x share one intermediate of 2 x 16 ranks; a third x adds its own
    wb = lib.lithe_lora_grouped_workspace_bytes
    arr = mods(3)
    arr[2].x = 1 << 14
    rows = 2 * 8
    assert wb(2, 3, arr, 16, 1, _hip.DT_BF16) == 256 + ((rows * 2 * 16 * 2 + 255) // 256) * 256 + \
        ((rows * 16 * 2 + 255) // 256) * 256
    assert wb(2, 9, arr, 16, 1, _hip.DT_BF16) == _hip.ERR_SHAPE
    assert wb(2, 3, arr, 16, 9, _hip.DT_BF16) == _hip.ERR_SHAPE                # 9 rank groups
    del words
