"""lithe_lora_delta_noalloc: the per-sample delta with its rank-r intermediate in the library's
static scratch instead of a workspace, called through the C ABI. It runs the kernels of
lithe_lora_delta with the same plan, so its outputs must equal lithe_lora_delta's bit for bit:
checked on two calls in a row, the second with a smaller input (the scratch keeps the first call's
contents), in write and accumulate mode, with one and two route entries, and with a slot id out of
range (recorded in the caller's error word by both entry points, the sample left alone).
The host-side rejections (an intermediate beyond the scratch, bad arguments) are checked on the
CPU in tests/test_abi.py."""
import ctypes

import pytest
import torch

from lithe_amd.kernels import PackedBank, _delta, _hip

from helpers import random_adapter

pytestmark = pytest.mark.gpu
RANK = 16


@pytest.fixture(scope="module")
def bank():
    ads = [random_adapter([("q", 3072, 3072), ("up", 512, 1280)], rank=RANK, seed=900 + s) for s in range(5)]
    bank, words = PackedBank.from_adapters(ads, "cuda")
    for w in words:
        bank.add(w)
    return bank


def _factors(bank, name):
    _, _, _, a_off, b_off = bank.layout.module(name)
    lut_a = _hip.lut_from_pools(bank.pool_a, torch.bfloat16)
    lut_b = _hip.lut_from_pools(bank.pool_b, torch.bfloat16)
    return _delta.indexed_factors(_delta.packed_source(bank.words, 3, a_off), _delta.packed_source(bank.words, 3, b_off),
                                  lut_a, lut_b)


def _noalloc(x, y, f, route, accumulate, scale, err):
    rc = _hip.load().lithe_lora_delta_noalloc(
        _hip.ptr(x), _hip.dtype_code(x.dtype), x.shape[0], x.shape[1], x.shape[2], _hip.ptr(y),
        _hip.dtype_code(y.dtype), y.shape[2], int(accumulate), RANK, ctypes.byref(f), ctypes.byref(route), None,
        ctypes.c_float(scale), None, _hip.ptr(err), _hip.stream_of(x.device))
    _hip.check(rc, "lithe_lora_delta_noalloc")


def _workspace(x, y, f, route, accumulate, scale, ws):
    lib = _hip.load()
    need = lib.lithe_lora_workspace_bytes(x.shape[0], x.shape[1], x.shape[2], y.shape[2], RANK, route.n_route,
                                          _hip.dtype_code(x.dtype))
    assert ws.numel() >= need
    rc = lib.lithe_lora_delta(_hip.ptr(x), _hip.dtype_code(x.dtype), x.shape[0], x.shape[1], x.shape[2], _hip.ptr(y),
                              _hip.dtype_code(y.dtype), y.shape[2], int(accumulate), RANK, ctypes.byref(f),
                              ctypes.byref(route), None, ctypes.c_float(scale), None, _hip.ptr(ws), ws.numel(),
                              _hip.stream_of(x.device))
    _hip.check(rc, "lithe_lora_delta")


@pytest.mark.parametrize("name,d_in,d_out,n_route", [("q", 3072, 3072, 1), ("up", 512, 1280, 2)])
def test_noalloc_equals_workspace_call(bank, name, d_in, d_out, n_route):
    f = _factors(bank, name)
    g = torch.Generator(device="cuda").manual_seed(d_out + n_route)
    ws = torch.zeros(64 << 20, dtype=torch.uint8, device="cuda")
    err = torch.zeros(1, dtype=torch.int32, device="cuda")
    for n_batch, seq in ((6, 700), (3, 130)):              # the second call is smaller
        x = torch.randn(n_batch, seq, d_in, device="cuda", generator=g).bfloat16()
        y0 = torch.randn(n_batch, seq, d_out, device="cuda", generator=g).bfloat16()
        slots = torch.randint(0, 5, (n_batch, n_route), device="cuda", generator=g, dtype=torch.int32)
        if n_route > 1:
            slots[0, 1] = -1                                # an empty mixture entry
        w = torch.rand(n_batch, n_route, device="cuda", generator=g).sqrt()
        route = _delta.routes(slots, w if n_route > 1 else None)
        for acc in (False, True):
            y_ws, y_na = y0.clone(), y0.clone()
            _workspace(x, y_ws, f, route, acc, 0.75, ws)
            _noalloc(x, y_na, f, route, acc, 0.75, err)
            torch.cuda.synchronize()
            assert torch.equal(y_na, y_ws), (n_batch, seq, acc)
            if acc:
                assert not torch.equal(y_na, y0)
    assert int(err.item()) == 0
    flags = ctypes.c_int32(0)
    _hip.check(_hip.load().lithe_workspace_errors(_hip.ptr(ws), ctypes.byref(flags), 1, None), "errors")
    assert flags.value == 0


def test_noalloc_records_bad_slot_in_callers_error_word(bank):
    f = _factors(bank, "q")
    g = torch.Generator(device="cuda").manual_seed(5)
    x = torch.randn(3, 64, 3072, device="cuda", generator=g).bfloat16()
    y0 = torch.randn(3, 64, 3072, device="cuda", generator=g).bfloat16()
    slots = torch.tensor([[1], [bank.num_slots], [4]], dtype=torch.int32, device="cuda")   # sample 1: no such slot
    route = _delta.routes(slots)
    err = torch.zeros(1, dtype=torch.int32, device="cuda")
    y_na = y0.clone()
    _noalloc(x, y_na, f, route, True, 1.0, err)
    ws = torch.zeros(1 << 20, dtype=torch.uint8, device="cuda")
    y_ws = y0.clone()
    _workspace(x, y_ws, f, route, True, 1.0, ws)
    torch.cuda.synchronize()
    assert int(err.item()) == 1
    assert torch.equal(y_na, y_ws) and torch.equal(y_na[1], y0[1])

