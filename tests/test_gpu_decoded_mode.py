"""Decoded-mode serving on the GPU: one-launch decode-on-swap into stacked per-module factors
(lithe_decode_stacked), bit-exact against per-slot decode + stack; the decoded-mode delta over
those factors equals the index-resident delta bit for bit (same factors after the bf16 cast,
same kernels and rounding chain)."""
import ctypes

import numpy as np
import pytest
import torch

from lithe_amd.kernels import PackedBank, _delta, _hip, split_decoded
from lithe_amd.kernels.prepared import prepare_dense, prepare_packed, shared_workspace, workspace_bytes

from helpers import SMALL, flux_modules, random_adapter

pytestmark = pytest.mark.gpu


def _bank(mods, n, seed):
    ads = [random_adapter(mods, rank=16, seed=seed + s) for s in range(n)]
    bank, words = PackedBank.from_adapters(ads, "cuda")
    for w in words:
        bank.add(w)
    return ads, bank


@pytest.mark.parametrize("mods,sel", [(SMALL, [2, 0, 2, 1]), (flux_modules(), [3, 1])])
def test_decode_stacked_matches_per_slot_decode(mods, sel):
    _, bank = _bank(mods, 4, 50)
    st = bank.decode_stacked(sel)
    torch.cuda.synchronize()
    per = [bank.decode(s) for s in sel]
    for name in bank.layout.names:
        a, b = st[name]
        assert a.is_contiguous() and b.is_contiguous()
        assert torch.equal(a, torch.stack([p[name][0] for p in per]))
        assert torch.equal(b, torch.stack([p[name][1] for p in per]))


def test_decode_stacked_flags_an_inconsistent_table():
    _, bank = _bank(SMALL, 2, 60)
    lay = bank.layout
    table = lay.ingest_table().clone()
    table[-1, 1] += 1000                      # last factor claims more blocks than the layout has
    tdev = table.cuda()
    n_sel = 2
    guard = 4096
    out = torch.full((n_sel * lay.total_blocks * 64 + guard,), 7.0, dtype=torch.bfloat16, device="cuda")
    err = torch.zeros(1, dtype=torch.int32, device="cuda")
    src = _delta.packed_source(bank.words, 3, 0)
    lut_a = _hip.lut_from_pools(bank.pool_a, torch.float32)
    lut_b = _hip.lut_from_pools(bank.pool_b, torch.float32)
    slots = torch.tensor([0, 1], dtype=torch.int32, device="cuda")
    rc = _hip.load().lithe_decode_stacked(ctypes.byref(src), _hip.ptr(slots), n_sel, lay.total_blocks,
                                          table.shape[0], _hip.ptr(tdev), _hip.ptr(lay.sides_on("cuda")),
                                          ctypes.byref(lut_a), ctypes.byref(lut_b), _hip.ptr(out),
                                          _hip.DT_BF16, _hip.ptr(err), _hip.stream_of(out.device))
    assert rc == 0
    torch.cuda.synchronize()
    assert int(err.item()) & 4
    assert (out[-guard:] == 7.0).all()        # nothing written past the output


def test_decoded_mode_delta_matches_index_resident_and_oracle():
    """(a) Factors decoded from pools rounded to bf16 are the index path's in-kernel factors
    (shared.py casts the pools to the activation dtype before the level sum), so where both
    plans give every wave a whole K range (d_in = 3072 with >= 2048 token groups) the dense
    delta over them equals the index-resident delta bit for bit. Where K is split over waves
    the dense plan cuts it at other points (4-block LDS pieces instead of 16 / 48), so only the
    fp32 grouping differs. (b) Decoded mode proper (bulk decode with fp32 pools,
    packed.py:205-222) on every shape against the oracle's LitheLinear chain (module.py:145-156:
    x A^T, then B^T, then * scaling, then + base, each rounded to bf16)."""
    from lithe_amd.kernels import decode_packed_stacked, split_stacked
    from oracle import codebook as ocb
    from oracle import decode as odec
    from oracle import delta as odelta
    from helpers import rel, to_np
    mods = [("q", 3072, 3072), ("up", 3072, 12288), ("down", 12288, 3072)]
    ads, bank = _bank(mods, 5, 70)
    slot_list = [4, 1, 1, 0]
    slots = torch.tensor(slot_list, dtype=torch.int32, device="cuda")
    uniq = [4, 1, 0]
    sel = torch.tensor([uniq.index(s) for s in slot_list], dtype=torch.int32, device="cuda")
    u = torch.tensor(uniq, dtype=torch.int32, device="cuda")
    rp = (bank.pool_a.bfloat16().float(), bank.pool_b.bfloat16().float())
    st_bf = split_stacked(decode_packed_stacked(bank.words, u, bank.layout, *rp), bank.layout, len(uniq))
    st = bank.decode_stacked(uniq)
    pools = (bank.pool_a.bfloat16(), bank.pool_b.bfloat16())
    gen = torch.Generator(device="cuda").manual_seed(3)

    def run(name, di, do, seq):
        x = torch.randn(4, seq, di, device="cuda", generator=gen).bfloat16()
        y0 = torch.randn(4, seq, do, device="cuda", generator=gen).bfloat16()
        ws = shared_workspace("cuda", workspace_bytes((4, seq, di), do, 16, 1, torch.bfloat16))
        _, _, _, a_off, b_off = bank.layout.module(name)
        yi, yb, yd = y0.clone(), y0.clone(), y0.clone()
        prepare_packed(x, yi, bank.words, a_off, b_off, 3, pools, slots, 16, 0.75, ws)()
        prepare_dense(x, yb, st_bf[name][0], st_bf[name][1], sel, 16, 0.75, ws)()
        prepare_dense(x, yd, st[name][0], st[name][1], sel, 16, 0.75, ws)()
        torch.cuda.synchronize()
        return x, y0, yi, yb, yd

    for name, di, do in mods[:2]:
        _, y0, yi, yb, _ = run(name, di, do, 8192)
        assert torch.equal(yi, yb), name
        assert not torch.equal(yi, y0)
    pa, pb = ocb.twin_pools()
    for name, di, do in mods:
        for seq in (77, 130):
            x, y0, yi, yb, yd = run(name, di, do, seq)
            assert rel(to_np(yb), to_np(yi)) < 2e-3, (name, seq)
            got, xn, y0n = to_np(yd), to_np(x), to_np(y0)
            for i, s in enumerate(slot_list):
                a = odec.decode(ads[s].indices[name]["A"], (16, di), pa)
                b = odec.decode(ads[s].indices[name]["B"], (do, 16), pb)
                want = odelta.lithe_linear(xn[i], y0n[i], a, b, 0.75, "bf16")
                assert rel(got[i], want) < 2e-3, (name, seq, i)
                assert rel(got[i] - y0n[i], want - y0n[i]) < 5e-2, (name, seq, i)   # the delta itself


def test_decode_stacked_from_int16_source_matches_packed():
    """The generic kernel (unpacked index kinds) writes the same stacked layout: block-major int16
    indices of three adapters (decode_int16's source) against the packed bank's stacked decode."""
    from lithe_amd.kernels import flat_indices
    ads, bank = _bank(SMALL, 3, 80)
    lay = bank.layout
    sel = [1, 2, 0, 1]
    want = bank.decode_stacked(sel)
    idx = torch.from_numpy(np.stack([flat_indices(ad, lay).astype(np.int16) for ad in ads])).cuda()
    src = _hip.IndexSrc()
    src.base = idx.data_ptr()
    src.kind = _hip.IDX_BLOCK_I16
    src.num_levels = 3
    src.slot_stride = idx.stride(0)
    src.level_stride = 0
    src.block_off = 0
    src.n_slots = 3
    out = torch.empty(len(sel) * lay.total_blocks * 64, dtype=torch.bfloat16, device="cuda")
    slots = torch.tensor(sel, dtype=torch.int32, device="cuda")
    lut_a = _hip.lut_from_pools(bank.pool_a, torch.float32)
    lut_b = _hip.lut_from_pools(bank.pool_b, torch.float32)
    table = lay.table_on("cuda")
    rc = _hip.load().lithe_decode_stacked(ctypes.byref(src), _hip.ptr(slots), len(sel), lay.total_blocks,
                                          table.shape[0], _hip.ptr(table), _hip.ptr(lay.sides_on("cuda")),
                                          ctypes.byref(lut_a), ctypes.byref(lut_b), _hip.ptr(out), _hip.DT_BF16,
                                          None, _hip.stream_of(out.device))
    assert rc == 0
    from lithe_amd.kernels import split_stacked
    got = split_stacked(out, lay, len(sel))
    torch.cuda.synchronize()
    for name in lay.names:
        assert torch.equal(got[name][0], want[name][0]) and torch.equal(got[name][1], want[name][1])


@pytest.mark.parametrize("accumulate,dtype", [(True, torch.bfloat16), (False, torch.bfloat16), (True, torch.float32)])
def test_grouped_decoded_mode_equals_per_module_dense_calls(monkeypatch, accumulate, dtype):
    """lithe_lora_delta_grouped over dense factors in the stacked decode layout (one buffer; module
    m's A / B at n_sel * 64 * a_off / b_off): with the shrink's K split fixed, every module's output
    equals the per-module decoded-mode call over its views of the buffer bit for bit. Covers
    modules sharing one x (one workgroup per tile and module), different widths, an empty route,
    and fp32 activations and factors (no grouped kernel: job by job through the per-call ones)."""
    from lithe_amd.kernels import decode_packed_stacked
    from lithe_amd.kernels.prepared import prepare_stacked_group
    monkeypatch.setenv("LITHE_SHRINK_KS", "1")
    mods = [("q", 512, 512), ("k", 512, 512), ("v", 512, 512), ("up", 512, 2048), ("down", 2048, 512)]
    _, bank = _bank(mods, 4, 90)
    uniq = [3, 0, 2]
    u = torch.tensor(uniq, dtype=torch.int32, device="cuda")
    buf = decode_packed_stacked(bank.words, u, bank.layout, bank.pool_a, bank.pool_b, dtype=dtype)
    st = bank.decode_stacked(uniq, dtype=dtype)
    sel = torch.tensor([2, -1, 0, 1], dtype=torch.int32, device="cuda")
    gen = torch.Generator(device="cuda").manual_seed(17)
    shape = {n: (di, do) for n, di, do in mods}
    spec = [("q", 96), ("k", 96), ("v", 96), ("up", 40), ("down", 33)]
    xq = torch.randn(4, 96, 512, device="cuda", generator=gen).to(dtype)
    xs = [xq if n in ("q", "k", "v") else torch.randn(4, m, shape[n][0], device="cuda", generator=gen).to(dtype)
          for n, m in spec]
    y0 = [torch.randn(4, m, shape[n][1], device="cuda", generator=gen).to(dtype) for n, m in spec]
    ws = shared_workspace("cuda", 16 << 20)
    offs = [bank.layout.module(n)[3:5] for n, _ in spec]
    got = [y.clone() for y in y0]
    prepare_stacked_group(xs, got, buf, len(uniq), offs, sel, 16, 0.75, ws, accumulate)()
    want = [y.clone() for y in y0]
    for (n, _), x, y in zip(spec, xs, want):
        prepare_dense(x, y, st[n][0], st[n][1], sel, 16, 0.75, ws, accumulate)()
    torch.cuda.synchronize()
    for (n, _), g, w, y in zip(spec, got, want, y0):
        assert torch.equal(g, w), n
        assert not torch.equal(g[0], y[0]), n
    assert _hip.workspace_errors() == 0


def test_grouped_decoded_mode_rejects_weighted_routes():
    from lithe_amd.kernels import decode_packed_stacked
    from lithe_amd.kernels.prepared import PreparedGroup
    _, bank = _bank(SMALL, 2, 95)
    u = torch.tensor([1, 0], dtype=torch.int32, device="cuda")
    buf = decode_packed_stacked(bank.words, u, bank.layout, bank.pool_a, bank.pool_b)
    name, d_in, d_out = SMALL[0]
    x = torch.zeros(2, 16, d_in, dtype=torch.bfloat16, device="cuda")
    y = torch.zeros(2, 16, d_out, dtype=torch.bfloat16, device="cuda")
    f = _hip.Factors()
    f.kind = _hip.FACTOR_DENSE
    f.dense_dtype = _hip.dtype_code(buf.dtype)
    f.dense_a = f.dense_b = buf.data_ptr()
    f.n_dense = 2
    slots = torch.tensor([[0], [1]], dtype=torch.int32, device="cuda")
    w = torch.ones(2, 1, device="cuda")
    call = PreparedGroup([x], [y], f, [bank.layout.module(name)[3:5]], _delta.routes(slots, w), 16, [1.0],
                         shared_workspace("cuda", 1 << 20), keep=(slots, w, buf))
    with pytest.raises(ValueError):
        call()
    # the prepared form refuses offsets that reach past the buffer, and a buffer of another dtype
    from lithe_amd.kernels.prepared import prepare_stacked_group
    ao, bo = bank.layout.module(name)[3:5]
    with pytest.raises(ValueError):
        prepare_stacked_group([x], [y], buf, 2, [(ao, bank.layout.total_blocks)], slots, 16, 1.0,
                              shared_workspace("cuda", 1 << 20))
    with pytest.raises(ValueError):
        prepare_stacked_group([x], [y], buf.float(), 2, [(ao, bo)], slots, 16, 1.0, shared_workspace("cuda", 1 << 20))


def test_random_grouped_decoded_mode_equals_per_module(monkeypatch):
    """Seeded random grouped decoded-mode calls: ranks 16-128 (one to eight rank groups), one to
    four modules with their own inputs and token counts or one shared x, 12,288-wide inputs, empty
    routes, write and accumulate mode, against per-module dense calls over views of the same
    stacked buffer with the K split fixed: bit for bit."""
    from lithe_amd.kernels import decode_packed_stacked, split_stacked
    from lithe_amd.kernels.prepared import prepare_stacked_group
    monkeypatch.setenv("LITHE_SHRINK_KS", "1")
    rng = np.random.default_rng(5)
    ws = shared_workspace("cuda", 64 << 20)
    for n in range(24):
        rank = int(rng.choice([16, 32, 48, 64, 128]))
        n_mod = int(rng.integers(1, 5))
        share = n_mod > 1 and bool(rng.integers(0, 2))
        d_in0 = 12288 if rng.integers(0, 5) == 0 else int(rng.integers(1, 17)) * 64
        mods = [(f"m{m}", d_in0 if share or m == 0 else int(rng.integers(1, 17)) * 64, int(rng.integers(2, 300)) * 4)
                for m in range(n_mod)]
        batch = int(rng.integers(1, 5))
        seq0 = int(rng.integers(1, 200))
        seqs = [seq0 if share else int(rng.integers(1, 200)) for _ in range(n_mod)]
        n_ad = int(rng.integers(1, 5))
        ads = [random_adapter([(nm, di, do) for nm, di, do in mods], rank=rank, seed=int(rng.integers(0, 1 << 30)))
               for _ in range(n_ad)]
        bank, words = PackedBank.from_adapters(ads, "cuda")
        for w in words:
            bank.add(w)
        uniq = sorted(set(rng.integers(0, n_ad, int(rng.integers(1, n_ad + 1))).tolist()))
        u = torch.tensor(uniq, dtype=torch.int32, device="cuda")
        buf = decode_packed_stacked(bank.words, u, bank.layout, bank.pool_a, bank.pool_b)
        st = split_stacked(buf, bank.layout, len(uniq))
        sel = torch.tensor(rng.integers(-1, len(uniq), batch), dtype=torch.int32, device="cuda")
        gen = torch.Generator(device="cuda").manual_seed(int(rng.integers(0, 1 << 30)))
        xs = [torch.randn(batch, s, di, device="cuda", generator=gen).bfloat16() for (_, di, _), s in zip(mods, seqs)]
        if share:
            xs = [xs[0]] * n_mod
        y0 = [torch.randn(batch, s, do, device="cuda", generator=gen).bfloat16() for (_, _, do), s in zip(mods, seqs)]
        acc, scale = bool(rng.integers(0, 2)), float(rng.choice([1.0, 0.5]))
        desc = (n, rank, share, mods, seqs, batch, uniq, sel.tolist(), acc)
        got = [y.clone() for y in y0]
        offs = [bank.layout.module(nm)[3:5] for nm, _, _ in mods]
        prepare_stacked_group(xs, got, buf, len(uniq), offs, sel, rank, scale, ws, acc)()
        want = [y.clone() for y in y0]
        for (nm, _, _), x, y in zip(mods, xs, want):
            prepare_dense(x, y, st[nm][0], st[nm][1], sel, rank, scale, ws, acc)()
        torch.cuda.synchronize()
        for m, (g, w) in enumerate(zip(got, want)):
            assert torch.equal(g, w), (desc, m)
        assert _hip.workspace_errors() == 0, desc
