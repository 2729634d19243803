"""Prepared ``lithe_lora_delta`` calls: every argument fixed once, one C call per launch.

A serving loop that runs the same modules over the same buffers (the 342
linears of a FLUX step, or one captured HIP graph of them) builds one
``PreparedDelta`` per module and replays it: no descriptor building, no
dtype checks and no allocation on the hot path. Calls that run one after
another on one stream can share a workspace (``shared_workspace``).
"""
from __future__ import annotations

import ctypes
from typing import List, Optional, Sequence, Tuple

import torch

from . import _delta, _hip


def workspace_bytes(x_shape, d_out: int, rank: int, n_route: int, x_dtype: torch.dtype) -> int:
    n = _hip.load().lithe_lora_workspace_bytes(x_shape[0], x_shape[1], x_shape[2], d_out, rank, n_route,
                                               _hip.dtype_code(x_dtype))
    _hip.check(int(n) if n < 0 else 0, "lithe_lora_workspace_bytes")
    return int(n)


def shared_workspace(device, nbytes: int) -> torch.Tensor:
    """A zero-filled workspace (the counter region must start at zero; kernels keep it so)."""
    return torch.zeros(max(int(nbytes), 256), dtype=torch.uint8, device=device)


def shared_x_workspace_bytes(x_shape, d_outs: Sequence[int], rank: int, n_route: int, x_dtype: torch.dtype) -> int:
    """Workspace of ``lithe_lora_delta_shared_x``: the 256-byte head and one rank-r intermediate
    row of every module per token (the layout of a grouped call whose modules share one x)."""
    b, m, d_in = x_shape
    return group_workspace_bytes([(m, d_in, d) for d in d_outs], [0] * len(d_outs), b, rank, n_route, x_dtype)


class PreparedDelta:
    """y <- delta(x) for fixed tensors; see ``lithe_lora_delta`` in include/lithe_amd.h."""

    def __init__(self, x: torch.Tensor, y: torch.Tensor, *, rank: int, factors: _hip.Factors, route: _hip.Routes,
                 accumulate: bool, workspace: torch.Tensor, out_scale: float = 1.0,
                 mid_scale: Optional[torch.Tensor] = None, out_scale_vec: Optional[torch.Tensor] = None,
                 keep: Sequence = ()):
        _hip.require_gpu(x, y, workspace)
        if x.dim() != 3 or y.dim() != 3 or not x.is_contiguous() or not y.is_contiguous():
            raise ValueError("x and y must be contiguous (B, M, D) tensors")
        need = workspace_bytes(tuple(x.shape), y.shape[2], rank, route.n_route, x.dtype)
        if workspace.numel() < need:
            raise ValueError(f"workspace holds {workspace.numel()} bytes, the call needs {need}")
        self.x, self.y, self.workspace = x, y, workspace
        self._keep: List = [factors, route, mid_scale, out_scale_vec, *keep]
        self._lib = _hip.load()
        n_batch, seq, d_in = x.shape
        self._args = (
            _hip.ptr(x), _hip.dtype_code(x.dtype), n_batch, seq, d_in, _hip.ptr(y), _hip.dtype_code(y.dtype),
            y.shape[2], int(bool(accumulate)), int(rank), ctypes.byref(factors), ctypes.byref(route),
            _hip.ptr(mid_scale), ctypes.c_float(float(out_scale)), _hip.ptr(out_scale_vec),
            _hip.ptr(workspace), workspace.numel())
        self.tokens = n_batch * seq
        self.d_in, self.d_out = d_in, y.shape[2]

    def algorithmic_bytes(self) -> int:
        """x read + y read + y write (accumulate mode), the path's compulsory traffic."""
        e = self.x.element_size()
        return self.tokens * (self.d_in * e + 2 * self.d_out * self.y.element_size())

    def __call__(self, stream: Optional[ctypes.c_void_p] = None) -> None:
        rc = self._lib.lithe_lora_delta(*self._args, stream if stream is not None else _hip.stream_of(self.x.device))
        if rc:
            _hip.check(rc, "lithe_lora_delta")


def prepare_packed(x: torch.Tensor, y: torch.Tensor, bank_words: torch.Tensor, a_off: int, b_off: int,
                   num_levels: int, pools: Tuple[torch.Tensor, torch.Tensor], slots: torch.Tensor, rank: int,
                   scaling: float, workspace: torch.Tensor, accumulate: bool = True) -> PreparedDelta:
    """Prepared index-resident delta of one module read straight from a packed bank."""
    lut_a = _hip.lut_from_pools(pools[0], x.dtype)
    lut_b = _hip.lut_from_pools(pools[1], x.dtype)
    f = _delta.indexed_factors(_delta.packed_source(bank_words, num_levels, a_off),
                               _delta.packed_source(bank_words, num_levels, b_off), lut_a, lut_b)
    sl = slots.to(device=x.device, dtype=torch.int32).reshape(-1, 1).contiguous()
    return PreparedDelta(x, y, rank=rank, factors=f, route=_delta.routes(sl), accumulate=accumulate,
                         workspace=workspace, out_scale=scaling, keep=(sl, bank_words))


def prepare_dense(x: torch.Tensor, y: torch.Tensor, a: torch.Tensor, b: torch.Tensor, slots: torch.Tensor, rank: int,
                  scaling: float, workspace: torch.Tensor, accumulate: bool = True) -> PreparedDelta:
    """Prepared decoded-mode delta: stacked dense factors ``a`` (n, r, d_in) and ``b``
    (n, d_out, r) in the activation dtype (e.g. views from ``PackedBank.decode_stacked``);
    sample i uses factor pair ``slots[i]``. Same kernels and rounding chain as the
    index-resident call, so equal factors give bit-equal outputs."""
    _hip.require_gpu(a, b)
    if a.dtype != x.dtype or b.dtype != x.dtype or not a.is_contiguous() or not b.is_contiguous():
        raise ValueError("dense factors must be contiguous and in the activation dtype")
    if a.shape[0] != b.shape[0] or a.shape[1] != rank or b.shape[2] != rank or a.shape[2] != x.shape[2] \
            or b.shape[1] != y.shape[2]:
        raise ValueError(f"factor shapes {tuple(a.shape)}, {tuple(b.shape)} do not match x / y and rank {rank}")
    f = _delta.dense_factors(a, b)
    sl = slots.to(device=x.device, dtype=torch.int32).reshape(-1, 1).contiguous()
    return PreparedDelta(x, y, rank=rank, factors=f, route=_delta.routes(sl), accumulate=accumulate,
                         workspace=workspace, out_scale=scaling, keep=(sl, a, b))


class PreparedSharedX:
    """y_m <- y_m + delta_m(x) for modules that read one input (``lithe_lora_delta_shared_x``):
    one shrink over x for all of them, then their expands (one launch when the modules read one
    B source and table, else one per module)."""

    def __init__(self, x: torch.Tensor, ys: Sequence[torch.Tensor], factors: Sequence[_hip.Factors],
                 route: _hip.Routes, rank: int, out_scales: Sequence[float], workspace: torch.Tensor,
                 accumulate: bool = True, keep: Sequence = ()):
        _hip.require_gpu(x, workspace, *ys)
        if x.dim() != 3 or not x.is_contiguous() or any(y.dim() != 3 or not y.is_contiguous() for y in ys):
            raise ValueError("x and every y must be contiguous (B, M, D) tensors")
        n = len(ys)
        if not (n == len(factors) == len(out_scales)) or n < 1:
            raise ValueError("one factor set and one scale per output")
        if any(y.shape[:2] != x.shape[:2] or y.dtype != ys[0].dtype for y in ys):
            raise ValueError("every y must be (B, M, d_out) like x, in one dtype")
        need = shared_x_workspace_bytes(tuple(x.shape), [y.shape[2] for y in ys], rank, route.n_route, x.dtype)
        if workspace.numel() < need:
            raise ValueError(f"workspace holds {workspace.numel()} bytes, the call needs {need}")
        self.x, self.ys, self.workspace = x, list(ys), workspace
        self._f = (_hip.Factors * n)(*factors)
        self._y = (ctypes.c_void_p * n)(*[y.data_ptr() for y in ys])
        self._d = (ctypes.c_int64 * n)(*[y.shape[2] for y in ys])
        self._s = (ctypes.c_float * n)(*[float(v) for v in out_scales])
        self._keep: List = [route, *keep]
        self._lib = _hip.load()
        b, m, d_in = x.shape
        self._args = (_hip.ptr(x), _hip.dtype_code(x.dtype), b, m, d_in, n, self._y, _hip.dtype_code(ys[0].dtype),
                      self._d, int(bool(accumulate)), int(rank), self._f, ctypes.byref(route), None, self._s,
                      _hip.ptr(workspace), workspace.numel())
        self.tokens = b * m
        self.d_in = d_in

    def algorithmic_bytes(self) -> int:
        """x read once + every y read and written."""
        return self.tokens * (self.d_in * self.x.element_size() + sum(2 * y.shape[2] * y.element_size() for y in self.ys))

    def __call__(self, stream: Optional[ctypes.c_void_p] = None) -> None:
        rc = self._lib.lithe_lora_delta_shared_x(*self._args,
                                                 stream if stream is not None else _hip.stream_of(self.x.device))
        if rc:
            _hip.check(rc, "lithe_lora_delta_shared_x")


def prepare_packed_shared_x(x: torch.Tensor, ys: Sequence[torch.Tensor], bank_words: torch.Tensor,
                            offsets: Sequence[Tuple[int, int]], num_levels: int,
                            pools: Tuple[torch.Tensor, torch.Tensor], slots: torch.Tensor, rank: int, scaling: float,
                            workspace: torch.Tensor, accumulate: bool = True) -> PreparedSharedX:
    """Prepared index-resident deltas of the modules at ``offsets`` [(a_off, b_off)] of a packed
    bank, all reading ``x`` (e.g. to_q / to_k / to_v of one attention block)."""
    lut_a = _hip.lut_from_pools(pools[0], x.dtype)
    lut_b = _hip.lut_from_pools(pools[1], x.dtype)
    fs = [_delta.indexed_factors(_delta.packed_source(bank_words, num_levels, ao),
                                 _delta.packed_source(bank_words, num_levels, bo), lut_a, lut_b) for ao, bo in offsets]
    sl = slots.to(device=x.device, dtype=torch.int32).reshape(-1, 1).contiguous()
    return PreparedSharedX(x, ys, fs, _delta.routes(sl), rank, [scaling] * len(ys), workspace, accumulate,
                           keep=(sl, bank_words))


def group_workspace_bytes(shapes: Sequence[Tuple[int, int, int]], shared: Sequence[int], n_batch: int, rank: int,
                          n_route: int, x_dtype: torch.dtype) -> int:
    """Workspace of a grouped call: ``shapes`` [(seq, d_in, d_out)] per module; modules with equal
    ``shared`` keys read one input (``lithe_lora_grouped_workspace_bytes``)."""
    mods = (_hip.Module * len(shapes))()
    for i, ((seq, d_in, d_out), key) in enumerate(zip(shapes, shared)):
        mods[i].x = 16 * (key + 1)          # stands for the input's identity only
        mods[i].seq, mods[i].d_in, mods[i].d_out = seq, d_in, d_out
    n = _hip.load().lithe_lora_grouped_workspace_bytes(n_batch, len(shapes), mods, rank, n_route,
                                                       _hip.dtype_code(x_dtype))
    _hip.check(int(n) if n < 0 else 0, "lithe_lora_grouped_workspace_bytes")
    return int(n)


class PreparedGroup:
    """y_m <- y_m + delta_m(x_m) for up to 8 independent modules of one batch in one shrink and one
    expand launch (``lithe_lora_delta_grouped``); modules given the same x tensor share its shrink."""

    def __init__(self, xs: Sequence[torch.Tensor], ys: Sequence[torch.Tensor], factors: _hip.Factors,
                 offsets: Sequence[Tuple[int, int]], route: _hip.Routes, rank: int, out_scales: Sequence[float],
                 workspace: torch.Tensor, accumulate: bool = True, keep: Sequence = ()):
        n = len(xs)
        if not (n == len(ys) == len(offsets) == len(out_scales)) or not 1 <= n <= _hip.MAX_GROUP_MODULES:
            raise ValueError(f"a group holds 1 to {_hip.MAX_GROUP_MODULES} modules, each with x, y, offsets and a scale")
        _hip.require_gpu(workspace, *xs, *ys)
        b = xs[0].shape[0]
        for x, y in zip(xs, ys):
            if x.dim() != 3 or y.dim() != 3 or not x.is_contiguous() or not y.is_contiguous():
                raise ValueError("every x and y must be a contiguous (B, M, D) tensor")
            if x.shape[0] != b or y.shape[:2] != x.shape[:2] or x.dtype != xs[0].dtype or y.dtype != ys[0].dtype:
                raise ValueError("every module needs y (B, M, d_out) over its x (B, M, d_in), one batch and dtype")
        self.xs, self.ys, self.workspace = list(xs), list(ys), workspace
        self._m = (_hip.Module * n)()
        for i, (x, y, (ao, bo), s) in enumerate(zip(xs, ys, offsets, out_scales)):
            self._m[i].x, self._m[i].y = x.data_ptr(), y.data_ptr()
            self._m[i].seq, self._m[i].d_in, self._m[i].d_out = x.shape[1], x.shape[2], y.shape[2]
            self._m[i].a_block_off, self._m[i].b_block_off = int(ao), int(bo)
            self._m[i].out_scale = float(s)
        self._lib = _hip.load()
        need = self._lib.lithe_lora_grouped_workspace_bytes(b, n, self._m, rank, route.n_route,
                                                            _hip.dtype_code(xs[0].dtype))
        _hip.check(int(need) if need < 0 else 0, "lithe_lora_grouped_workspace_bytes")
        if workspace.numel() < need:
            raise ValueError(f"workspace holds {workspace.numel()} bytes, the call needs {need}")
        self._f = factors
        self._keep: List = [route, *keep]
        self._args = (n, self._m, _hip.dtype_code(xs[0].dtype), _hip.dtype_code(ys[0].dtype), b,
                      int(bool(accumulate)), int(rank), ctypes.byref(factors), ctypes.byref(route),
                      _hip.ptr(workspace), workspace.numel())
        self.tokens = b * max(x.shape[1] for x in xs)

    def algorithmic_bytes(self) -> int:
        """Every distinct x read once + every y read and written."""
        seen, total = set(), 0
        for x in self.xs:
            if x.data_ptr() not in seen:
                seen.add(x.data_ptr())
                total += x.numel() * x.element_size()
        return total + sum(2 * y.numel() * y.element_size() for y in self.ys)

    def __call__(self, stream: Optional[ctypes.c_void_p] = None) -> None:
        rc = self._lib.lithe_lora_delta_grouped(*self._args,
                                                stream if stream is not None else _hip.stream_of(self.xs[0].device))
        if rc:
            _hip.check(rc, "lithe_lora_delta_grouped")


def prepare_packed_group(xs: Sequence[torch.Tensor], ys: Sequence[torch.Tensor], bank_words: torch.Tensor,
                         offsets: Sequence[Tuple[int, int]], num_levels: int,
                         pools: Tuple[torch.Tensor, torch.Tensor], slots: torch.Tensor, rank: int, scaling: float,
                         workspace: torch.Tensor, accumulate: bool = True) -> PreparedGroup:
    """Prepared grouped index-resident deltas of the modules at ``offsets`` [(a_off, b_off)] of a
    packed bank, module m reading ``xs[m]`` and updating ``ys[m]``."""
    lut_a = _hip.lut_from_pools(pools[0], xs[0].dtype)
    lut_b = _hip.lut_from_pools(pools[1], xs[0].dtype)
    f = _delta.indexed_factors(_delta.packed_source(bank_words, num_levels, 0),
                               _delta.packed_source(bank_words, num_levels, 0), lut_a, lut_b)
    sl = slots.to(device=xs[0].device, dtype=torch.int32).reshape(-1, 1).contiguous()
    return PreparedGroup(xs, ys, f, offsets, _delta.routes(sl), rank, [scaling] * len(xs), workspace, accumulate,
                         keep=(sl, bank_words))


def prepare_stacked_group(xs: Sequence[torch.Tensor], ys: Sequence[torch.Tensor], stacked: torch.Tensor, n_sel: int,
                          offsets: Sequence[Tuple[int, int]], slots: torch.Tensor, rank: int, scaling: float,
                          workspace: torch.Tensor, accumulate: bool = True) -> PreparedGroup:
    """Prepared grouped decoded-mode deltas: ``stacked`` is a ``decode_packed_stacked`` buffer of
    ``n_sel`` selections (module m's A / B at elements n_sel * 64 * a_off / b_off of it, offsets
    [(a_off, b_off)] of the bank layout); sample i uses selection ``slots[i]``. Each module gets
    what ``prepare_dense`` over its views of the buffer computes."""
    _hip.require_gpu(stacked)
    if stacked.dim() != 1 or not stacked.is_contiguous() or stacked.dtype != xs[0].dtype:
        raise ValueError("stacked factors must be a flat contiguous buffer in the activation dtype")
    if n_sel < 1:
        raise ValueError("n_sel must be >= 1")
    for (ao, bo), x, y in zip(offsets, xs, ys):
        end = max(n_sel * 64 * int(ao) + n_sel * rank * x.shape[2], n_sel * 64 * int(bo) + n_sel * y.shape[2] * rank)
        if int(ao) < 0 or int(bo) < 0 or end > stacked.numel():
            raise ValueError(f"offsets ({ao}, {bo}) reach past the stacked buffer of {stacked.numel()} elements")
    f = _hip.Factors()
    f.kind = _hip.FACTOR_DENSE
    f.dense_dtype = _hip.dtype_code(stacked.dtype)
    f.dense_a = f.dense_b = stacked.data_ptr()
    f.n_dense = int(n_sel)
    sl = slots.to(device=xs[0].device, dtype=torch.int32).reshape(-1, 1).contiguous()
    return PreparedGroup(xs, ys, f, offsets, _delta.routes(sl), rank, [scaling] * len(xs), workspace, accumulate,
                         keep=(sl, stacked))
