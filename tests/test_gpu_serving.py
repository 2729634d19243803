"""GPU checks of the serving helpers on a FLUX-shaped toy transformer:

* ``wrap_index`` (per-layer int32 index stacks, the reference's serving/_common.py:294-306)
  and ``wrap_bank`` (slots read from the packed bank) give bit-equal outputs (same factors,
  same kernels and plan);
* the shared-input groups (q / k / v in one grouped call sharing a shrink) match the unfused
  model at the bf16 delta tolerance (the shrink plans split K differently);
* decoded mode through ``install_decoded_bank`` matches the index-resident model at that
  tolerance (decoded factors are summed from fp32 pools, the fused path's from bf16 pools);
* ``torch.compile`` traces the wrapped model without graph breaks (the delta is one
  ``lithe_amd::`` op) and its result equals eager bit for bit.
"""
import copy

import pytest
import torch

from lithe_amd import serving
from lithe_amd.kernels import PackedBank

from helpers import random_adapter, rel, to_np
from toy_flux import ToyFlux, target_modules

pytestmark = pytest.mark.gpu


def _setup(seed=0, n_ad=4):
    torch.manual_seed(seed)
    model = ToyFlux().cuda().bfloat16()
    mods = target_modules(model)
    ads = [random_adapter(mods, rank=16, seed=200 + s) for s in range(n_ad)]
    bank, words = PackedBank.from_adapters(ads, "cuda")
    for w in words:
        bank.add(w)
    g = torch.Generator(device="cuda").manual_seed(seed + 1)
    h = torch.randn(3, 64, 256, device="cuda", generator=g).bfloat16()
    c = torch.randn(3, 24, 256, device="cuda", generator=g).bfloat16()
    return model, ads, bank, h, c


def test_wrap_index_equals_wrap_bank():
    model, ads, bank, h, c = _setup()
    m1, m2 = copy.deepcopy(model), copy.deepcopy(model)
    w1 = serving.wrap_index(m1, ads, "cuda")
    w2 = serving.wrap_bank(m2, bank)
    assign = torch.tensor([2, 0, 3], dtype=torch.int32, device="cuda")
    serving.set_assign(w1, assign)
    serving.set_assign(w2, assign)
    with torch.no_grad():
        base = model(h, c)
        o1, o2 = m1(h, c), m2(h, c)
    assert torch.equal(o1, o2)
    assert rel(to_np(o1), to_np(base)) > 1e-3          # the adapters changed the output


def test_shared_input_groups_match_unfused():
    model, ads, bank, h, c = _setup(1)
    m1, m2 = copy.deepcopy(model), copy.deepcopy(model)
    w1 = serving.wrap_bank(m1, bank)
    w2 = serving.wrap_bank(m2, bank, fuse_shared_inputs=True)
    assign = torch.tensor([1, 3, 1], dtype=torch.int32, device="cuda")
    serving.set_assign(w1, assign)
    serving.set_assign(w2, assign)
    with torch.no_grad():
        o1, o2 = m1(h, c), m2(h, c)
        o3 = m2(h, c)                                  # second pass: no stale group state
    assert rel(to_np(o2), to_np(o1)) < 2e-3
    assert torch.equal(o2, o3)
    # a member called with another input than its group's pending one recomputes
    q = m2.transformer_blocks[0].attn.to_q(h)
    k_other = m2.transformer_blocks[0].attn.to_k(h + 1)
    with torch.no_grad():
        k_ref = m1.transformer_blocks[0].attn.to_k(h + 1)
    assert rel(to_np(k_other), to_np(k_ref)) < 2e-3 and q.shape == h.shape


def test_decoded_bank_mode_matches_index_resident():
    model, ads, bank, h, c = _setup(2)
    m1, m2 = copy.deepcopy(model), copy.deepcopy(model)
    w1 = serving.wrap_bank(m1, bank)
    w2 = serving.wrap_decoded(m2, [n for n, _, _ in target_modules(model)])
    sel = [3, 0]
    serving.install_decoded_bank(w2, bank, sel)
    serving.set_assign(w1, torch.tensor([3, 0, 3], dtype=torch.int32, device="cuda"))
    serving.set_assign(w2, torch.tensor([0, 1, 0], dtype=torch.int32, device="cuda"))   # pairs of sel
    with torch.no_grad():
        o1, o2 = m1(h, c), m2(h, c)
    assert rel(to_np(o2), to_np(o1)) < 1e-2


def test_torch_compile_traces_the_lithe_ops():
    model, ads, bank, h, c = _setup(3)
    w = serving.wrap_bank(model, bank)
    serving.set_assign(w, torch.tensor([0, 2, 1], dtype=torch.int32, device="cuda"))
    torch._dynamo.reset()
    with torch.no_grad():
        eager = model(h, c)
        explain = torch._dynamo.explain(model)(h, c)
        compiled = torch.compile(model, backend="aot_eager", fullgraph=True)(h, c)
    assert explain.graph_break_count == 0
    assert torch.equal(compiled, eager)


def test_shared_input_group_rank64_and_stale_state():
    """Shared-input groups at rank 64 (4 rank groups per module, 12 for a q / k / v group: each
    workgroup carries one module's groups) match the unfused model; a pending member output is
    not reused after the routing or a bank slot changed, nor for another tensor."""
    torch.manual_seed(4)
    model = ToyFlux().cuda().bfloat16()
    mods = target_modules(model)
    ads = [random_adapter(mods, rank=64, seed=400 + s) for s in range(3)]
    bank, words = PackedBank.from_adapters(ads, "cuda")
    for w in words:
        bank.add(w)
    g = torch.Generator(device="cuda").manual_seed(5)
    h = torch.randn(2, 48, 256, device="cuda", generator=g).bfloat16()
    c = torch.randn(2, 16, 256, device="cuda", generator=g).bfloat16()
    m1, m2 = copy.deepcopy(model), copy.deepcopy(model)
    w1 = serving.wrap_bank(m1, bank)
    w2 = serving.wrap_bank(m2, bank, fuse_shared_inputs=True)
    a0 = torch.tensor([2, 0], dtype=torch.int32, device="cuda")
    serving.set_assign(w1, a0)
    serving.set_assign(w2, a0)
    with torch.no_grad():
        assert rel(to_np(m2(h, c)), to_np(m1(h, c))) < 2e-3
        attn1, attn2 = m1.transformer_blocks[0].attn, m2.transformer_blocks[0].attn
        attn2.to_q(h)                                    # k and v now pending for (h, a0)
        a1 = torch.tensor([1, 1], dtype=torch.int32, device="cuda")
        serving.set_assign(w1, a1)
        serving.set_assign(w2, a1)
        assert rel(to_np(attn2.to_k(h)), to_np(attn1.to_k(h))) < 2e-3      # recomputed under a1
        attn2.to_q(h)                                    # pending again, then slot 1 is rewritten
        saved = bank.words[1].clone()
        bank.words[1].copy_(bank.words[0])
        bank.generation += 1
        assert rel(to_np(attn2.to_v(h)), to_np(attn1.to_v(h))) < 2e-3
        attn2.to_q(h)
        h2 = h.clone()                                   # equal values, another tensor
        bank.words[1].copy_(saved)
        bank.generation += 1
        assert rel(to_np(attn2.to_k(h2)), to_np(attn1.to_k(h2))) < 2e-3


def _grouped_double(block, groups, prefix, h, c):
    """DoubleBlock.forward of tests/toy_flux.py with every stage's deltas in one grouped call."""
    q, k, v, cq, ck, cv = groups[(prefix, "proj")]([h, h, h, c, c, c])
    ho, co = groups[(prefix, "out")]([q * torch.sigmoid(k) + v, cq * torch.sigmoid(ck) + cv])
    h, c = h + ho, c + co
    up_h, up_c = groups[(prefix, "up")]([h, c])
    act = block.ff.net[1]
    dn_h, dn_c = groups[(prefix, "down")]([act(up_h), act(up_c)])
    return h + dn_h, c + dn_c


def _grouped_forward(model, groups, h, c):
    for i, b in enumerate(model.transformer_blocks):
        h, c = _grouped_double(b, groups, f"transformer_blocks.{i}.", h, c)
    h = torch.cat([c, h], dim=1)
    for i, b in enumerate(model.single_transformer_blocks):
        q, k, v = groups[(f"single_transformer_blocks.{i}.", "proj")]([h, h, h])
        h = h + (q * torch.sigmoid(k) + v)
    return h


def test_stage_groups_equal_per_module_layers_and_compile(monkeypatch):
    """A forward that issues each block stage as one grouped call (serving.stage_groups) equals the
    wrapped model's per-module forward bit for bit when both plans split K the same way, and
    torch.compile traces it (the grouped delta is one lithe_amd:: op) with no graph break."""
    monkeypatch.setenv("LITHE_SHRINK_KS", "1")
    model, ads, bank, h, c = _setup(6)
    w = serving.wrap_bank(model, bank)
    serving.set_assign(w, torch.tensor([3, 1, 0], dtype=torch.int32, device="cuda"))
    groups = serving.stage_groups(w)
    with torch.no_grad():
        per_module = model(h, c)
        grouped = _grouped_forward(model, groups, h, c)
        assert torch.equal(grouped, per_module)
        torch._dynamo.reset()
        explain = torch._dynamo.explain(_grouped_forward)(model, groups, h, c)
        compiled = torch.compile(_grouped_forward, backend="aot_eager", fullgraph=True)(model, groups, h, c)
    assert explain.graph_break_count == 0
    assert torch.equal(compiled, per_module)


def test_attention_groups_equal_per_module_layers(monkeypatch):
    """wrap_bank(group_attention=True): one grouped call per double-block attention entry, every
    output bit-identical to the per-module layers with the same K split; a projection called outside
    its attention (or with another tensor) runs its own forward."""
    monkeypatch.setenv("LITHE_SHRINK_KS", "1")
    model, ads, bank, h, c = _setup(6)
    m1, m2 = copy.deepcopy(model), copy.deepcopy(model)
    w1 = serving.wrap_bank(m1, bank)
    w2 = serving.wrap_bank(m2, bank, group_attention=True)
    groups = {id(m._group): m._group for m in w2.values() if isinstance(m, serving.AttentionMember)}
    assert len(groups) == len(m2.transformer_blocks)
    assign = torch.tensor([3, 1, 0], dtype=torch.int32, device="cuda")
    serving.set_assign(w1, assign)
    serving.set_assign(w2, assign)
    with torch.no_grad():
        o1, o2 = m1(h, c), m2(h, c)
        o3 = m2(h, c)
    assert torch.equal(o2, o1) and torch.equal(o3, o1)
    assert all(g.calls == 2 for g in groups.values())
    assert all(p is None for g in groups.values() for p in g._pending)     # every output was taken
    with torch.no_grad():
        k_alone = m2.transformer_blocks[0].attn.add_k_proj(c)
        k_ref = m1.transformer_blocks[0].attn.add_k_proj(c)
        g0 = m2.transformer_blocks[0].attn.to_q._group
        before = g0.calls
        pos = m2.transformer_blocks[0].attn(h, c)              # positional arguments reach the hook too
        ref = m1.transformer_blocks[0].attn(h, c)
    assert torch.equal(k_alone, k_ref)
    assert g0.calls == before + 1 and all(torch.equal(p, r) for p, r in zip(pos, ref))


def test_grouped_serving_under_inference_mode(monkeypatch):
    """Shared-input and attention groups under torch.inference_mode (inference tensors keep no
    version counter): the same outputs as the per-module layers."""
    monkeypatch.setenv("LITHE_SHRINK_KS", "1")
    model, ads, bank, h, c = _setup(7)
    m1, m2 = copy.deepcopy(model), copy.deepcopy(model)
    w1 = serving.wrap_bank(m1, bank)
    w2 = serving.wrap_bank(m2, bank, fuse_shared_inputs=True, group_attention=True)
    assign = torch.tensor([0, 2, 3], dtype=torch.int32, device="cuda")
    serving.set_assign(w1, assign)
    serving.set_assign(w2, assign)
    with torch.inference_mode():
        hi, ci = h.clone(), c.clone()
        o1, o2 = m1(hi, ci), m2(hi, ci)
    assert torch.equal(o2, o1)
