"""CPU checks of the serving helpers: target selection, bank-backed wrapping of a FLUX-shaped
model (with and without shared-input groups) and routing propagation. No kernel runs here."""
import pytest
import torch

from lithe_amd import serving
from lithe_amd.kernels import IndexLoRALinear, PackedBank, PackedLayout

from toy_flux import ToyFlux, target_modules


def _bank(model):
    mods = target_modules(model)
    lay = PackedLayout.from_modules([{"name": n, "shape_a": [16, di], "shape_b": [do, 16]} for n, di, do in mods])
    return PackedBank(lay, "cpu", capacity=2)


def test_target_selection_counts():
    model = ToyFlux(n_double=2, n_single=3)
    paths = [n for n, _, _ in target_modules(model)]
    assert len(paths) == 2 * 12 + 3 * 3          # the 19 x 12 + 38 x 3 = 342 rule of FLUX.1-dev, scaled down
    extra = paths + ["single_transformer_blocks.0.proj_mlp", "norm_out.linear"]
    assert serving.select_paths(extra, "attn-ff") == paths
    assert serving.select_paths(extra) == extra
    with pytest.raises(ValueError):
        serving.select_paths(extra, "nope")


@pytest.mark.parametrize("fuse", [False, True])
def test_wrap_bank_structure_and_assign(fuse):
    model = ToyFlux()
    bank = _bank(model)
    wrapped = serving.wrap_bank(model, bank, fuse_shared_inputs=fuse)
    assert len(wrapped) == len(target_modules(ToyFlux()))
    members = [p for p, m in wrapped.items() if isinstance(m, serving.SharedInputMember)]
    if fuse:
        # 2 double blocks x (img q/k/v + txt q/k/v) + 2 single blocks x q/k/v
        assert len(members) == 2 * 6 + 2 * 3
        assert model.transformer_blocks[0].attn.to_k is wrapped["transformer_blocks.0.attn.to_k"]
    else:
        assert not members and all(isinstance(m, IndexLoRALinear) for m in wrapped.values())
    assign = torch.tensor([1, 0, 1], dtype=torch.int32)
    serving.set_assign(wrapped, assign)
    assert all(m.assign is assign for m in wrapped.values())
    lead = model.single_transformer_blocks[1].attn.to_q
    assert (lead.layer if fuse else lead).assign is assign


@pytest.mark.parametrize("fuse", [False, True])
def test_stage_groups_structure(fuse):
    """stage_groups: per double block the proj (6), out (2), up (2) and down (2) stages, per single
    block its q / k / v, members in call order (shared-input stand-ins resolved to their layers)."""
    model = ToyFlux(n_double=2, n_single=3)
    wrapped = serving.wrap_bank(model, _bank(model), fuse_shared_inputs=fuse)
    groups = serving.stage_groups(wrapped)
    assert len(groups) == 2 * 4 + 3
    g = groups[("transformer_blocks.1.", "proj")]
    names = ["attn.to_q", "attn.to_k", "attn.to_v", "attn.add_q_proj", "attn.add_k_proj", "attn.add_v_proj"]
    assert [l.base for l in g.layers] == [getattr(wrapped["transformer_blocks.1." + n], "base") for n in names]
    assert len(groups[("single_transformer_blocks.2.", "proj")].layers) == 3
    assert len(groups[("transformer_blocks.0.", "down")].layers) == 2
    with pytest.raises(ValueError):
        serving.StageGroup([])


@pytest.mark.parametrize("fuse", [False, True])
def test_wrap_bank_attention_groups_structure(fuse):
    """group_attention: each double block's six q / k / v projections become stand-ins of one
    AttentionGroup hooked on its attention module; single blocks keep their q / k / v as shared-input
    groups (with fuse_shared_inputs) or plain layers; routing reaches every layer."""
    model = ToyFlux(n_double=2, n_single=2)
    wrapped = serving.wrap_bank(model, _bank(model), fuse_shared_inputs=fuse, group_attention=True)
    att = [p for p, m in wrapped.items() if isinstance(m, serving.AttentionMember)]
    shared = [p for p, m in wrapped.items() if isinstance(m, serving.SharedInputMember)]
    assert len(att) == 2 * 6 and all(p.startswith("transformer_blocks.") for p in att)
    assert len(shared) == (2 * 3 if fuse else 0)
    groups = {id(wrapped[p]._group) for p in att}
    assert len(groups) == 2
    attn = model.transformer_blocks[1].attn
    assert attn.add_k_proj is wrapped["transformer_blocks.1.attn.add_k_proj"]
    assert len(attn._forward_pre_hooks) == 1
    assign = torch.tensor([0, 1], dtype=torch.int32)
    serving.set_assign(wrapped, assign)
    assert all(m.assign is assign for m in wrapped.values())
    assert len(serving.stage_groups(wrapped)) == 2 * 4 + 2
    with pytest.raises(ValueError):
        serving.AttentionGroup(attn, [wrapped[att[0]].layer])
