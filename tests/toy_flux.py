"""A FLUX-shaped toy transformer (module paths of diffusers' FluxTransformer2DModel, tiny widths)
for the serving tests: double blocks with image / text attention projections and feed-forwards,
single blocks with q / k / v."""
import torch
from torch import nn


class _Proj(nn.Module):
    def __init__(self, d_in, d_out):
        super().__init__()
        self.proj = nn.Linear(d_in, d_out)


class _Attn(nn.Module):
    """Called like diffusers' FLUX attention: ``attn(hidden_states=..., encoder_hidden_states=...)``,
    every projection reading the tensors passed in (a toy mixing stands in for attention)."""

    def __init__(self, d, context=True):
        super().__init__()
        self.to_q, self.to_k, self.to_v = nn.Linear(d, d), nn.Linear(d, d), nn.Linear(d, d)
        if context:     # single-block attention is projection-only (no to_out), as in FLUX
            self.to_out = nn.ModuleList([nn.Linear(d, d)])
            self.add_q_proj, self.add_k_proj, self.add_v_proj = nn.Linear(d, d), nn.Linear(d, d), nn.Linear(d, d)
            self.to_add_out = nn.Linear(d, d)

    def forward(self, hidden_states, encoder_hidden_states=None):
        h = hidden_states
        mixed = self.to_q(h) * torch.sigmoid(self.to_k(h)) + self.to_v(h)
        if encoder_hidden_states is None:
            return mixed
        c = encoder_hidden_states
        mixed_c = self.add_q_proj(c) * torch.sigmoid(self.add_k_proj(c)) + self.add_v_proj(c)
        return self.to_out[0](mixed), self.to_add_out(mixed_c)


class _FF(nn.Module):
    def __init__(self, d, ff):
        super().__init__()
        self.net = nn.ModuleList([_Proj(d, ff), nn.GELU(), nn.Linear(ff, d)])

    def forward(self, x):
        return self.net[2](self.net[1](self.net[0].proj(x)))


class DoubleBlock(nn.Module):
    def __init__(self, d, ff):
        super().__init__()
        self.attn = _Attn(d)
        self.ff = _FF(d, ff)
        self.ff_context = _FF(d, ff)

    def forward(self, h, c):
        dh, dc = self.attn(hidden_states=h, encoder_hidden_states=c)
        h, c = h + dh, c + dc
        return h + self.ff(h), c + self.ff_context(c)


class SingleBlock(nn.Module):
    def __init__(self, d):
        super().__init__()
        self.attn = _Attn(d, context=False)

    def forward(self, h):
        return h + self.attn(hidden_states=h)


class ToyFlux(nn.Module):
    def __init__(self, d=256, ff=512, n_double=2, n_single=2):
        super().__init__()
        self.transformer_blocks = nn.ModuleList([DoubleBlock(d, ff) for _ in range(n_double)])
        self.single_transformer_blocks = nn.ModuleList([SingleBlock(d) for _ in range(n_single)])

    def forward(self, h, c):
        for b in self.transformer_blocks:
            h, c = b(h, c)
        h = torch.cat([c, h], dim=1)
        for b in self.single_transformer_blocks:
            h = b(h)
        return h


TARGETS = ("attn.to_q", "attn.to_k", "attn.to_v", "attn.to_out.0", "attn.add_q_proj", "attn.add_k_proj",
           "attn.add_v_proj", "attn.to_add_out", "ff.net.0.proj", "ff.net.2", "ff_context.net.0.proj",
           "ff_context.net.2")


def target_modules(model: nn.Module):
    """(path, d_in, d_out) of the model's FLUX target linears, in model order."""
    out = []
    for name, mod in model.named_modules():
        if isinstance(mod, nn.Linear) and any(name.endswith(t) for t in TARGETS):
            out.append((name, mod.in_features, mod.out_features))
    return out
