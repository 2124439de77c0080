"""A tiny attention-only model written the way model code calls attention
(a module-level ``scaled_dot_product_attention(q, k, v, cache=, scale=,
mask=)`` looked up at call time, a plain ``KVCache`` per layer from
``make_cache``), for the kvattn.patch_model / kvcache.install tests.  Its
own attention is dense float32 torch: the test-side reference, and the
function patch_model keeps as the base for dense K/V."""
from __future__ import annotations

import sys

import torch

NAME = __name__


def scaled_dot_product_attention(queries, keys, values, cache=None, scale=1.0, mask=None, sinks=None):
    q, k, v = queries.float(), keys.float(), values.float()
    rep = q.shape[1] // k.shape[1]
    k = k.repeat_interleave(rep, dim=1)
    v = v.repeat_interleave(rep, dim=1)
    s = (q * scale) @ k.transpose(-1, -2)
    L, N = s.shape[-2], s.shape[-1]
    if isinstance(mask, str):
        keep = torch.arange(N - L, N, device=s.device)[:, None] >= torch.arange(N, device=s.device)[None]
        s = s.masked_fill(~keep, float("-inf"))
    elif mask is not None:
        s = s.masked_fill(~mask, float("-inf"))
    return (torch.softmax(s, -1) @ v).to(queries.dtype)


class KVCache:
    """The unquantized cache: dense K/V concatenated along the sequence."""

    def __init__(self):
        self.keys = self.values = None
        self.offset = 0

    def update_and_fetch(self, k, v):
        self.keys = k if self.keys is None else torch.cat([self.keys, k], 2)
        self.values = v if self.values is None else torch.cat([self.values, v], 2)
        self.offset += k.shape[2]
        return self.keys, self.values


class Attention(torch.nn.Module):
    def __init__(self, dim, heads, kv_heads, head_dim, seed):
        super().__init__()
        g = torch.Generator().manual_seed(seed)
        w = lambda o, i: torch.nn.Parameter(torch.randn(o, i, generator=g) / i ** 0.5, requires_grad=False)
        self.h, self.hk, self.d = heads, kv_heads, head_dim
        self.wq, self.wk = w(heads * head_dim, dim), w(kv_heads * head_dim, dim)
        self.wv, self.wo = w(kv_heads * head_dim, dim), w(dim, heads * head_dim)

    def forward(self, x, cache):
        B, L, _ = x.shape
        split = lambda t, n: t.reshape(B, L, n, self.d).transpose(1, 2)
        q = split(x @ self.wq.T, self.h)
        k, v = cache.update_and_fetch(split(x @ self.wk.T, self.hk), split(x @ self.wv.T, self.hk))
        attend = sys.modules[NAME].scaled_dot_product_attention      # looked up per call
        o = attend(q, k, v, cache=cache, scale=self.d ** -0.5, mask="causal" if L > 1 else None)
        return x + o.transpose(1, 2).reshape(B, L, -1) @ self.wo.T


class Model(torch.nn.Module):
    def __init__(self, dim=256, heads=8, kv_heads=2, head_dim=128, layers=2):
        super().__init__()
        self.layers = torch.nn.ModuleList(Attention(dim, heads, kv_heads, head_dim, 10 + i) for i in range(layers))

    def make_cache(self):
        return [KVCache() for _ in self.layers]

    def forward(self, x, cache):
        for layer, c in zip(self.layers, cache):
            x = layer(x, c)
        return x


def run(model, x, prefill: int):
    """Prefill x[:, :prefill] ([B, L, dim]), then feed the remaining
    positions one token per step (a forced decode); returns the outputs at
    the prefill's last position and at every decode step."""
    cache = model.make_cache()
    outs = [model(x[:, :prefill], cache)[:, -1:]]
    for t in range(prefill, x.shape[1]):
        outs.append(model(x[:, t:t + 1], cache))
    return torch.cat(outs, 1)
