"""Host logic of the gated LoRA (no GPU): ``install`` stacks a fused projection's A's and wraps the
layer's method with its B's in shard order (plm/gated_lora.py:60-89); calls outside ``rows_from`` run
the inner method; CPU calls take the reference's unfused composition and equal the oracle bit for
bit (the same operations)."""

from __future__ import annotations

import torch
import torch.nn.functional as F

import oracle
from plm_amd.gated_lora import GatedLoraMethod, install, rows_from


class _Linear(torch.nn.Module):
    def __init__(self, n, k, seed):
        super().__init__()
        g = torch.Generator().manual_seed(seed)
        self.weight = torch.nn.Parameter((0.02 * torch.randn(n, k, generator=g)).bfloat16(), requires_grad=False)
        self.quant_method = _Plain()


class _Plain:
    def apply(self, layer, x, bias=None):
        return F.linear(x, layer.weight, bias)


def _model():
    m = torch.nn.Module()
    m.layers = torch.nn.ModuleList([torch.nn.Module()])
    m.layers[0].self_attn = torch.nn.Module()
    m.layers[0].self_attn.qkv_proj = _Linear(64 + 16 + 16, 32, 1)
    m.layers[0].self_attn.o_proj = _Linear(32, 64, 2)
    return m


def _adapter(rank=4):
    g = torch.Generator().manual_seed(9)
    t = {}
    for proj, n, k in (("q_proj", 64, 32), ("k_proj", 16, 32), ("v_proj", 16, 32), ("o_proj", 32, 64)):
        t[f"layers.0.self_attn.{proj}.lora_a"] = (0.1 * torch.randn(rank, k, generator=g)).bfloat16()
        t[f"layers.0.self_attn.{proj}.lora_b"] = (0.1 * torch.randn(n, rank, generator=g)).bfloat16()
    return t


def test_install_stacks_shards_in_order_and_routes_gated_rows():
    m, t = _model(), _adapter()
    install(m, t)
    qkv = m.layers[0].self_attn.qkv_proj
    assert torch.equal(qkv.lora_a, torch.cat([t[f"layers.0.self_attn.{p}.lora_a"] for p in ("q_proj", "k_proj", "v_proj")]))
    assert isinstance(qkv.quant_method, GatedLoraMethod) and len(qkv.quant_method.lora_bs) == 3
    assert [b.shape[0] for b in qkv.quant_method.lora_bs] == [64, 16, 16]
    x = torch.randn(9, 32, generator=torch.Generator().manual_seed(4)).bfloat16()
    plain = qkv.quant_method.apply(qkv, x)
    assert torch.equal(plain, F.linear(x, qkv.weight))
    with rows_from(3):
        gated = qkv.quant_method.apply(qkv, x)
    ref = oracle.gated_lora(x, qkv.weight.data, qkv.lora_a, qkv.quant_method.lora_bs, 3)
    assert torch.equal(gated, ref)
    assert torch.equal(gated[:3], plain[:3]) and not torch.equal(gated[3:], plain[3:])
    o = m.layers[0].self_attn.o_proj
    with rows_from(0):
        assert torch.equal(o.quant_method.apply(o, torch.ones(2, 64).bfloat16()),
                           oracle.gated_lora(torch.ones(2, 64).bfloat16(), o.weight.data, o.lora_a,
                                             o.quant_method.lora_bs, 0))
    with rows_from(None):
        assert torch.equal(o.quant_method.apply(o, torch.ones(2, 64).bfloat16()),
                           F.linear(torch.ones(2, 64).bfloat16(), o.weight))
