"""Host-side layer plumbing (CPU): which q/k/v wrappers fuse, and what fusion keeps.

The grouping rule follows multi_lora/layers.py:128-142: the q, k and v
projections of one attention block (same parent module) form a group only
when all three are wrapped.  Fusion makes each layer's weight a view of one
concatenated weight (multi_lora/layers.py:101-111) and leaves every
layer's output unchanged.
"""

import torch
from torch import nn

from multi_lora_amd import LinearWithLoRA, fuse_qkv_projections


def _wrap(names_dims, in_dim=32):
    torch.manual_seed(0)
    return {n: LinearWithLoRA(nn.Linear(in_dim, d, bias=False)) for n, d in names_dims}


def test_only_complete_blocks_fuse():
    ws = _wrap([("model.layers.0.self_attn.q_proj", 64), ("model.layers.0.self_attn.k_proj", 16),
                ("model.layers.0.self_attn.v_proj", 16),
                ("model.layers.1.self_attn.q_proj", 64), ("model.layers.1.self_attn.k_proj", 16),
                ("model.layers.1.self_attn.v_proj", 16),
                ("model.layers.2.self_attn.q_proj", 64), ("model.layers.2.self_attn.k_proj", 16),
                ("model.layers.2.self_attn.o_proj", 64),
                ("q_proj", 64), ("k_proj", 16), ("v_proj", 16)])
    assert fuse_qkv_projections(ws) == 2
    fused = [n for n, w in ws.items() if w.qkv_group is not None]
    assert sorted(fused) == sorted(f"model.layers.{i}.self_attn.{p}_proj" for i in (0, 1) for p in "qkv")
    g0 = ws["model.layers.0.self_attn.q_proj"].qkv_group
    assert g0 is ws["model.layers.0.self_attn.v_proj"].qkv_group
    assert g0 is not ws["model.layers.1.self_attn.q_proj"].qkv_group


def test_fused_weights_are_views_in_q_k_v_order_and_outputs_hold():
    p = "blk.attn."
    ws = _wrap([(p + "v_proj", 8), (p + "q_proj", 24), (p + "k_proj", 8)])
    x = torch.randn(3, 1, 32)
    before = {n: w(x).clone() for n, w in ws.items()}
    assert fuse_qkv_projections(ws) == 1
    grp = ws[p + "q_proj"].qkv_group
    assert grp.weight.shape == (40, 32)
    base = grp.weight.data_ptr()
    for leaf, start in (("q_proj", 0), ("k_proj", 24), ("v_proj", 32)):
        w = ws[p + leaf]
        assert w.qkv_slice[0] == start
        assert w.base_layer.weight.data_ptr() == base + start * 32 * grp.weight.element_size()
    for n, w in ws.items():
        torch.testing.assert_close(w(x), before[n], rtol=1e-6, atol=1e-6)
    # prefill shapes (more than one token) take each layer's own GEMM
    xs = torch.randn(2, 5, 32)
    torch.testing.assert_close(ws[p + "k_proj"](xs), xs @ ws[p + "k_proj"].base_layer.weight.T)


def test_gate_up_groups_and_all_shape_fusion():
    """gate/up siblings fuse like q/k/v; with all_shapes a prefill-shaped input
    takes the fused GEMM too, and outputs still equal the separate layers."""
    from multi_lora_amd import fuse_gate_up_projections

    p = "model.layers.0.mlp."
    ws = _wrap([(p + "gate_proj", 48), (p + "up_proj", 48), (p + "down_proj", 32),
                ("model.layers.1.mlp.gate_proj", 48)])
    xs = torch.randn(2, 5, 32)
    before = {n: w(xs).clone() for n, w in ws.items() if "layers.0" in n}
    assert fuse_gate_up_projections(ws) == 1
    grp = ws[p + "gate_proj"].qkv_group
    assert grp is ws[p + "up_proj"].qkv_group and grp.all_shapes
    assert ws[p + "down_proj"].qkv_group is None and ws["model.layers.1.mlp.gate_proj"].qkv_group is None
    for n in before:
        out = ws[n](xs)
        torch.testing.assert_close(out, before[n], rtol=1e-6, atol=1e-6)
    assert grp._cached_x is xs  # the fused GEMM ran for the prefill shape
    # already grouped wrappers are left alone
    assert fuse_gate_up_projections(ws) == 0
