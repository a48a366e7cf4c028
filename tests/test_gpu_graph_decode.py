"""Graph-captured decode step (GPU), re-expressing the reference's pins
(multi_lora/tests/test_graph_decode.py:61-106) on this package's decoder:
replaying the captured step gives the logits of running the same step
directly, step after step, and capture allocates none of the resident
tensors anew.  The LoRA launches in the step are the HIP kernels.
"""

import pytest
import torch

from multi_lora_amd import AdapterWeights, MultiLoRAManager
from multi_lora_amd.decoder import Decoder, DecoderConfig
from multi_lora_amd.graph_decode import DecodeStep, capture_graph

pytestmark = pytest.mark.gpu

BATCH = 4
CHECK_STEPS = 5
PROJ = ("self_attn.q_proj", "self_attn.k_proj", "self_attn.v_proj", "self_attn.o_proj", "mlp.gate_proj",
        "mlp.up_proj", "mlp.down_proj")


def build(dtype):
    torch.manual_seed(0)
    cfg = DecoderConfig()
    model = Decoder(cfg).to("cuda", dtype).eval()
    adapters = {}
    for j, name in enumerate(("a", "b")):
        g = torch.Generator().manual_seed(10 + j)
        mods = {}
        for layer in range(cfg.num_hidden_layers):
            for p in PROJ:
                lin = model.get_submodule(f"layers.{layer}.{p}")
                mods[f"layers.{layer}.{p}"] = ((torch.randn(8, lin.in_features, generator=g) * 0.05).to(dtype),
                                               (torch.randn(lin.out_features, 8, generator=g) * 0.05).to(dtype))
        adapters[name] = AdapterWeights(rank=8, scaling=2.0, modules=mods)
    mgr = MultiLoRAManager.from_adapters(model, adapters, max_loras_per_batch=4, max_lora_rank=16)
    return mgr, cfg


def prefill(mgr, cfg, names, start, max_len):
    ids = (torch.arange(start, device="cuda") % cfg.vocab_size).repeat(BATCH, 1)
    mask = torch.ones_like(ids)
    step = DecodeStep.new(mgr, BATCH, start, max_len)
    first = step.prefill(mgr, ids, mask, names)
    step.input_ids.copy_(first)
    mgr._setup_forward_batch(names, seq_lens=[1] * BATCH)
    return step


@pytest.mark.parametrize("dtype,atol", [(torch.float32, 1e-4), (torch.bfloat16, 5e-2)])
def test_replay_matches_direct_run(dev, dtype, atol):
    mgr, cfg = build(dtype)
    names = ["a", "b", "a", "b"]
    start = 6
    max_len = start + 3 + 1 + CHECK_STEPS + 2
    with torch.inference_mode():
        recorded = prefill(mgr, cfg, names, start, max_len)
        graph, out = capture_graph(mgr, recorded)
        direct = prefill(mgr, cfg, names, start, max_len)
        for step in range(CHECK_STEPS):
            graph.replay()
            mine = out.logits[:, -1]
            theirs = direct.run(mgr).logits[:, -1]
            gap = (mine.float() - theirs.float()).abs().max().item()
            assert gap <= atol, f"step {step}: max|diff| = {gap}"
            nxt = mine.argmax(dim=-1, keepdim=True)
            recorded.input_ids.copy_(nxt)
            direct.input_ids.copy_(nxt)


def test_capture_reuses_same_tensors(dev):
    mgr, cfg = build(torch.bfloat16)
    names = ["a", "b", "a", "b"]
    start = 6
    with torch.inference_mode():
        step = prefill(mgr, cfg, names, start, start + 8)
        tensors = lambda: [t.data_ptr() for t in (step.kv.keys[0], step.input_ids, step.position_ids,  # noqa: E731
                                                  step.kv_pos, step.attn_mask)]
        before = tensors()
        capture_graph(mgr, step)
        assert tensors() == before
        assert int(step.kv_pos.item()) == start and int(step.position_ids[0, 0].item()) == start


def test_adapters_change_the_decode(dev):
    """The captured step really applies each row's adapter: rows with
    different adapters but the same prompt get different logits, rows with
    the same adapter get the same."""
    mgr, cfg = build(torch.float32)
    with torch.inference_mode():
        step = prefill(mgr, cfg, ["a", "b", "a", None], 6, 12)
        graph, out = capture_graph(mgr, step)
        graph.replay()
        lg = out.logits[:, -1].float()
        assert torch.allclose(lg[0], lg[2], atol=1e-5)
        assert (lg[0] - lg[1]).abs().max() > 1e-3 and (lg[0] - lg[3]).abs().max() > 1e-3
