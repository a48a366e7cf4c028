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


def test_mixed_step_with_adapters_equals_separate_runs(dev):
    """The packed serving step of the 32-layer benchmark, on the small model:
    2 prompts and 3 decode rows in one forward, each row with its adapter
    (HIP kernels, one segment table over the packed rows), give the logits of
    running the prompts and the decode rows through the manager separately."""
    from multi_lora_amd.decoder import StaticKV

    mgr, cfg = build(torch.float32)
    g = torch.Generator().manual_seed(7)
    prompts = torch.randint(0, cfg.vocab_size, (2, 6), generator=g).to("cuda")
    history = torch.randint(0, cfg.vocab_size, (3, 4), generator=g).to("cuda")
    nxt = torch.randint(0, cfg.vocab_size, (3, 1), generator=g).to("cuda")
    names_p, names_d = ["a", "b"], ["b", None, "a"]
    with torch.inference_mode():
        want_p = mgr.forward_with_lora(input_ids=prompts, lora_names=names_p, seq_lens=[6, 6],
                                       use_cache=False).logits[:, -1]
        kv_ref = StaticKV(cfg, 3, 8, "cuda", torch.float32)
        mgr.forward_with_lora(input_ids=history, lora_names=names_d, seq_lens=[4] * 3, past_key_values=kv_ref,
                              cache_position=torch.arange(4, device="cuda"))
        kv = StaticKV(cfg, 3, 8, "cuda", torch.float32)
        for layer in range(cfg.num_hidden_layers):
            kv.keys[layer].copy_(kv_ref.keys[layer])
            kv.values[layer].copy_(kv_ref.values[layer])
        pos = torch.tensor([4], device="cuda")
        mask = (torch.arange(8, device="cuda") <= pos).view(1, 1, 1, -1).expand(3, 1, 1, 8)
        want_d = mgr.forward_with_lora(input_ids=nxt, lora_names=names_d, seq_lens=[1] * 3, attention_mask=mask,
                                       position_ids=pos.view(1, 1).expand(3, 1), past_key_values=kv_ref,
                                       cache_position=pos).logits[:, 0]
        mgr._setup_forward_batch(names_p + names_d, seq_lens=[6, 6, 1, 1, 1])
        got = mgr.model.forward_mixed(prompts, nxt, kv, pos)
    torch.testing.assert_close(got[:2], want_p, atol=1e-4, rtol=1e-4)
    torch.testing.assert_close(got[2:], want_d, atol=1e-4, rtol=1e-4)
    assert (want_d[0] - want_d[1]).abs().max() > 1e-3  # the adapters matter


@pytest.mark.parametrize("dtype,atol", [(torch.float32, 1e-4), (torch.bfloat16, 6e-2)])
def test_fused_norms_equal_the_torch_norms(dev, dtype, atol):
    """``fuse_rmsnorm`` routes the decoder's norms, and its residual add +
    norm (``add_forward``), through the HIP kernels; the logits of a prefill
    and of a packed mixed step equal the model's own torch norms (the HIP
    norm rounds once where the torch one rounds the fp32 result once too,
    so fp32 agrees to rounding and bf16 within a few units)."""
    from multi_lora_amd.decoder import StaticKV
    from multi_lora_amd.kernels.rmsnorm import fuse_rmsnorm

    torch.manual_seed(0)
    cfg = DecoderConfig()
    plain = Decoder(cfg).to("cuda", dtype).eval()
    for mod in plain.modules():
        if type(mod).__name__.endswith("RMSNorm"):
            with torch.no_grad():
                mod.weight.copy_(1.0 + 0.1 * torch.randn_like(mod.weight))
    fused = Decoder(cfg).to("cuda", dtype).eval()
    fused.load_state_dict(plain.state_dict())
    assert fuse_rmsnorm(fused) == 2 * cfg.num_hidden_layers + 1
    g = torch.Generator().manual_seed(5)
    ids = torch.randint(0, cfg.vocab_size, (2, 7), generator=g).to("cuda")
    nxt = torch.randint(0, cfg.vocab_size, (3, 1), generator=g).to("cuda")
    pos = torch.tensor([3], device="cuda")
    with torch.inference_mode():
        torch.testing.assert_close(fused(input_ids=ids, use_cache=False).logits.float(),
                                   plain(input_ids=ids, use_cache=False).logits.float(), atol=atol, rtol=atol)
        got = fused.forward_mixed(ids, nxt, StaticKV(cfg, 3, 8, "cuda", dtype), pos)
        want = plain.forward_mixed(ids, nxt, StaticKV(cfg, 3, 8, "cuda", dtype), pos)
    torch.testing.assert_close(got.float(), want.float(), atol=atol, rtol=atol)


@pytest.mark.parametrize("dtype,atol", [(torch.float32, 2e-4), (torch.bfloat16, 6e-2)])
def test_mixed_step_matches_oracle_backend(dev, dtype, atol):
    """The 32-layer benchmark's packed step on the small model, configured as
    the benchmark configures it (q|k|v and gate|up fused on every shape, one
    multi-slice LoRA call each; the manager's HIP norms): its logits against
    the same model whose LoRA deltas come from the oracle's per-segment
    PyTorch backend (oracle/lora_ref.py, restating
    multi_lora/backend/torch_backend.py:17-90), layer by layer through the
    whole forward."""
    from multi_lora_amd import fuse_gate_up_projections, fuse_qkv_projections
    from multi_lora_amd.decoder import StaticKV
    from oracle.lora_ref import TorchLoRABackend

    mgr, cfg = build(dtype)
    layers = cfg.num_hidden_layers
    assert fuse_qkv_projections(mgr.lora_wrappers, all_shapes=True) == layers
    assert fuse_gate_up_projections(mgr.lora_wrappers) == layers
    g = torch.Generator().manual_seed(9)
    prompts = torch.randint(0, cfg.vocab_size, (2, 6), generator=g).to("cuda")
    nxt = torch.randint(0, cfg.vocab_size, (3, 1), generator=g).to("cuda")
    pos = torch.tensor([4], device="cuda")
    names = ["a", "b", "b", None, "a"]

    def step(names=names):
        mgr._setup_forward_batch(names, seq_lens=[6, 6, 1, 1, 1])
        with torch.inference_mode():
            return mgr.model.forward_mixed(prompts, nxt, StaticKV(cfg, 3, 8, "cuda", dtype), pos).float()

    got = step()
    hip_backend = mgr._lora_backend
    mgr._lora_backend = TorchLoRABackend()
    try:
        want = step()
    finally:
        mgr._lora_backend = hip_backend
    torch.testing.assert_close(got, want, atol=atol, rtol=atol)
    mgr._lora_backend = hip_backend
    assert torch.equal(step(), got)  # the HIP step again, bit for bit
    if dtype == torch.float32:  # the deltas move the logits far beyond the tolerance
        assert (got - step([None] * 5)).abs().max() > 50 * atol
