"""The decoder around the LoRA path (CPU, fp32, no LoRA): its static KV
cache must make token-by-token decoding equal to one prefill over the same
tokens, and a 4-D boolean mask must act as given."""

import torch

from multi_lora_amd.decoder import Decoder, DecoderConfig, StaticKV


def model():
    torch.manual_seed(0)
    return Decoder(DecoderConfig(vocab_size=97, hidden_size=64, intermediate_size=96, num_hidden_layers=2,
                                 num_attention_heads=4, num_key_value_heads=2)).eval()


@torch.inference_mode()
def test_incremental_decode_equals_prefill():
    m = model()
    ids = torch.randint(0, 97, (3, 9), generator=torch.Generator().manual_seed(1))
    full = m(input_ids=ids, use_cache=False).logits
    kv = StaticKV(m.config, 3, 16, "cpu", torch.float32)
    m(input_ids=ids[:, :4], past_key_values=kv, cache_position=torch.arange(4))
    grid = torch.arange(16)
    for t in range(4, 9):
        pos = torch.tensor([t])
        mask = (grid <= pos).view(1, 1, 1, -1).expand(3, 1, 1, 16)
        out = m(input_ids=ids[:, t:t + 1], attention_mask=mask, position_ids=pos.view(1, 1).expand(3, 1),
                past_key_values=kv, cache_position=pos).logits
        torch.testing.assert_close(out[:, 0], full[:, t], atol=2e-5, rtol=2e-5)


@torch.inference_mode()
def test_padding_mask_hides_positions():
    """A masked-out prompt position changes nothing when its token changes."""
    m = model()
    ids = torch.randint(0, 97, (2, 6), generator=torch.Generator().manual_seed(2))
    mask = torch.ones(2, 6, dtype=torch.long)
    mask[:, 1] = 0
    a = m(input_ids=ids, attention_mask=mask, use_cache=False).logits[:, -1]
    ids2 = ids.clone()
    ids2[:, 1] = (ids2[:, 1] + 5) % 97
    b = m(input_ids=ids2, attention_mask=mask, use_cache=False).logits[:, -1]
    torch.testing.assert_close(a, b)


@torch.inference_mode()
def test_mixed_step_equals_separate_prefill_and_decode():
    """One packed step (2 prompts of 7 tokens, then 3 decode rows at position
    5 over their own caches) gives the logits of running the prompts and the
    decode rows through the ordinary forward separately, and writes the same
    KV entries."""
    m = model()
    g = torch.Generator().manual_seed(3)
    prompts = torch.randint(0, 97, (2, 7), generator=g)
    history = torch.randint(0, 97, (3, 5), generator=g)
    nxt = torch.randint(0, 97, (3, 1), generator=g)
    want_p = m(input_ids=prompts, use_cache=False).logits[:, -1]
    kv_ref = StaticKV(m.config, 3, 12, "cpu", torch.float32)
    m(input_ids=history, past_key_values=kv_ref, cache_position=torch.arange(5))
    kv = StaticKV(m.config, 3, 12, "cpu", torch.float32)
    for layer in range(m.config.num_hidden_layers):
        kv.keys[layer].copy_(kv_ref.keys[layer])
        kv.values[layer].copy_(kv_ref.values[layer])
    pos = torch.tensor([5])
    mask = (torch.arange(12) <= pos).view(1, 1, 1, -1).expand(3, 1, 1, 12)
    want_d = m(input_ids=nxt, attention_mask=mask, position_ids=pos.view(1, 1).expand(3, 1), past_key_values=kv_ref,
               cache_position=pos).logits[:, 0]
    got = m.forward_mixed(prompts, nxt, kv, pos)
    assert got.shape == (5, 97)
    torch.testing.assert_close(got[:2], want_p, atol=2e-5, rtol=2e-5)
    torch.testing.assert_close(got[2:], want_d, atol=2e-5, rtol=2e-5)
    for layer in range(m.config.num_hidden_layers):
        torch.testing.assert_close(kv.keys[layer], kv_ref.keys[layer], atol=1e-6, rtol=1e-6)
        torch.testing.assert_close(kv.values[layer], kv_ref.values[layer], atol=1e-6, rtol=1e-6)


@torch.inference_mode()
def test_rotary_over_a_fused_qkv_output_equals_q_and_k_apart():
    """When q and k are adjacent column views of one projection output (the
    fused q|k|v group's), rotary runs once over both; the result equals
    rotating q and k apart, and a reference rotate_half rotation."""
    from multi_lora_amd.decoder import Rotary

    m = model()
    c = m.config
    h, kvh, d = c.num_attention_heads, c.num_key_value_heads, c.head_dim
    rows = 7
    qkv = torch.randn(rows, (h + 2 * kvh) * d, generator=torch.Generator().manual_seed(3))
    q, k = qkv[:, : h * d], qkv[:, h * d: (h + kvh) * d]
    pos = torch.tensor([0, 1, 2, 5, 9, 40, 511])
    rot = Rotary.make(pos, m.inv_freq, torch.float32)
    attn = m.layers[0].self_attn
    qj, kj = attn._rotate_qk(q, k, rot)
    qa, ka = attn._rotate_qk(q.clone(), k.clone(), rot)  # separate tensors: rotated apart
    torch.testing.assert_close(qj, qa, atol=0, rtol=0)
    torch.testing.assert_close(kj, ka, atol=0, rtol=0)
    ang = pos.float()[:, None] * m.inv_freq                                 # [rows, d/2]
    cos, sin = torch.cat((ang.cos(), ang.cos()), -1)[:, None], torch.cat((ang.sin(), ang.sin()), -1)[:, None]

    def rotate_half(x):
        return torch.cat((-x[..., d // 2:], x[..., : d // 2]), -1)

    qr = q.reshape(rows, h, d)
    torch.testing.assert_close(qj, qr * cos + rotate_half(qr) * sin, atol=1e-6, rtol=1e-6)


def test_decode_step_like_new_and_layer_views():
    """DecodeStep.like_new (multi_lora/graph_decode.py:55-57) gives a second
    step of the same shape with its own empty cache, counter at start and
    prompt-only mask; kv.layers[i].keys / .values are the cache's buffers
    (the view multi_lora/tests/test_graph_decode.py:93-97 reads)."""
    from types import SimpleNamespace

    from multi_lora_amd.graph_decode import DecodeStep

    m = model()
    mgr = SimpleNamespace(model=m, pool=SimpleNamespace(device=torch.device("cpu"), dtype=torch.float32))
    step = DecodeStep.new(mgr, batch=2, start=3, max_len=8)
    step.kv_pos.add_(2)
    step.kv.keys[0].fill_(1.0)
    twin = step.like_new(mgr)
    assert (twin.batch, twin.start, twin.max_len) == (2, 3, 8)
    assert int(twin.kv_pos) == 3 and int(step.kv_pos) == 5
    assert twin.kv.keys[0].data_ptr() != step.kv.keys[0].data_ptr()
    assert not twin.kv.keys[0].any()
    assert twin.attn_mask[..., :3].all() and not twin.attn_mask[..., 3:].any()
    layers = step.kv.layers
    assert len(layers) == m.config.num_hidden_layers
    for i, layer in enumerate(layers):
        assert layer.keys.data_ptr() == step.kv.keys[i].data_ptr()
        assert layer.values.data_ptr() == step.kv.values[i].data_ptr()
