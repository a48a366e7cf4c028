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
