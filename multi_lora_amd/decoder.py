"""A minimal Llama-style decoder used as the caller of the LoRA path.

The reference drives its decode step through a Hugging Face model and
``transformers.StaticCache`` (multi_lora/graph_decode.py:23-111).  Weights
cannot be downloaded here, so this module provides the model around the
path: token embedding, ``n_layers`` blocks of [RMSNorm -> q/k/v projections
-> rotary attention over a static KV cache -> o projection -> residual ->
RMSNorm -> SiLU-gated MLP -> residual], final RMSNorm and LM head.  Every
projection is a plain ``nn.Linear`` named like Llama's
(``layers.{i}.self_attn.q_proj`` ... ``layers.{i}.mlp.down_proj``), so the
manager wraps them with ``LinearWithLoRA`` exactly as it wraps a Hugging Face
model, and ``fuse_rmsnorm`` routes the norms through the HIP RMSNorm.

Attention runs its two products in the model dtype (fp32 accumulation,
contiguous operands, the score scale applied inside the first) with the
softmax in fp32; the query heads that share a key head are stacked as rows,
so keys are never repeated.  Rotary runs once per layer over q and k
together when they are adjacent columns of one projection output (the fused
q|k|v group's).  A block's residual adds travel to the next RMSNorm, which
``fuse_rmsnorm`` turns into one fused add + RMSNorm kernel.  The KV cache is
written in place at ``cache_position`` and read whole under a boolean mask,
so a decode step touches fixed addresses and can be captured in a HIP graph.
``forward`` accepts the keyword arguments the reference passes to its model
(input_ids, attention_mask, position_ids, past_key_values, cache_position,
use_cache) and returns an object with ``.logits``.
"""

from __future__ import annotations

import math
from dataclasses import dataclass
from types import SimpleNamespace
from typing import List, Optional

import torch
import torch.nn as nn
import torch.nn.functional as F


@dataclass
class DecoderConfig:
    vocab_size: int = 512
    hidden_size: int = 256
    intermediate_size: int = 512
    num_hidden_layers: int = 2
    num_attention_heads: int = 4
    num_key_value_heads: int = 2
    rms_norm_eps: float = 1e-5
    rope_theta: float = 500000.0

    @property
    def head_dim(self) -> int:
        return self.hidden_size // self.num_attention_heads

    @classmethod
    def llama3_8b(cls) -> "DecoderConfig":
        return cls(vocab_size=128256, hidden_size=4096, intermediate_size=14336, num_hidden_layers=32,
                   num_attention_heads=32, num_key_value_heads=8, rms_norm_eps=1e-5, rope_theta=500000.0)


class StaticKV:
    """Per-layer key and value buffers, allocated once: keys
    ``[batch, kv_heads, head_dim, max_len]`` (stored transposed, so the score
    product reads them in place as its contiguous right operand) and values
    ``[batch, kv_heads, max_len, head_dim]``."""

    def __init__(self, config: DecoderConfig, batch: int, max_len: int, device, dtype) -> None:
        kshape = (batch, config.num_key_value_heads, config.head_dim, max_len)
        vshape = (batch, config.num_key_value_heads, max_len, config.head_dim)
        self.max_len = max_len
        self.keys: List[torch.Tensor] = [torch.zeros(kshape, device=device, dtype=dtype)
                                         for _ in range(config.num_hidden_layers)]
        self.values: List[torch.Tensor] = [torch.zeros(vshape, device=device, dtype=dtype)
                                           for _ in range(config.num_hidden_layers)]

    @property
    def layers(self) -> List["KVLayer"]:
        """Per-layer views ``layers[i].keys`` / ``layers[i].values`` of the same
        buffers, as a transformers ``StaticCache`` exposes its layers
        (multi_lora/tests/test_graph_decode.py:93-97 reads them)."""
        return [KVLayer(k, v) for k, v in zip(self.keys, self.values)]


@dataclass
class KVLayer:
    """One layer's key buffer (``[batch, kv_heads, head_dim, max_len]``) and
    value buffer (``[batch, kv_heads, max_len, head_dim]``) of a ``StaticKV``."""

    keys: torch.Tensor
    values: torch.Tensor


class DecoderRMSNorm(nn.Module):
    """``x * rsqrt(mean(x^2) + eps) * w`` (fp32 math, one rounding); replaced by the HIP kernel via fuse_rmsnorm."""

    def __init__(self, hidden: int, eps: float) -> None:
        super().__init__()
        self.weight = nn.Parameter(torch.ones(hidden))
        self.variance_epsilon = eps

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        h = x.float()
        h = h * torch.rsqrt(h.pow(2).mean(-1, keepdim=True) + self.variance_epsilon) * self.weight.float()
        return h.to(x.dtype)

    def add_forward(self, delta: torch.Tensor, residual: torch.Tensor) -> torch.Tensor:
        """``residual += delta`` (in place, rounded to the dtype), then the
        norm of it; ``fuse_rmsnorm`` rebinds this to the fused HIP kernel."""
        residual.add_(delta)
        return self(residual)


@dataclass
class Rotary:
    """Rotary tables for ``R`` rows in the model dtype, shaped ``[R, 1, head_dim]``
    to broadcast over rows viewed as ``[R, heads, head_dim]``: ``cos`` and the
    signed ``sin`` (``-sin`` on the first half), so that
    ``rotate(x) = x * cos + roll(x, d/2) * sin``."""

    cos: torch.Tensor
    sin: torch.Tensor

    @staticmethod
    def make(positions: torch.Tensor, inv_freq: torch.Tensor, dtype) -> "Rotary":
        ang = positions.reshape(-1).float()[:, None] * inv_freq          # [R, d/2]
        c, s = ang.cos(), ang.sin()
        cos = torch.cat((c, c), dim=-1)[:, None]                          # [R, 1, d]
        sin = torch.cat((-s, s), dim=-1)[:, None]
        return Rotary(cos.to(dtype), sin.to(dtype))


def _rotate(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor) -> torch.Tensor:
    """``x * cos + rotate_half(x) * sin`` with the sign of rotate_half folded
    into ``sin``: three element-wise kernels in the model dtype."""
    return torch.addcmul(x * cos, x.roll(x.shape[-1] // 2, dims=-1), sin)


class Attention(nn.Module):
    def __init__(self, c: DecoderConfig) -> None:
        super().__init__()
        self.c = c
        d = c.head_dim
        self.scale = 1.0 / math.sqrt(d)
        self.q_proj = nn.Linear(c.hidden_size, c.num_attention_heads * d, bias=False)
        self.k_proj = nn.Linear(c.hidden_size, c.num_key_value_heads * d, bias=False)
        self.v_proj = nn.Linear(c.hidden_size, c.num_key_value_heads * d, bias=False)
        self.o_proj = nn.Linear(c.num_attention_heads * d, c.hidden_size, bias=False)

    def forward(self, x, rot: Rotary, hide, kv: Optional[StaticKV], layer: int, cache_position):
        b, t, _ = x.shape
        q, k = self._rotate_qk(self.q_proj(x).reshape(b * t, -1), self.k_proj(x).reshape(b * t, -1), rot)
        out = self._attend(q, k, self.v_proj(x), b, t, hide, kv, layer, cache_position)
        return self.o_proj(out.to(x.dtype))

    def _rotate_qk(self, q: torch.Tensor, k: torch.Tensor, rot: Rotary):
        """Rotary on rows ``q [R, h*d]`` and ``k [R, kvh*d]``; returns them as
        ``[R, h, d]`` and ``[R, kvh, d]``.  When k's columns directly follow
        q's in one tensor (the fused q|k|v output), both go through one set
        of three kernels over the ``[R, h + kvh, d]`` view."""
        c = self.c
        h, kvh, d = c.num_attention_heads, c.num_key_value_heads, c.head_dim
        rows = q.shape[0]
        if (q.stride(-1) == 1 and k.stride(-1) == 1 and q.stride(0) == k.stride(0) and q.dtype == k.dtype
                and q.untyped_storage().data_ptr() == k.untyped_storage().data_ptr()
                and k.data_ptr() == q.data_ptr() + h * d * q.element_size()):
            qk = torch.as_strided(q, (rows, h + kvh, d), (q.stride(0), d, 1))
            r = _rotate(qk, rot.cos, rot.sin)
            return r[:, :h], r[:, h:]
        return (_rotate(q.reshape(rows, h, d), rot.cos, rot.sin), _rotate(k.reshape(rows, kvh, d), rot.cos, rot.sin))

    def _attend(self, q, k, v, b, t, hide, kv: Optional[StaticKV], layer: int, cache_position):
        """Attention of ``b`` sequences of ``t`` rows, given rotated ``q
        [b*t, h, d]`` and ``k [b*t, kvh, d]`` and ``v`` row-major; writes this
        step's keys and values into ``kv`` at ``cache_position`` and attends
        over the whole cache, except the key positions ``hide`` marks
        (boolean ``[b, 1, t, L]``, True = not attended).  Returns ``[b, t, heads*d]`` in
        the model dtype."""
        c = self.c
        h, kvh, d = c.num_attention_heads, c.num_key_value_heads, c.head_dim
        rep = h // kvh
        dt = q.dtype
        q = q.reshape(b, t, h, d).transpose(1, 2).contiguous()              # [b, h, t, d]
        k = k.reshape(b, t, kvh, d)
        v = v.reshape(b, t, kvh, d).transpose(1, 2)                           # [b, kvh, t, d]
        if kv is not None:
            kv.keys[layer].index_copy_(3, cache_position, k.permute(0, 2, 3, 1).to(kv.keys[layer].dtype))
            kv.values[layer].index_copy_(2, cache_position, v.to(kv.values[layer].dtype))
            keys_t, v = kv.keys[layer].to(dt), kv.values[layer]                  # keys_t [b, kvh, d, L]
        else:
            keys_t = k.permute(0, 2, 3, 1).contiguous()
        length = keys_t.shape[-1]
        # The query heads sharing a key head are stacked as rows, so keys and
        # values are read once per key head, never repeated.  The score scale
        # is the product's alpha (beta 0: its input is not read).  Scores stay
        # in the model dtype, masked in place; softmax computes a 16-bit
        # input in fp32 and rounds its output once.
        qg = q.view(b * kvh, rep * t, d)
        unused = torch.empty((1, 1, 1), dtype=dt, device=q.device).expand(b * kvh, rep * t, length)
        scores = torch.baddbmm(unused, qg, keys_t.reshape(b * kvh, d, length), beta=0.0, alpha=self.scale)
        scores.view(b, kvh, rep, t, length).masked_fill_(hide[:, :, None], float("-inf"))
        probs = torch.softmax(scores, dim=-1)
        out = torch.bmm(probs, v.to(dt).contiguous().view(b * kvh, length, d))    # [b*kvh, rep*t, d]
        return out.view(b, h, t, d).transpose(1, 2).reshape(b, t, h * d)

    def forward_mixed(self, x, rot: Rotary, pre: "Packed", dec: "Packed", layer: int):
        """Packed rows ``x [R, hidden]``: ``pre.n`` prompts of ``pre.t`` tokens,
        then ``dec.n`` decode rows, with ``rot`` covering all R rows.  The
        projections (and their LoRA deltas) and rotary run once over all
        rows; attention runs per part, prompts causally over themselves,
        decode rows over their own KV caches."""
        q, k = self._rotate_qk(self.q_proj(x), self.k_proj(x), rot)
        v = self.v_proj(x)
        outs = []
        for part in (pre, dec):
            if part.n == 0:
                continue
            rows = slice(part.row0, part.row0 + part.n * part.t)
            o = self._attend(q[rows], k[rows], v[rows], part.n, part.t, part.hide, part.kv, layer,
                             part.cache_position)
            outs.append(o.reshape(part.n * part.t, -1))
        return self.o_proj(torch.cat(outs).to(x.dtype))


class MLP(nn.Module):
    def __init__(self, c: DecoderConfig) -> None:
        super().__init__()
        self.gate_proj = nn.Linear(c.hidden_size, c.intermediate_size, bias=False)
        self.up_proj = nn.Linear(c.hidden_size, c.intermediate_size, bias=False)
        self.down_proj = nn.Linear(c.intermediate_size, c.hidden_size, bias=False)

    def forward(self, x):
        return self.down_proj(F.silu(self.gate_proj(x)) * self.up_proj(x))


class Block(nn.Module):
    def __init__(self, c: DecoderConfig) -> None:
        super().__init__()
        self.input_layernorm = DecoderRMSNorm(c.hidden_size, c.rms_norm_eps)
        self.self_attn = Attention(c)
        self.post_attention_layernorm = DecoderRMSNorm(c.hidden_size, c.rms_norm_eps)
        self.mlp = MLP(c)

    def forward(self, x, rot: Rotary, hide, kv, layer, cache_position, pending=None):
        """Returns ``(x, delta)``: the residual stream after the attention half
        and the MLP output still to be added to it.  ``pending``, the previous
        block's such delta, is added in by this block's first RMSNorm (``x``
        is updated in place)."""
        h = self.input_layernorm(x) if pending is None else self.input_layernorm.add_forward(pending, x)
        attn = self.self_attn(h, rot, hide, kv, layer, cache_position)
        return x, self.mlp(self.post_attention_layernorm.add_forward(attn, x))

    def forward_mixed(self, x, rot, pre, dec, layer, pending=None):
        h = self.input_layernorm(x) if pending is None else self.input_layernorm.add_forward(pending, x)
        attn = self.self_attn.forward_mixed(h, rot, pre, dec, layer)
        return x, self.mlp(self.post_attention_layernorm.add_forward(attn, x))


@dataclass
class Packed:
    """One part of a packed mixed batch: ``n`` sequences of ``t`` rows from row ``row0``."""

    n: int
    t: int
    row0: int
    hide: torch.Tensor  # True: key position not attended
    kv: Optional[StaticKV]
    cache_position: Optional[torch.Tensor]


class Decoder(nn.Module):
    def __init__(self, config: DecoderConfig) -> None:
        super().__init__()
        self.config = config
        self.embed_tokens = nn.Embedding(config.vocab_size, config.hidden_size)
        self.layers = nn.ModuleList(Block(config) for _ in range(config.num_hidden_layers))
        self.norm = DecoderRMSNorm(config.hidden_size, config.rms_norm_eps)
        self.lm_head = nn.Linear(config.hidden_size, config.vocab_size, bias=False)
        d = config.head_dim
        inv = 1.0 / (config.rope_theta ** (torch.arange(0, d, 2, dtype=torch.float32) / d))
        self.register_buffer("inv_freq", inv, persistent=False)

    def forward(self, input_ids: torch.Tensor, attention_mask: Optional[torch.Tensor] = None,
                position_ids: Optional[torch.Tensor] = None, past_key_values: Optional[StaticKV] = None,
                cache_position: Optional[torch.Tensor] = None, use_cache: bool = True, **_):
        b, t = input_ids.shape
        dev = input_ids.device
        kv = past_key_values if use_cache else None
        if cache_position is None:
            cache_position = torch.arange(t, device=dev)
        if position_ids is None:
            position_ids = cache_position.view(1, t).expand(b, t)
        x = self.embed_tokens(input_ids)
        rot = Rotary.make(position_ids.expand(b, t), self.inv_freq, x.dtype)
        length = kv.max_len if kv is not None else t
        hide = ~self._mask(attention_mask, b, t, length, cache_position, dev)  # once for every layer
        pending = None
        for i, layer in enumerate(self.layers):
            x, pending = layer(x, rot, hide, kv, i, cache_position, pending)
        return SimpleNamespace(logits=self.lm_head(self.norm.add_forward(pending, x)))

    def forward_mixed(self, prompt_ids: torch.Tensor, decode_ids: torch.Tensor, decode_kv: StaticKV,
                      decode_pos: torch.Tensor):
        """One serving step over a mixed batch, rows packed as the segment table
        lists them: every prompt's tokens (``prompt_ids [p, t]``, positions
        0..t-1, causal within the prompt), then one row per decode sequence
        (``decode_ids [d, 1]``) at position ``decode_pos`` (a 1-element device
        tensor), attending over its KV cache ``decode_kv`` (written there).
        Returns logits ``[p + d, vocab]`` for each prompt's last token and each
        decode row.  Every shape is fixed by the arguments' shapes, so the
        step can be captured in a graph and replayed with new ids and a new
        ``decode_pos``."""
        dev = prompt_ids.device
        p, t = prompt_ids.shape
        d = decode_ids.shape[0]
        x = torch.cat((self.embed_tokens(prompt_ids).reshape(p * t, -1),
                       self.embed_tokens(decode_ids).reshape(d, -1)))
        pos = torch.arange(t, device=dev)
        later = (pos[None, :] > pos[:, None]).view(1, 1, t, t)
        pre = Packed(p, t, 0, later, None, None)
        unseen = (torch.arange(decode_kv.max_len, device=dev) > decode_pos).view(1, 1, 1, -1)
        dec = Packed(d, 1, p * t, unseen, decode_kv, decode_pos)
        rot = Rotary.make(torch.cat((pos.repeat(p), decode_pos.reshape(1).expand(d))), self.inv_freq, x.dtype)
        pending = None
        for i, layer in enumerate(self.layers):
            x, pending = layer.forward_mixed(x, rot, pre, dec, i, pending)
        last = torch.cat((torch.arange(t - 1, p * t, t, device=dev), torch.arange(p * t, p * t + d, device=dev)))
        return self.lm_head(self.norm(x[last] + pending[last]))

    @staticmethod
    def _mask(attention_mask, b, t, length, cache_position, dev) -> torch.Tensor:
        """Boolean [b, 1, t, length]: a 4-D mask is used as given; a 2-D
        padding mask over the first positions is combined with causality."""
        if attention_mask is not None and attention_mask.dim() == 4:
            return attention_mask.bool()
        keys = torch.arange(length, device=dev)
        causal = keys[None, :] <= cache_position[:, None]                # [t, length]
        mask = causal[None, None].expand(b, 1, t, length)
        if attention_mask is not None:
            pad = torch.zeros(b, length, dtype=torch.bool, device=dev)
            pad[:, : attention_mask.shape[1]] = attention_mask.bool()
            mask = mask & pad[:, None, None, :]
        return mask
