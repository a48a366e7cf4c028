"""Everything one decode step touches, at fixed addresses, and its graph capture.

Mirrors multi_lora/graph_decode.py:23-111 on the model of
``multi_lora_amd.decoder`` (whose ``StaticKV`` plays the part of
``transformers.StaticCache``):

    step = DecodeStep.new(mgr, batch, start, max_len)
    first = step.prefill(mgr, input_ids, attention_mask, names)
    step.input_ids.copy_(first)
    mgr._setup_forward_batch(names, seq_lens=[1] * batch)
    graph, out = capture_graph(mgr, step)        # then graph.replay() per step

A decode step reads and writes only resident tensors: the KV cache is
written in place at ``kv_pos``, the attention mask is recomputed in place
from ``grid <= kv_pos``, and ``position_ids`` / ``kv_pos`` are advanced in
place, so the captured graph advances by itself on every replay.  The LoRA
launches inside read the resident segment table, which the manager rewrites
in place between batches.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch

from .decoder import StaticKV

WARMUP_ROUNDS = 3  # steps run before capture, on a second set of buffers


@dataclass
class DecodeStep:
    kv: StaticKV
    input_ids: torch.Tensor     # (batch, 1) token fed this step
    position_ids: torch.Tensor  # (batch, 1) rotary position
    kv_pos: torch.Tensor        # (1,) KV slot written this step
    attn_mask: torch.Tensor     # (batch, 1, 1, max_len) visible slots
    grid: torch.Tensor          # (max_len,) 0..max_len-1, for the mask
    batch: int
    start: int                  # first position after the prompt; rewind target
    max_len: int

    @classmethod
    def new(cls, mgr, batch: int, start: int, max_len: int) -> "DecodeStep":
        device = mgr.pool.device
        return cls(
            kv=StaticKV(mgr.model.config, batch, max_len, device, mgr.pool.dtype),
            input_ids=torch.zeros((batch, 1), device=device, dtype=torch.long),
            position_ids=torch.full((batch, 1), start, device=device, dtype=torch.long),
            kv_pos=torch.tensor([start], device=device, dtype=torch.long),
            attn_mask=torch.zeros((batch, 1, 1, max_len), device=device, dtype=torch.bool),
            grid=torch.arange(max_len, device=device, dtype=torch.long),
            batch=batch,
            start=start,
            max_len=max_len,
        )

    def like_new(self, mgr) -> "DecodeStep":
        return DecodeStep.new(mgr, self.batch, self.start, self.max_len)

    def rewind(self) -> None:
        """Back to ``start``; KV slots past it are simply overwritten later."""
        self.position_ids.fill_(self.start)
        self.kv_pos.fill_(self.start)

    def prefill(self, mgr, input_ids: torch.Tensor, attention_mask: torch.Tensor, lora_names) -> torch.Tensor:
        """Fill the first ``start`` KV slots; returns the next token (batch, 1)."""
        t = int(input_ids.shape[1])
        out = mgr.forward_with_lora(
            input_ids=input_ids, attention_mask=attention_mask, lora_names=lora_names,
            seq_lens=[t] * self.batch, past_key_values=self.kv, use_cache=True,
            cache_position=torch.arange(t, device=input_ids.device))
        return out.logits[:, -1].argmax(dim=-1, keepdim=True)

    def run(self, mgr):
        """One decode step: refresh the mask, forward (writing KV), advance the position."""
        self.attn_mask.copy_((self.grid <= self.kv_pos).view(1, 1, 1, -1))
        out = mgr.model(input_ids=self.input_ids, attention_mask=self.attn_mask, position_ids=self.position_ids,
                        past_key_values=self.kv, cache_position=self.kv_pos, use_cache=True)
        self.position_ids.add_(1)
        self.kv_pos.add_(1)
        return out


def capture_graph(mgr, step: DecodeStep):
    """Warm up on a second set of buffers, capture one step, rewind; returns (graph, output).

    One-time work (library workspaces, allocator growth) cannot be recorded,
    so it is done first in the warm-up, on a side stream.  The captured run
    really executes once, hence the rewind before returning.
    """
    warm = step.like_new(mgr)
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        for _ in range(WARMUP_ROUNDS):
            warm.run(mgr)
    torch.cuda.current_stream().wait_stream(stream)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = step.run(mgr)
    step.rewind()
    return graph, out
