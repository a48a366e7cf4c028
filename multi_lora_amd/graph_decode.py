"""Batched single-token decoding as one replayable HIP graph.

API of multi_lora/graph_decode.py:23-111 (``DecodeStep.new``, ``prefill``,
``run``, ``rewind``, ``capture_graph`` and the resident tensors the
reference's tests inspect), built on this package's decoder:

    step = DecodeStep.new(mgr, batch, start, max_len)
    first = step.prefill(mgr, input_ids, attention_mask, names)
    step.input_ids.copy_(first)
    mgr._setup_forward_batch(names, seq_lens=[1] * batch)
    graph, out = capture_graph(mgr, step)        # then graph.replay() per step

Design.  The whole decode state is device memory that a step updates in
place, so a captured step is its own successor:

* one int64 counter, ``kv_pos``, is both the KV slot written this step and
  every row's rotary position (``position_ids`` is a broadcast view of it);
* the attention mask is kept, not recomputed: the prompt's slots are
  visible from the start and each step makes its own slot visible with one
  indexed write before the forward;
* the KV cache (``decoder.StaticKV``) is written at ``kv_pos`` by the
  attention layers.

Slots past ``kv_pos`` may hold stale keys (from the warm-up or from an
earlier pass before a rewind); they stay masked until the step that owns
them overwrites them.  LoRA launches inside the step read the resident
segment table, which the manager rewrites in place between batches.
"""

from __future__ import annotations

import torch

from .decoder import StaticKV

WARMUP_STEPS = 3


class DecodeStep:
    """Resident state of ``batch`` sequences decoding one token per step from position ``start``."""

    def __init__(self, mgr, batch: int, start: int, max_len: int) -> None:
        if not 0 < start < max_len:
            raise ValueError(f"need 0 < start < max_len (start={start}, max_len={max_len})")
        device, dtype = mgr.pool.device, mgr.pool.dtype
        self.batch, self.start, self.max_len = batch, start, max_len
        self.kv = StaticKV(mgr.model.config, batch, max_len, device, dtype)
        self.input_ids = torch.zeros((batch, 1), dtype=torch.long, device=device)
        self.kv_pos = torch.full((1,), start, dtype=torch.long, device=device)
        self.position_ids = self.kv_pos.view(1, 1).expand(batch, 1)
        self.attn_mask = torch.zeros((batch, 1, 1, max_len), dtype=torch.bool, device=device)
        self.attn_mask[..., :start] = True

    @classmethod
    def new(cls, mgr, batch: int, start: int, max_len: int) -> "DecodeStep":
        return cls(mgr, batch, start, max_len)

    def like_new(self, mgr) -> "DecodeStep":
        """A second step of the same shape (batch, start, max_len), with its own
        empty KV cache and its counter at ``start`` (multi_lora/graph_decode.py:55-57)."""
        return DecodeStep.new(mgr, self.batch, self.start, self.max_len)

    def rewind(self) -> None:
        """Return to position ``start``: the counter and the mask, nothing else."""
        self.kv_pos.fill_(self.start)
        self.attn_mask[..., self.start:] = False

    def prefill(self, mgr, input_ids: torch.Tensor, attention_mask: torch.Tensor, lora_names) -> torch.Tensor:
        """Run the prompt (``start`` tokens per row) through the model with each
        row's adapter, filling KV slots ``[0, start)``; returns the greedy next
        token of every row, shape ``(batch, 1)``."""
        t = int(input_ids.shape[1])
        if t != self.start:
            raise ValueError(f"prompt length {t} differs from the step's start position {self.start}")
        out = mgr.forward_with_lora(
            input_ids=input_ids, attention_mask=attention_mask, lora_names=lora_names,
            seq_lens=[t] * self.batch, past_key_values=self.kv, use_cache=True,
            cache_position=torch.arange(t, device=input_ids.device))
        return out.logits[:, -1].argmax(dim=-1, keepdim=True)

    def run(self, mgr):
        """One step: expose this step's KV slot, forward ``input_ids``, advance the counter."""
        self.attn_mask.index_fill_(-1, self.kv_pos, True)
        out = mgr.model(input_ids=self.input_ids, attention_mask=self.attn_mask, position_ids=self.position_ids,
                        past_key_values=self.kv, cache_position=self.kv_pos, use_cache=True)
        self.kv_pos.add_(1)
        return out


def capture_graph(mgr, step: DecodeStep, warmup: int = WARMUP_STEPS):
    """Capture one ``step.run`` into a HIP graph; returns ``(graph, output)``.

    Warm-up steps run first on the stream the capture will use, on the
    step's own buffers, so every lazily created resource (the decode
    path's per-stream workspace, library handles, allocator blocks) exists
    before capture and nothing is allocated or cleared inside the graph.
    The warm-up advances the state and is rewound; the capture only
    records, so the step is at ``start`` when this returns and the first
    replay decodes position ``start``.  ``output`` is the captured run's
    result, whose tensors every replay overwrites.
    """
    if step.start + warmup + 1 > step.max_len:
        raise ValueError(f"max_len {step.max_len} leaves no room for {warmup} warm-up steps and the capture")
    side = torch.cuda.Stream(device=step.kv_pos.device)
    side.wait_stream(torch.cuda.current_stream(step.kv_pos.device))
    with torch.cuda.stream(side):
        for _ in range(warmup):
            step.run(mgr)
        step.rewind()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=side):
        out = step.run(mgr)
    torch.cuda.current_stream(step.kv_pos.device).wait_stream(side)
    return graph, out
