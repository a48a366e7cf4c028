"""Packed segment metadata on the GPU (one pinned copy per rewrite).

The five device columns must equal, bit for bit, what the column-by-column
path writes on the CPU (itself pinned to the reference's padding rules in
test_oracle_known_answers.py), keep their addresses while the capacity holds
the batch, and drive a captured graph correctly after each rewrite.  The
table's plan, built on the host and packed with the columns, must equal the
plan the device builder makes of the same table.
"""

import random

import pytest
import torch

from multi_lora_amd import HipLoRABackend, synthetic
from multi_lora_amd.batch_info import (BatchLoRAInfo, empty_kernel_input_metadata,
                                       write_kernel_input_metadata)
from multi_lora_amd.kernels.lora_ops import build_plan_device

pytestmark = pytest.mark.gpu

COLS = ("seg_lens", "seg_indptr", "weight_indices", "lora_ranks", "scalings")


def random_batch(rng, rows, k):
    return BatchLoRAInfo(weight_indices=[rng.randrange(k) for _ in range(rows)],
                         lora_ranks=[rng.choice([0, 8, 16]) for _ in range(k)],
                         scalings=[rng.choice([0.0, 0.5, 2.0]) for _ in range(k)])


def pb_rows(meta):
    return meta.bs


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_packed_columns_match_cpu_path_and_keep_addresses(dev, dtype):
    rng = random.Random(3)
    k = 16
    gmeta = empty_kernel_input_metadata(device=dev, dtype=dtype)
    cmeta = empty_kernel_input_metadata(device=torch.device("cpu"), dtype=dtype)
    sizes = [40, 12, 40, 1, 33, 64, 7, 64, 20]
    addr = None
    for rows in sizes:
        pb = random_batch(rng, rows, k)
        seq = [] if rng.random() < 0.5 else [rng.randint(0, 9) for _ in range(rows)]
        before = gmeta
        gmeta = write_kernel_input_metadata(gmeta, pb, device=dev, dtype=dtype, seq_lens=seq)
        cmeta = write_kernel_input_metadata(cmeta, pb, device=torch.device("cpu"), dtype=dtype, seq_lens=seq)
        torch.cuda.synchronize()
        assert gmeta.packed is not None
        if before.packed is not None and rows <= before.packed.capacity:
            assert gmeta is before and gmeta.weight_indices.data_ptr() == addr
        addr = gmeta.weight_indices.data_ptr()
        assert (gmeta.bs, gmeta.max_len) == (cmeta.bs, cmeta.max_len)
        for c in COLS:
            g, h = getattr(gmeta, c).cpu(), getattr(cmeta, c)
            n = min(g.shape[0], h.shape[0])
            assert torch.equal(g[:n], h[:n]), c
            if c in ("lora_ranks", "scalings"):
                assert g.shape == h.shape
        # The plan packed with the table equals the device builder's plan of the same table.
        assert gmeta.plan is not None and gmeta.plan_entries >= 0
        total = int(cmeta.seg_indptr[pb_rows(cmeta)].item())
        used = 16 + 32 * min(gmeta.plan_entries, gmeta.plan_cap)
        built = build_plan_device(gmeta, total, k, gmeta.plan_cap).cpu()
        assert torch.equal(gmeta.plan.cpu()[:used], built[:used])


def test_graph_replay_follows_packed_rewrites(dev):
    """A captured apply_lora reads the packed columns; rewriting them for a
    new batch of the same size changes the replay's result to the new
    batch's eager result."""
    wl = synthetic.decode_q(device=dev, tokens=64, in_dim=1024, out=1024, n_slots=16, n_adapters=8, rank=16, seed=4)
    a, b = wl.a_stacks[0], wl.b_stacks[0]
    ranks, scal = wl.slot_ranks, wl.scalings
    meta = empty_kernel_input_metadata(device=dev, dtype=torch.bfloat16)
    meta = write_kernel_input_metadata(meta, BatchLoRAInfo(wl.seg_slots, ranks, scal), device=dev,
                                       dtype=torch.bfloat16, seq_lens=[])
    be = HipLoRABackend()
    be.set_kernel_input_metadata(meta)
    out = wl.clone_base()
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        be.apply_lora(wl.x, a, b, out)     # warm up the capture stream's workspace
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=stream):
        be.apply_lora(wl.x, a, b, out)
    rng = random.Random(9)
    for _ in range(4):
        slots = [rng.randrange(8) for _ in range(64)]
        same = write_kernel_input_metadata(meta, BatchLoRAInfo(slots, ranks, scal), device=dev,
                                           dtype=torch.bfloat16, seq_lens=[])
        assert same is meta
        eager = wl.clone_base()
        be.apply_lora(wl.x, a, b, eager)
        out.copy_(wl.base)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager)
