#!/usr/bin/env python3
"""Segment-LoRA shrink+expand benchmark on one MI355X.

Workload (the headline configuration): Llama-3-8B q_proj 4096->4096, bf16,
128 decode tokens, each its own segment; a 64-slot pool holding 32 rank-16
adapters; slot per token uniform; x~N(0,1), A~N(0,1/4096), B~N(0,0.02),
scaling 2.0, seed 1.  One step = one shrink+expand pass
(``HipLoRABackend.apply_lora``) over the 128 tokens, inputs resident in HBM.

Cold-cache protocol: the step rotates through ``--replicas`` independent
copies of x / A pool / B pool / output.  A step touches 10.5 MiB of them
(x 1 MiB, the 32 used adapters' A and B rows 4 MiB each, the output 1 MiB
read and written), so the default 64 replicas touch 672 MiB a rotation,
over twice the 256 MiB MALL.  Every timed region of exactly ``--steps``
steps starts at the replica after the previous region's last (one captured
graph per start offset), so no region finds its replicas in the caches.

Output: one JSON line.  ``value`` is the step's algorithmic HBM bytes divided
by its time (GB/s); ``ms_per_step`` gives the latency.  ``roofline`` covers
the dominant kernel, timed with HIP events on the launch stream; the
``cpu_baseline`` is the oracle's per-segment PyTorch path on the host cores
over a bounded sample of the same workload.
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

METRIC = "seg-LoRA shrink+expand µs & HBM GB/s, 8B shapes, 128 mixed-adapter decode"
HEADLINE_WORKLOAD = "decode q_proj 4096->4096, 128 one-token segments, 64-slot pool, 32 rank-16 adapters"
HBM_PEAK_GBS = 8000.0


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=256)
    ap.add_argument("--warmup", type=int, default=50)
    ap.add_argument("--replicas", type=int, default=64)
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-other-configs", action="store_true",
                    help="headline only: skip the prefill (c3), RMSNorm + q|k|v (c4) and mixed-batch (c5) calls "
                         "that the default line carries under other_configs")
    ap.add_argument("--kernel-steps", type=int, default=2000, help="launches in each per-kernel timing")
    ap.add_argument("--workload", choices=("decode_q",) + tuple(OTHER_WORKLOADS), default="decode_q",
                    help="decode_q is the headline; the others print a line of the same form for their shape")
    ap.add_argument("--profile-traffic", action="store_true",
                    help="run only the LoRA path of --workload (a decode or prefill workload) and a copy kernel "
                         "of known size, for rocprofv3 --pmc runs")
    ap.add_argument("--summarize-pmc", nargs="+", metavar="DIR",
                    help="FETCH_SIZE and WRITE_SIZE run directories of --profile-traffic (and optionally an MFMA "
                         "counter run's) -> the workload's counter summary under profiles/")
    ap.add_argument("--sweep", choices=("decode",),
                    help="decode: one JSON line per decode shape (tokens, adapters, rank, slices), graph-timed "
                         "over cold replicas, with the schedule the library picks")
    ap.add_argument("--calibrate", action="store_true",
                    help="launch floors (empty kernel, one-launch cold stream of the headline's bytes) and the "
                         "planned decode kernel's per-phase timeline, from the measurement library")
    ap.add_argument("--regions", type=int, default=0,
                    help="timed regions of exactly --steps steps each (default: enough for ~2000 steps, 5..101); "
                         "the step time is their median")
    return ap.parse_args()


OTHER_WORKLOADS = {
    "prefill_gate_up": "prefill MLP gate|up 4096->2x14336, 8 segments of U[64,1024] tokens, ranks {16,32,64}, r_max 64",
    "prefill_down": "prefill MLP down 14336->4096, 8 segments of U[64,1024] tokens, ranks {16,32,64}, r_max 64",
    "decode_qkv": "RMSNorm then q|k|v 4096->[4096,1024,1024], 256 one-token segments, 256-slot pool, "
                  "128 rank-32 adapters",
    "decode_qkv_fused": "RMSNorm folded into the q|k|v LoRA call (mlora_rmsnorm_apply_grouped, two launches): "
                        "4096->[4096,1024,1024], 256 one-token segments, 256-slot pool, 128 rank-32 adapters",
    "decode_q_resident": "decode q_proj 4096->4096, 128 one-token segments, 64-slot pool holding 64 resident "
                         "rank-16 adapters, tokens drawn over 32 of them",
    "decode_q_device_plan": "decode q_proj 4096->4096, 128 one-token segments, 64-slot pool, 32 rank-16 adapters; "
                            "the segment table carries no plan (device tensors only, as a hand-built "
                            "KernelInputMetaData), so the library builds the plan on the device for every call",
    "c5_gate_up": "the 32-layer step's gate|up LoRA call: 4096->2x14336, mixed batch of 2 x 512 prefill + 64 decode "
                  "rows (66 segments), 128-slot pool holding 35 rank-16 adapters",
    "c5_qkv": "the 32-layer step's q|k|v LoRA call: 4096->[4096,1024,1024], mixed batch of 2 x 512 prefill + 64 "
              "decode rows (66 segments), 128-slot pool holding 35 rank-16 adapters",
    "c5_o": "the 32-layer step's o LoRA call: 4096->4096, mixed batch of 2 x 512 prefill + 64 decode rows "
            "(66 segments), 128-slot pool holding 35 rank-16 adapters",
    "c5_down": "the 32-layer step's down LoRA call: 14336->4096, mixed batch of 2 x 512 prefill + 64 decode rows "
               "(66 segments), 128-slot pool holding 35 rank-16 adapters",
    "pool_upload": "pool upload scatter, Llama-3-8B 32 layers x 7 projections (224 keys), rank 16, "
                   "4 staged adapters (84 MB each) into an 8-slot pool",
    "c5_step": "Llama-3-8B-shaped 32-layer model step (random init): 7 projections per layer LoRA-ed at rank 16, "
               "mixed batch of 2 x 512 prefill + 64 decode tokens, 128-slot pool (10.7 GB), adapters Zipf(1.1) over 512",
}


def bench_c5_step(args) -> int:
    """Per-step latency of a 32-layer Llama-3-8B-shaped model serving a mixed
    batch, with the slot pool in the loop.

    The model is ``decoder.Decoder(DecoderConfig.llama3_8b())``, random-init
    on the GPU, bf16, all 7 projections of every layer wrapped by the
    manager (``LinearWithLoRA``, HIP backend) and its RMSNorms on the HIP
    kernel.  A step is one packed forward (``Decoder.forward_mixed``) of 2
    prompts of 512 tokens and 64 decode rows (position 512 over their own
    KV caches): base GEMMs, attention, norms, every LoRA delta, LM head on
    the 66 next-token rows.  Every step draws 66 requests from Zipf(1.1)
    over 512 adapters, makes them resident in the 128-slot pool (LRU
    eviction; misses are uploaded from pinned host banks by the copy stream
    and the scatter kernel), rewrites the resident segment table (66
    segments, one per request, in row order) and replays the captured
    forward.  Host banks: the 512 adapter names share 16 distinct weight
    sets, so host memory stays at 1.3 GB while every miss still moves its
    84 MB over PCIe.
    """
    import statistics

    import torch

    from multi_lora_amd import (AdapterWeights, MultiLoRAManager, fuse_gate_up_projections, fuse_qkv_projections,
                                set_lora_enabled, write_kernel_input_metadata)
    from multi_lora_amd.decoder import Decoder, DecoderConfig, StaticKV

    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    cfg = DecoderConfig.llama3_8b()
    L, R, K, N_AD, SETS = cfg.num_hidden_layers, 16, 128, 512, 16
    torch.manual_seed(4)
    with torch.device(dev):
        model = Decoder(cfg)
    model = model.to(torch.bfloat16).eval()
    names7 = ("self_attn.q_proj", "self_attn.k_proj", "self_attn.v_proj", "self_attn.o_proj", "mlp.gate_proj",
              "mlp.up_proj", "mlp.down_proj")
    dims = {f"layers.{l}.{n}": (model.get_submodule(f"layers.{l}.{n}").in_features,
                                model.get_submodule(f"layers.{l}.{n}").out_features) for l in range(L) for n in names7}
    g = torch.Generator().manual_seed(4)
    shared = [AdapterWeights(rank=R, scaling=2.0, modules={
        k: ((torch.randn(R, i, generator=g) * i ** -0.5).bfloat16(), (torch.randn(o, R, generator=g) * 0.02).bfloat16())
        for k, (i, o) in dims.items()}) for _ in range(SETS)]
    store = {f"a{i}": shared[i % SETS] for i in range(N_AD)}
    mgr = MultiLoRAManager.from_adapters(model, store, max_loras_per_batch=K, max_lora_rank=R)
    # q|k|v and gate|up as one base GEMM and one multi-slice LoRA call each,
    # for every input shape (the mixed batch included).
    assert fuse_qkv_projections(mgr.lora_wrappers, all_shapes=True) == L
    assert fuse_gate_up_projections(mgr.lora_wrappers) == L
    pool, be = mgr.pool, mgr._lora_backend
    zipf = torch.tensor([(i + 1) ** -1.1 for i in range(N_AD)])
    lens = [512, 512] + [1] * 64
    rows = sum(lens)

    def draw():
        return [f"a{i}" for i in torch.multinomial(zipf, len(lens), replacement=True, generator=g).tolist()]

    def setup(names):
        """The manager's per-step setup, one segment per request (no merging of
        neighbours, so the captured launch shapes hold for every step)."""
        pool.prepare_lora_batch(list(dict.fromkeys(names)), weight_store=mgr._weight_store)
        return write_kernel_input_metadata(mgr._resident_meta, pool.build_batch_info(names), device=dev,
                                           dtype=torch.bfloat16, seq_lens=lens)

    mgr._resident_meta = setup(draw())
    meta = mgr._resident_meta
    be.set_kernel_input_metadata(meta)
    for key, wrapper in mgr.lora_wrappers.items():
        wrapper.set_lora_info(be, *pool.get_module_buffers(key))
    prompts = torch.randint(0, cfg.vocab_size, (2, 512), device=dev)
    decode_ids = torch.randint(0, cfg.vocab_size, (64, 1), device=dev)
    kv = StaticKV(cfg, 64, 520, dev, torch.bfloat16)
    pos = torch.tensor([512], device=dev)
    stream = torch.cuda.current_stream(dev)
    out = {}

    def forward(_):
        out["logits"] = model.forward_mixed(prompts, decode_ids, kv, pos)

    with torch.inference_mode():
        g_fwd = capture(torch, forward, 1)
        set_lora_enabled(False)
        try:
            g_base = capture(torch, forward, 1)
        finally:
            set_lora_enabled(True)

        # Serving loop: warm the pool to its steady state, then time steps.
        warm, timed = 96, max(20, min(args.steps // 20, 60))
        ev = [[torch.cuda.Event(enable_timing=True) for _ in range(3)] for _ in range(timed)]
        step_ms, misses = [], []
        bank_bytes = pool.buffers.layout(R).total * 2
        for it in range(warm + timed):
            names = draw()
            before = set(pool.name_to_slot)
            k = it - warm
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            if k >= 0:
                ev[k][0].record(stream)
            assert setup(names) is meta
            if k >= 0:
                ev[k][1].record(stream)
            g_fwd.replay()
            if k >= 0:
                ev[k][2].record(stream)
            torch.cuda.synchronize()
            if k >= 0:
                step_ms.append((time.perf_counter() - t0) * 1e3)
                misses.append(sum(1 for n in dict.fromkeys(names) if n not in before))
        finite = bool(torch.isfinite(out["logits"]).all())

        # Pipelined serving: the next batch is prepared (its misses uploaded on
        # the copy stream) while this batch's forward runs; the step period is
        # the time between consecutive forwards' ends.
        ev_p = [torch.cuda.Event(enable_timing=True) for _ in range(timed + 1)]
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for k in range(timed + 1):
            g_fwd.replay()
            ev_p[k].record(stream)
            if k < timed:
                assert setup(draw()) is meta
        torch.cuda.synchronize()
        pipe_wall = (time.perf_counter() - t0) * 1e3 / (timed + 1)
        period_ms = [ev_p[k].elapsed_time(ev_p[k + 1]) for k in range(timed)]
        upload_ms = [a[0].elapsed_time(a[1]) for a in ev]
        fwd_ms = [a[1].elapsed_time(a[2]) for a in ev]
        miss_steps = [(u, m) for u, m in zip(upload_ms, misses) if m > 0]
        h2d = (sum(m for _, m in miss_steps) * bank_bytes / (sum(u for u, _ in miss_steps) * 1e-3) / 1e9
               if miss_steps else None)

        # The forward alone (adapters resident), with and without the LoRA deltas.
        reps = max(10, min(args.steps // 20, 50))
        t_fwd = time_graph(torch, g_fwd, reps, 1, stream)
        t_base = time_graph(torch, g_base, reps, 1, stream)

        # The LoRA calls of one layer at this batch's shapes, as the fused
        # model makes them (q|k|v and gate|up multi-slice), 32 layers each.
        used = len({int(s) for s in meta.weight_indices[: meta.bs].tolist()})
        xs = {4096: torch.randn(rows, 4096, device=dev).bfloat16(), 14336: torch.randn(rows, 14336, device=dev).bfloat16()}
        e = 2
        kernels = {}
        groups = {"q|k|v": names7[0:3], "o": names7[3:4], "gate|up": names7[4:6], "down": names7[6:7]}
        for gname, projs in groups.items():
            i = dims[f"layers.0.{projs[0]}"][0]
            outs = [dims[f"layers.0.{p}"][1] for p in projs]
            cols = [sum(outs[:k]) for k in range(len(outs))]
            y = torch.zeros(rows, sum(outs), device=dev, dtype=torch.bfloat16)
            bufs = [[pool.get_module_buffers(f"layers.{l}.{p}") for p in projs] for l in range(L)]

            def call(l, x=xs[i], y=y, bufs=bufs, cols=cols):
                ab = bufs[l % L]
                be.apply_lora_multi(x, [t[0] for t in ab], [t[1] for t in ab], y, cols)

            ms = time_graph(torch, capture(torch, call, L), reps * L, L, stream)
            nbytes = rows * i * e + sum(used * R * (i + o) * e + 2 * rows * o * e for o in outs)
            kernels[gname] = {"us_per_layer": round(ms * 1e3, 2), "us_per_step": round(ms * 1e3 * L, 1),
                              "bytes_per_layer": nbytes, "GB/s": round(nbytes / (ms * 1e-3) / 1e9, 1)}
    lora_calls_ms = sum(k["us_per_step"] for k in kernels.values()) / 1e3
    step_bytes = L * sum(k["bytes_per_layer"] for k in kernels.values())
    dom = max(kernels, key=lambda k: kernels[k]["us_per_step"])
    med = statistics.median
    result = {
        "metric": "c5 per-step latency (pool upload + 32-layer forward of the mixed batch)",
        "value": round(med(step_ms), 3),
        "unit": "ms",
        "n_gpus": 1,
        "steps": timed,
        "warmup": warm,
        "ms_per_step": round(statistics.mean(step_ms), 3),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (random-init weights, random token ids)",
        "config": {"workload": OTHER_WORKLOADS["c5_step"], "rows": rows, "segments": len(lens),
                   "model": "decoder.Decoder(DecoderConfig.llama3_8b()): base GEMMs (q|k|v and gate|up fused), "
                            "attention, HIP RMSNorm, LoRA on q/k/v/o/gate/up/down (q|k|v and gate|up as multi-slice "
                            "calls), LM head on the 66 next-token rows",
                   "timing": "wall clock per step (synchronised); events around the upload and the graph replay"},
        "breakdown": {"upload_ms_median": round(med(upload_ms), 3), "forward_ms_median": round(med(fwd_ms), 3),
                      "upload_share": round(med(upload_ms) / med(step_ms), 3),
                      "misses_per_step_mean": round(statistics.mean(misses), 2),
                      "miss_bytes_per_adapter": bank_bytes,
                      "h2d_GB/s_on_miss_steps": round(h2d, 1) if h2d else None},
        "pipelined": {"step_period_ms_median": round(med(period_ms), 3), "wall_ms_per_step": round(pipe_wall, 3),
                      "note": "next batch prepared while this batch's forward runs; uploads wait only for the "
                              "compute that last read the slot they overwrite"},
        "forward_resident": {"with_lora_ms": round(t_fwd, 3), "base_only_ms": round(t_base, 3),
                             "lora_ms": round(t_fwd - t_base, 3),
                             "lora_share_of_forward": round((t_fwd - t_base) / t_fwd, 3),
                             "logits_finite": finite},
        "lora_calls": {"ms_per_step": round(lora_calls_ms, 3), "distinct_adapters": used,
                       "algorithmic_bytes_per_step": step_bytes,
                       "GB/s": round(step_bytes / (lora_calls_ms * 1e-3) / 1e9, 1), "kernels": kernels},
        "roofline": {"kernel": f"LoRA {dom}", "bound": "hbm", "achieved": kernels[dom]["GB/s"], "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(kernels[dom]["GB/s"] / HBM_PEAK_GBS, 4), "traffic": None},
    }
    print(json.dumps(result), flush=True)
    return 0


def bench_pool_upload(args) -> int:
    """mlora_pool_scatter from device-resident stage rows (the kernel's own
    rate), plus one PCIe-inclusive prepare_lora_batch of 4 new adapters."""
    import torch

    from multi_lora_amd import AdapterWeights, LoRAMemoryPool, _ffi

    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    proj = {"q": (4096, 4096), "k": (4096, 1024), "v": (4096, 1024), "o": (4096, 4096),
            "gate": (4096, 14336), "up": (4096, 14336), "down": (14336, 4096)}
    dims = {f"layers.{l}.{n}": d for l in range(32) for n, d in proj.items()}
    rank, h, k_slots = 16, 4, 8
    g = torch.Generator().manual_seed(5)

    def make(seed):
        g.manual_seed(seed)
        return AdapterWeights(rank=rank, scaling=2.0, modules={
            k: (torch.randn(rank, i, generator=g).bfloat16(), torch.randn(o, rank, generator=g).bfloat16())
            for k, (i, o) in dims.items()})

    pool = LoRAMemoryPool(k_slots, rank, dev, torch.bfloat16)
    store = {f"a{i}": make(i) for i in range(h)}
    t0 = time.perf_counter()
    pool.prepare_lora_batch(list(store), weight_store=store)
    torch.cuda.synchronize()
    upload_ms = (time.perf_counter() - t0) * 1e3   # includes packing the host banks once
    # Two more batches fill the 8 slots and then evict the first 4 (LRU), so
    # the timed call reloads them from their packed, pinned host banks.
    store2 = {f"b{i}": make(100 + i) for i in range(h)}
    store3 = {f"c{i}": make(200 + i) for i in range(h)}
    pool.prepare_lora_batch(list(store2), weight_store=store2)
    pool.prepare_lora_batch(list(store3), weight_store=store3)
    torch.cuda.synchronize()
    assert not any(n in pool.name_to_slot for n in store), "the first adapters should have been evicted"
    t0 = time.perf_counter()
    pool.prepare_lora_batch(list(store), weight_store=store)
    torch.cuda.synchronize()
    reload_ms = (time.perf_counter() - t0) * 1e3

    buf = pool.buffers
    plan = buf.layout(rank)
    table = buf._key_table(plan)
    stage = torch.randn(h, plan.total, device=dev).bfloat16()
    slots = torch.arange(h, dtype=torch.int32, device=dev)
    lib = _ffi.lib()
    stream = torch.cuda.current_stream(dev)

    def scatter(_):
        _ffi.check(lib.mlora_pool_scatter(stage.data_ptr(), stage.stride(0), h, slots.data_ptr(), table.data_ptr(),
                                          len(plan.keys), rank, k_slots, plan.max_numel, _ffi.MLORA_BF16,
                                          _ffi.stream_ptr(dev)), "mlora_pool_scatter")

    scatter(0)
    torch.cuda.synchronize()
    ms = time_graph(torch, capture(torch, scatter, 16), max(args.kernel_steps // 8, 64), 16, stream)
    nbytes = 2 * h * plan.total * 2
    result = {
        "metric": "pool upload scatter GB/s",
        "value": round(nbytes / (ms * 1e-3) / 1e9, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": max(args.kernel_steps // 8, 64),
        "warmup": 1,
        "ms_per_step": ms,
        "us_per_step": ms * 1e3,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {"workload": OTHER_WORKLOADS["pool_upload"], "keys": len(plan.keys),
                   "bank_elements": plan.total, "algorithmic_bytes_per_step": nbytes,
                   "timing": "HIP graph replay of the scatter alone; stage rows resident in HBM"},
        "pcie_inclusive": {"first_upload_ms": upload_ms, "reload_ms": reload_ms,
                           "note": "prepare_lora_batch of 4 adapters: pinned-bank H2D on the copy stream + scatter; "
                                   "the first upload also packs the host banks"},
        "roofline": {"kernel": "scatter_kernel", "bound": "hbm", "achieved": round(nbytes / (ms * 1e-3) / 1e9, 2),
                     "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(nbytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4), "traffic": None},
    }
    print(json.dumps(result), flush=True)
    return 0


class RotatingTimer:
    """Regions of exactly ``k`` calls of ``fn`` over ``n_rep`` rotating replicas.

    Call ``i`` of the sequence uses replica ``i % n_rep`` (``fn(i)`` picks it),
    and every region starts at the call after the previous region's last, so a
    replica comes back only after the ``n_rep - 1`` others, however ``k`` and
    ``n_rep`` relate.  One HIP graph is captured per start offset the rotation
    reaches (``n_rep / gcd(k, n_rep)`` of them); constructing the timer replays
    each once, in rotation order, untimed.  ``run(regions)`` returns the
    milliseconds per call of each region, each timed with HIP events on
    ``stream`` between synchronisations.
    """

    MAX_CAPTURED_CALLS = 40000

    def __init__(self, torch, fn, n_rep: int, k: int, stream):
        import math

        n_off = n_rep // math.gcd(k, n_rep)
        if n_off * k > self.MAX_CAPTURED_CALLS:
            raise SystemExit(f"{k} steps over {n_rep} replicas need {n_off} graphs of {k} calls; "
                             f"pick a step count with a larger common divisor with {n_rep}")
        self.torch, self.k, self.stream = torch, k, stream
        self.graphs = [capture(torch, lambda i, o=(j * k) % n_rep: fn(o + i), k) for j in range(n_off)]
        self.next = 0
        self.run(n_off)

    def run(self, regions: int) -> list:
        torch = self.torch
        t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        out = []
        for _ in range(regions):
            g = self.graphs[self.next % len(self.graphs)]
            self.next += 1
            torch.cuda.synchronize()
            t0.record(self.stream)
            g.replay()
            t1.record(self.stream)
            torch.cuda.synchronize()
            out.append(t0.elapsed_time(t1) / self.k)
        return out

    def median(self, regions: int) -> float:
        t = sorted(self.run(regions))
        return t[len(t) // 2]


def touched_bytes(host) -> int:
    """Distinct bytes one call touches: the algorithmic bytes with the output counted once."""
    from multi_lora_amd import synthetic

    return synthetic.algorithmic_bytes(host) - host.base.numel() * host.base.element_size()


def replicas_for(touched_bytes: int, floor: int = 2) -> int:
    """Replicas whose touched bytes add up to at least 600 MB, over twice the
    256 MiB MALL, so a replica's lines are gone from it when it comes back."""
    return max(floor, -(-600_000_000 // max(1, touched_bytes)))


def rotation_calls(n_rep: int, at_least: int = 32) -> int:
    """A region length that is a whole number of rotations (one graph) and at least ``at_least`` calls."""
    return n_rep * max(1, -(-at_least // n_rep))


def time_graph(torch, g, calls: int, per_graph: int, stream) -> float:
    """Milliseconds per call of a graph holding `per_graph` calls, replayed back to back."""
    replays = max(1, calls // per_graph)
    g.replay()
    torch.cuda.synchronize()
    t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0.record(stream)
    for _ in range(replays):
        g.replay()
    t1.record(stream)
    torch.cuda.synchronize()
    return t0.elapsed_time(t1) / (replays * per_graph)


_CAPTURE_STREAM = []


def capture_stream(torch):
    """The one stream every graph of the bench is captured on."""
    if not _CAPTURE_STREAM:
        _CAPTURE_STREAM.append(torch.cuda.Stream())
    return _CAPTURE_STREAM[0]


def capture(torch, fn, n: int):
    """Graph of fn(0), ..., fn(n-1), captured after running the same calls
    once on the capture stream (so per-stream workspaces exist beforehand
    and nothing is allocated or cleared inside the graph)."""
    s = capture_stream(torch)
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for i in range(n):
            fn(i)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        for i in range(n):
            fn(i)
    torch.cuda.synchronize()
    return g


def bench_other(args) -> int:
    """One line for a non-headline workload: the backend step and each of its kernels, graph-timed
    over cold replicas (at least 600 MB in total, more than twice the 256 MB MALL)."""
    import torch

    from multi_lora_amd import HipLoRABackend, synthetic
    from multi_lora_amd.kernels.lora_ops import (LinkedWorkspace, Workspace, apply_grouped, expand,
                                                 rmsnorm_apply_grouped, shrink)
    from multi_lora_amd.kernels.rmsnorm import rmsnorm_fwd

    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    name = args.workload
    host = workload_host(name)
    bare = name == "decode_q_device_plan"
    meta = synthetic.make_meta(host.seg_lens, host.seg_slots, host.slot_ranks, host.scalings, dev, torch.bfloat16,
                               host_copies=not bare, with_plan=not bare)
    e = host.x.element_size()
    n_rep = replicas_for(touched_bytes(host))
    reps = []
    for _ in range(n_rep):
        reps.append((host.x.to(dev), [a.to(dev) for a in host.a_stacks], [b.to(dev) for b in host.b_stacks],
                     host.base.to(dev)))
    S, in_dim, r_max, n = host.tokens, host.x.shape[1], host.a_stacks[0].shape[1], len(host.a_stacks)
    cols = host.col_offsets
    be = HipLoRABackend()
    be.set_kernel_input_metadata(meta)
    stream = torch.cuda.current_stream(dev)
    lora_bytes = synthetic.algorithmic_bytes(host)
    kernels = {}
    calls = max(args.kernel_steps // 8, 128)

    if name in ("decode_qkv", "decode_qkv_fused"):
        w = host.extra["norm_weight"].to(dev)
        eps = host.extra["eps"]
        xn = [torch.empty_like(r[0]) for r in reps]
        norm_bytes = 2 * S * in_dim * e + in_dim * e
        from multi_lora_amd import _ffi

        lib = _ffi.lib()

        def norm(i):
            x = reps[i % n_rep][0]
            _ffi.check(lib.mlora_rmsnorm(x.data_ptr(), x.stride(0), x.stride(0), 1, w.data_ptr(),
                                         _ffi.dtype_code(w.dtype), xn[i % n_rep].data_ptr(), xn[i % n_rep].stride(0),
                                         S, in_dim, eps, _ffi.dtype_code(x.dtype), _ffi.stream_ptr(dev)),
                       "mlora_rmsnorm")

        def lora(i):
            _, a, b, out = reps[i % n_rep]
            assert apply_grouped(xn[i % n_rep], a, b, meta, out, cols, be.linked_workspace, mode=0)

        def step(i):
            x, a, b, out = reps[i % n_rep]
            if name == "decode_qkv_fused":
                be.rmsnorm_apply_lora_multi(x, w, eps, a, b, out, cols)
                return
            y = rmsnorm_fwd(x, w, eps)
            be.apply_lora_multi(y, a, b, out, cols)

        def lora_two(i):
            _, a, b, out = reps[i % n_rep]
            assert apply_grouped(xn[i % n_rep], a, b, meta, out, cols, be.linked_workspace, mode=2)

        resid = [torch.randn_like(r[0]) for r in reps]
        ys = [torch.empty_like(r[0]) for r in reps]

        def add_norm(i):
            x = reps[i % n_rep][0]
            _ffi.check(lib.mlora_add_rmsnorm(x.data_ptr(), x.stride(0), resid[i % n_rep].data_ptr(), in_dim,
                                             w.data_ptr(), _ffi.dtype_code(w.dtype), ys[i % n_rep].data_ptr(),
                                             in_dim, S, in_dim, eps, _ffi.dtype_code(x.dtype), _ffi.stream_ptr(dev)),
                       "mlora_add_rmsnorm")

        def add_then_norm(i):
            x, r = reps[i % n_rep][0], resid[i % n_rep]
            r.add_(x)
            _ffi.check(lib.mlora_rmsnorm(r.data_ptr(), r.stride(0), r.stride(0), 1, w.data_ptr(),
                                         _ffi.dtype_code(w.dtype), ys[i % n_rep].data_ptr(), in_dim, S, in_dim, eps,
                                         _ffi.dtype_code(x.dtype), _ffi.stream_ptr(dev)), "mlora_rmsnorm")

        # Fused, x is one input of both the norm rows and the shrink: y written and the weight on top of
        # the LoRA bytes.  Unfused, the RMSNorm reads x and the LoRA path reads y.
        fused_bytes = lora_bytes + S * in_dim * e + in_dim * e
        total_bytes = fused_bytes if name == "decode_qkv_fused" else lora_bytes + norm_bytes
        add_bytes = 4 * S * in_dim * e + in_dim * e
        def lora_one(i):
            _, a, b, out = reps[i % n_rep]
            assert apply_grouped(xn[i % n_rep], a, b, meta, out, cols, be.linked_workspace, mode=1)

        def fused_norm(i):
            x, a, b, out = reps[i % n_rep]
            assert rmsnorm_apply_grouped(x, w, eps, xn[i % n_rep], a, b, meta, out, cols, be.linked_workspace)

        parts = {"rmsnorm": (norm, norm_bytes),
                 "rmsnorm folded into the planned decode's shrink launch (two launches)": (fused_norm, fused_bytes),
                 "planned decode (3 slices, the library's choice of schedule)": (lora, lora_bytes),
                 "planned decode, one launch (schedule comparison)": (lora_one, lora_bytes),
                 "planned decode, two launches (schedule comparison)": (lora_two, lora_bytes),
                 "add_rmsnorm fused (schedule comparison)": (add_norm, add_bytes),
                 "add then rmsnorm, unfused (schedule comparison)": (add_then_norm, add_bytes)}
        path = ("HipLoRABackend.rmsnorm_apply_lora_multi (the RMSNorm in the planned decode's shrink launch)"
                if name == "decode_qkv_fused" else
                "rmsnorm_fwd, then HipLoRABackend.apply_lora_multi (slot-planned decode, the library's schedule)")
    elif name in GROUPED_WORKLOADS:
        def lora(i):
            x, a, b, out = reps[i % n_rep]
            assert apply_grouped(x, a, b, meta, out, cols, be.linked_workspace, mode=0)

        def lora_two(i):
            x, a, b, out = reps[i % n_rep]
            assert apply_grouped(x, a, b, meta, out, cols, be.linked_workspace, mode=2)

        def step(i):
            x, a, b, out = reps[i % n_rep]
            be.apply_lora_multi(x, a, b, out, cols)

        total_bytes = lora_bytes
        parts = {"planned decode (the library's choice of schedule)": (lora, lora_bytes),
                 "planned decode, two launches (schedule comparison)": (lora_two, lora_bytes)}
        path = "HipLoRABackend.apply_lora (slot-planned decode, the library's schedule)"
    else:
        mids = [torch.empty(S, n * r_max, dtype=host.x.dtype, device=dev) for _ in range(n_rep)]
        ws = Workspace()
        a_bytes = host.x.numel() * e + sum(host.slot_ranks[s] * in_dim * e * n for s in set(host.seg_slots))
        b_bytes = lora_bytes - a_bytes

        def sh(i):
            x, a, _, _ = reps[i % n_rep]
            shrink(x, a, meta, mids[i % n_rep], workspace=ws)

        def ex(i):
            _, _, b, out = reps[i % n_rep]
            expand(mids[i % n_rep], b, meta, out, cols)

        def step(i):
            x, a, b, out = reps[i % n_rep]
            be.apply_lora_multi(x, a, b, out, cols)

        total_bytes = lora_bytes
        parts = {"shrink": (sh, a_bytes), "expand": (ex, b_bytes)}
        path = ("HipLoRABackend.apply_lora_multi (one mlora_apply_segments call: segment shrink, then the "
                "mixed-batch expand; the parts are the two-call path)" if name.startswith("c5_") else
                "HipLoRABackend.apply_lora_multi (segment shrink, then expand)")

    for i in range(max(args.warmup // 10, 2 * n_rep)):
        step(i)
    torch.cuda.synchronize()
    regions = args.regions or min(101, max(5, -(-2000 // args.steps)))
    step_ms = RotatingTimer(torch, step, n_rep, args.steps, stream).median(regions)
    # Parts: regions of whole rotations (one graph of at least 32 calls).
    per_graph = rotation_calls(n_rep)
    for k, (fn, nbytes) in parts.items():
        ms = RotatingTimer(torch, fn, n_rep, per_graph, stream).median(max(3, calls // per_graph))
        kernels[k] = {"us": ms * 1e3, "bytes": nbytes, "GB/s": nbytes / (ms * 1e-3) / 1e9}
    fb, pe = be.linked_workspace.counters()
    if pe:
        raise RuntimeError(f"{pe} plan errors; timings are void")
    dom = max((k for k in kernels if "comparison" not in k), key=lambda k: kernels[k]["us"])
    fl = synthetic.flops(host)
    result = {
        "metric": METRIC,
        "value": round(total_bytes / (step_ms * 1e-3) / 1e9, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": step_ms,
        "us_per_step": step_ms * 1e3,
        "tokens_per_s": S / (step_ms * 1e-3),
        "tflops": fl / (step_ms * 1e-3) / 1e12,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {"workload": OTHER_WORKLOADS[name], "tokens": S, "segments": len(host.seg_lens),
                   "algorithmic_bytes_per_step": total_bytes, "flops_per_step": fl, "replicas": n_rep,
                   "timing": "HIP graph replay, HIP events on the launch stream", "path": path,
                   "handoff_fallback_chunks": fb},
        "kernels": kernels,
        "roofline": {"kernel": dom, "bound": "hbm", "achieved": round(kernels[dom]["GB/s"], 2),
                     "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": round(kernels[dom]["GB/s"] / HBM_PEAK_GBS, 4),
                     "traffic": traffic_bytes(name, "" if name in GROUPED_WORKLOADS else dom)},
    }
    if not args.no_cpu_baseline:
        result["cpu_baseline"] = cpu_baseline_other(name, host, total_bytes, args.cpu_seconds)
    print(json.dumps(result), flush=True)
    return 0


def sweep_decode(args) -> int:
    """The planned decode path over decode shapes around the headline: token
    counts, adapter counts and ranks at q_proj 4096->4096, and q|k|v at
    4096->[4096,1024,1024].  Each shape: the backend's call, graph-timed over
    cold replicas (at least 600 MB), and both schedules for comparison."""
    import torch

    from multi_lora_amd import synthetic
    from multi_lora_amd.kernels.lora_ops import LinkedWorkspace, apply_grouped

    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    stream = torch.cuda.current_stream(dev)
    shapes = [dict(tokens=t, n_adapters=32, rank=16) for t in (16, 32, 64, 128, 256, 512)]
    shapes += [dict(tokens=128, n_adapters=a, rank=16) for a in (1, 8, 64)]
    shapes += [dict(tokens=128, n_adapters=32, rank=r) for r in (8, 32, 64)]
    shapes += [dict(tokens=t, n_adapters=64, rank=16, qkv=True) for t in (64, 256)]
    for sh in shapes:
        qkv = sh.pop("qkv", False)
        n_slots = max(64, 2 * sh["n_adapters"])
        if qkv:
            host = synthetic.decode_qkv(device="cpu", tokens=sh["tokens"], n_slots=n_slots, n_adapters=sh["n_adapters"],
                                        rank=sh["rank"], seed=5)
        else:
            host = synthetic.decode_q(device="cpu", n_slots=n_slots, seed=5, **sh)
        meta = synthetic.make_meta(host.seg_lens, host.seg_slots, host.slot_ranks, host.scalings, dev, torch.bfloat16)
        n_rep = replicas_for(touched_bytes(host))
        reps = [(host.x.to(dev), [a.to(dev) for a in host.a_stacks], [b.to(dev) for b in host.b_stacks],
                 host.base.to(dev)) for _ in range(n_rep)]
        lws = LinkedWorkspace()
        nbytes = synthetic.algorithmic_bytes(host)
        res = {}
        for mode in (0, 1, 2):
            def call(i, mode=mode):
                x, a, b, out = reps[i % n_rep]
                assert apply_grouped(x, a, b, meta, out, host.col_offsets, lws, mode=mode)
            per_graph = rotation_calls(n_rep)
            timer = RotatingTimer(torch, call, n_rep, per_graph, stream)
            res[mode] = timer.median(max(5, args.kernel_steps // per_graph)) * 1e3
        fb, pe = lws.counters()
        if pe:
            raise RuntimeError(f"{pe} plan errors; timings are void")
        us = res[0]
        print(json.dumps({
            "shape": ("q|k|v 4096->[4096,1024,1024]" if qkv else "q_proj 4096->4096"), **sh,
            "slots": n_slots, "entries": meta.plan_entries, "us": round(us, 2),
            "GB/s": round(nbytes / (us * 1e-6) / 1e9, 1), "frac": round(nbytes / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
            "algorithmic_bytes": nbytes, "one_launch_us": round(res[1], 2), "two_launches_us": round(res[2], 2),
            "library_pick": "one launch" if abs(res[0] - res[1]) <= abs(res[0] - res[2]) else "two launches",
            "handoff_fallback_chunks": fb}), flush=True)
    return 0


def cpu_baseline_other(name: str, host, total_bytes: int, budget_s: float) -> dict:
    """The oracle's per-segment PyTorch path (plus its RMSNorm for decode_qkv)
    on the host cores, bf16, same inputs; at least 3 timed steps."""
    import torch

    from oracle.lora_ref import TorchLoRABackend
    from oracle.rmsnorm_ref import rmsnorm_ref

    cores = cpu_cores()
    torch.set_num_threads(cores)
    be = TorchLoRABackend()
    be.set_kernel_input_metadata(host.meta)
    w = host.extra.get("norm_weight")

    def step():
        x = host.x
        if w is not None:
            x = rmsnorm_ref(x, w, host.extra["eps"])
        out = host.base.clone()
        for a, b, c0 in zip(host.a_stacks, host.b_stacks, host.col_offsets):
            be.apply_lora(x, a, b, out[:, c0:c0 + b.shape[1]])

    step()
    times = []
    start = time.perf_counter()
    while (time.perf_counter() - start < budget_s and len(times) < 50) or len(times) < 3:
        t = time.perf_counter_ns()
        step()
        times.append(time.perf_counter_ns() - t)
    times.sort()
    med_s = times[len(times) // 2] * 1e-9
    return {
        "value": round(total_bytes / med_s / 1e9, 4),
        "unit": "GB/s",
        "us_per_step": med_s * 1e6,
        "cores": cores,
        "kind": "port",
        "cpu": cpu_model(),
        "sample": f"median of {len(times)} full {name} steps (bf16, host tensors)",
    }


# --profile-traffic: the copy kernel used to calibrate the counters moves
# COPY_ELEMS bf16 values (read once, written once).
COPY_ELEMS = 32 << 20
PROFILE_CALLS = 64
GROUPED_WORKLOADS = ("decode_q", "decode_q_resident", "decode_q_device_plan", "decode_qkv", "decode_qkv_fused")
PREFILL_WORKLOADS = ("prefill_gate_up", "prefill_down", "c5_gate_up", "c5_qkv", "c5_o", "c5_down")
MFMA_COUNTERS = ("SQ_INSTS_VALU_MFMA_MOPS_BF16", "SQ_VALU_MFMA_BUSY_CYCLES", "GRBM_GUI_ACTIVE")


def grouped_host(name: str):
    from multi_lora_amd import synthetic

    if name in ("decode_q", "decode_q_device_plan"):
        return synthetic.decode_q(device="cpu")
    if name == "decode_q_resident":
        return synthetic.decode_q(device="cpu", resident=64)
    return synthetic.decode_qkv(device="cpu")


def workload_host(name: str):
    from multi_lora_amd import synthetic

    if name in GROUPED_WORKLOADS:
        return grouped_host(name)
    if name.startswith("c5_"):
        return synthetic.mixed_c5(device="cpu", part=name.split("_", 1)[1])
    return synthetic.prefill_mlp(device="cpu", part=name.split("_", 1)[1])


def traffic_file(name: str) -> Path:
    family = "planned_decode" if name in GROUPED_WORKLOADS else "segment"
    return ROOT / "profiles" / f"{family}_{name}_traffic.json"


def traffic_bytes(name: str, prefix: str = ""):
    """Counter HBM bytes per call of the workload's LoRA path, or of its kernels whose short name starts
    with ``prefix``; None when no counter summary is committed."""
    f = traffic_file(name)
    if not f.exists():
        return None
    d = json.loads(f.read_text())
    if not prefix:
        return d.get("hbm_bytes_per_call")
    ks = [v for k, v in d.get("kernels", {}).items() if k.startswith(prefix)]
    return round(sum(k["hbm_bytes_per_call"] for k in ks)) if ks else None


def profile_traffic(name: str) -> int:
    """PROFILE_CALLS calls of a workload's LoRA path as the backend runs it
    (HipLoRABackend.apply_lora_multi; decode_qkv's input normalised
    beforehand; decode_qkv_fused: HipLoRABackend.rmsnorm_apply_lora_multi on
    the raw rows), over rotating replicas, then a plain copy kernel of known
    size.  Meant to run under rocprofv3 --pmc."""
    import torch

    from multi_lora_amd import HipLoRABackend, synthetic
    from multi_lora_amd.kernels.rmsnorm import rmsnorm_fwd

    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    host = workload_host(name)
    bare = name == "decode_q_device_plan"
    meta = synthetic.make_meta(host.seg_lens, host.seg_slots, host.slot_ranks, host.scalings, dev, torch.bfloat16,
                               host_copies=not bare, with_plan=not bare)
    n_rep = replicas_for(touched_bytes(host))
    reps = [(host.x.to(dev), [a.to(dev) for a in host.a_stacks], [b.to(dev) for b in host.b_stacks],
             host.base.to(dev)) for _ in range(n_rep)]
    fused = name == "decode_qkv_fused"
    if "norm_weight" in host.extra:
        w = host.extra["norm_weight"].to(dev)
        if not fused:
            reps = [(rmsnorm_fwd(x, w, host.extra["eps"]), a, b, out) for x, a, b, out in reps]
    be = HipLoRABackend()
    be.set_kernel_input_metadata(meta)
    torch.cuda.synchronize()
    for i in range(PROFILE_CALLS):
        x, a, b, out = reps[i % n_rep]
        if fused:
            be.rmsnorm_apply_lora_multi(x, w, host.extra["eps"], a, b, out, host.col_offsets)
        else:
            be.apply_lora_multi(x, a, b, out, host.col_offsets)
    torch.cuda.synchronize()
    src = torch.randn(COPY_ELEMS, device=dev).bfloat16()
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    for _ in range(16):
        torch.neg(src, out=dst)
    torch.cuda.synchronize()
    fb, pe = be.linked_workspace.counters()
    print(json.dumps({"workload": name, "calls": PROFILE_CALLS, "copy_launches": 16,
                      "copy_bytes_each_way": COPY_ELEMS * 2, "fallback_chunks": fb, "plan_errors": pe}))
    return 0


def _short_kernel(name: str) -> str:
    """``void mlora::(anonymous namespace)::planned_kernel<mlora::BF16, 2>(int const*, ...)``
    -> ``planned_kernel<BF16, 2>``."""
    s = name.replace("(anonymous namespace)::", "").replace("mlora::", "")
    if s.startswith("void "):
        s = s[5:]
    depth = 0
    for i, ch in enumerate(s):
        depth += ch == "<"
        depth -= ch == ">"
        if ch == "(" and depth == 0:
            return s[:i].strip()
    return s.strip()


def _pmc_sums(directory: str, counter: str) -> dict:
    """Per short kernel name, the sum of ``counter`` over the LoRA path's
    dispatches; the copy kernel's mean per dispatch under ``"copy"``."""
    import csv

    files = sorted(Path(directory).rglob("*counter_collection.csv"))
    if not files:
        raise SystemExit(f"no counter_collection.csv under {directory}")
    sums, copy = {}, []
    for f in files:
        with open(f, newline="") as fh:
            for row in csv.DictReader(fh):
                if row.get("Counter_Name") != counter:
                    continue
                full = row.get("Kernel_Name", "")
                v = float(row["Counter_Value"])
                if "mlora::" in full:
                    k = _short_kernel(full)
                    if not k.startswith("rmsnorm_kernel"):
                        sums[k] = sums.get(k, 0.0) + v
                elif "neg" in full:
                    copy.append(v)
    if not sums:
        raise SystemExit(f"{counter}: no path kernels in {directory}")
    return {"kernels": sums, "copy": sum(copy) / len(copy) if copy else None}


def summarize_pmc(name: str, dirs) -> int:
    """FETCH_SIZE and WRITE_SIZE runs (and optionally an MFMA-counter run) of
    --profile-traffic -> the workload's counter summary under profiles/."""
    from multi_lora_amd import synthetic

    fetch = _pmc_sums(dirs[0], "FETCH_SIZE")
    write = _pmc_sums(dirs[1], "WRITE_SIZE")
    copy_kib = COPY_ELEMS * 2 / 1024
    f_scale, w_scale = copy_kib / fetch["copy"], copy_kib / write["copy"]
    host = workload_host(name)
    algo = synthetic.algorithmic_bytes(host)
    reads = algo - host.base.numel() * host.x.element_size()
    if name == "decode_qkv_fused":
        # the RMSNorm's y written and its weight read; x, which the norm rows and the shrink items both
        # read, is counted once, with the LoRA bytes
        e = host.x.element_size()
        algo += host.x.numel() * e + host.extra["norm_weight"].numel() * e
        reads += host.extra["norm_weight"].numel() * e
    kernels = {}
    for k in sorted(set(fetch["kernels"]) | set(write["kernels"])):
        fb = fetch["kernels"].get(k, 0.0) / PROFILE_CALLS * f_scale * 1024
        wb = write["kernels"].get(k, 0.0) / PROFILE_CALLS * w_scale * 1024
        kernels[k] = {"fetch_bytes_per_call": round(fb), "write_bytes_per_call": round(wb),
                      "hbm_bytes_per_call": round(fb + wb)}
    commands = [
        f"timeout -s KILL 60 rocprofv3 --pmc FETCH_SIZE -d <FETCH_DIR> -f csv -- python3 bench.py "
        f"--profile-traffic --workload {name}",
        f"timeout -s KILL 60 rocprofv3 --pmc WRITE_SIZE -d <WRITE_DIR> -f csv -- python3 bench.py "
        f"--profile-traffic --workload {name}",
    ]
    if len(dirs) > 2:
        fl = synthetic.flops(host)
        for c in MFMA_COUNTERS:
            sums = _pmc_sums(dirs[2], c)["kernels"]
            for k, v in sums.items():
                kernels.setdefault(k, {})[c + "_per_call"] = round(v / PROFILE_CALLS)
        mops = sum(kernels[k].get("SQ_INSTS_VALU_MFMA_MOPS_BF16_per_call", 0) for k in kernels)
        mfma = {"algorithmic_flops_per_call": fl, "mfma_flops_per_call": mops * 512,
                "mfma_over_algorithmic": round(mops * 512 / fl, 4) if fl else None,
                "note": "SQ_INSTS_VALU_MFMA_MOPS_BF16 counts units of 512 flops; the excess over the "
                        "algorithmic flops is the zero padding of rank and row tiles"}
        commands.append(f"timeout -s KILL 60 rocprofv3 --pmc {' '.join(MFMA_COUNTERS)} -d <MFMA_DIR> -f csv -- "
                        f"python3 bench.py --profile-traffic --workload {name}")
    else:
        mfma = None
    total_f = sum(k.get("fetch_bytes_per_call", 0) for k in kernels.values())
    total_w = sum(k.get("write_bytes_per_call", 0) for k in kernels.values())
    commands.append(f"python3 bench.py --workload {name} --summarize-pmc <FETCH_DIR> <WRITE_DIR>"
                    + (" <MFMA_DIR>" if len(dirs) > 2 else ""))
    out = {
        "workload": OTHER_WORKLOADS.get(name, HEADLINE_WORKLOAD),
        "path": ("HipLoRABackend.rmsnorm_apply_lora_multi (the RMSNorm in the shrink launch)"
                 if name == "decode_qkv_fused" else "HipLoRABackend.apply_lora_multi, the library's choice of kernels"),
        "calls": PROFILE_CALLS,
        "algorithmic_bytes_per_call": algo,
        "hbm_bytes_per_call": total_f + total_w,
        "fetch_bytes_per_call": total_f,
        "write_bytes_per_call": total_w,
        "traffic_over_algorithmic": round((total_f + total_w) / algo, 4),
        "fetch_over_algorithmic_reads": round(total_f / reads, 4),
        "kernels": kernels,
        "mfma": mfma,
        "copy_calibration": {"bytes_each_way": COPY_ELEMS * 2, "FETCH_SIZE_kib": fetch["copy"],
                             "WRITE_SIZE_kib": write["copy"], "fetch_scale": f_scale, "write_scale": w_scale},
        "commands": commands,
    }
    traffic_file(name).write_text(json.dumps(out, indent=1) + "\n")
    print(json.dumps(out))
    return 0


def cpu_cores() -> int:
    n = len(os.sched_getaffinity(0))
    try:
        quota, period = open("/sys/fs/cgroup/cpu.max").read().split()
        if quota != "max":
            n = min(n, max(1, int(int(quota) / int(period))))
    except (OSError, ValueError):
        pass
    return n


def cpu_model() -> str:
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def main() -> int:
    args = parse()
    if args.summarize_pmc:
        if len(args.summarize_pmc) not in (2, 3):
            raise SystemExit("--summarize-pmc takes FETCH_DIR WRITE_DIR [MFMA_DIR]")
        return summarize_pmc(args.workload, args.summarize_pmc)
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (asked for --gpus {args.gpus}); "
              "multi-GPU sharding of this path is design-only", file=sys.stderr)
        return 2

    if args.profile_traffic:
        return profile_traffic(args.workload)
    if args.calibrate:
        return calibrate(args)
    if args.sweep == "decode":
        return sweep_decode(args)
    if args.workload == "pool_upload":
        return bench_pool_upload(args)
    if args.workload == "c5_step":
        return bench_c5_step(args)
    if args.workload != "decode_q":
        return bench_other(args)

    import torch

    from multi_lora_amd import HipLoRABackend, synthetic
    from multi_lora_amd.kernels.lora_ops import apply_grouped

    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    host = synthetic.decode_q(device="cpu")
    meta = synthetic.make_meta(host.seg_lens, host.seg_slots, host.slot_ranks, host.scalings, dev, torch.bfloat16)

    reps = []
    for _ in range(args.replicas):
        reps.append((host.x.to(dev), host.a_stacks[0].to(dev), host.b_stacks[0].to(dev), host.base.to(dev)))
    torch.cuda.synchronize()

    be = HipLoRABackend()
    be.set_kernel_input_metadata(meta)
    stream = torch.cuda.current_stream(dev)

    def step(i, phases=3, mode=None):
        x, a, b, out = reps[i % len(reps)]
        if mode is None:
            be.apply_lora(x, a, b, out)
        else:
            launched = apply_grouped(x, [a], [b], meta, out, [0], be.linked_workspace, phases=phases, mode=mode)
            assert launched, "decode workload is expected to take the slot-planned path"

    for i in range(args.warmup):
        step(i)
    torch.cuda.synchronize()

    # The host enqueues a call in ~12 us, slower than the kernels run, so
    # steps are timed as HIP graph replays.  Each region is exactly `steps`
    # steps and starts at the replica after the previous region's last, so a
    # replica's lines have left the MALL when it comes back.
    regions = args.regions or min(101, max(5, -(-2000 // args.steps)))
    ms_per_step = RotatingTimer(torch, step, args.replicas, args.steps, stream).median(regions)
    timed_steps = args.steps
    # The backend's step is one launch of the planned kernel; the two-launch
    # schedule of the same work items is timed for comparison (regions of
    # whole rotations).
    per_rot = rotation_calls(args.replicas)
    kreg = max(3, -(-args.kernel_steps // per_rot))
    shrink_ms = RotatingTimer(torch, lambda i: step(i, 1, 2), args.replicas, per_rot, stream).median(kreg)
    expand_ms = RotatingTimer(torch, lambda i: step(i, 2, 2), args.replicas, per_rot, stream).median(kreg)
    fb, pe = be.linked_workspace.counters()
    if pe:
        raise RuntimeError(f"{pe} plan errors; timings are void")

    e = 2
    used = sorted({s for s in host.seg_slots if host.slot_ranks[s] > 0})
    r, in_dim, out_dim = 16, host.x.shape[1], host.b_stacks[0].shape[1]
    shrink_bytes = host.x.numel() * e + len(used) * r * in_dim * e
    expand_bytes = len(used) * out_dim * r * e + 2 * host.tokens * out_dim * e
    total_bytes = synthetic.algorithmic_bytes(host)
    assert total_bytes == shrink_bytes + expand_bytes
    touched = total_bytes - host.base.numel() * e  # the output's lines are read and written once each
    step_gbs = total_bytes / (ms_per_step * 1e-3) / 1e9

    def entry(ms, nbytes):
        return {"us": ms * 1e3, "bytes": nbytes, "GB/s": nbytes / (ms * 1e-3) / 1e9}

    kernels = {
        "planned_decode (one launch)": entry(ms_per_step, total_bytes),
        "planned_decode shrink half (two-launch schedule)": entry(shrink_ms, shrink_bytes),
        "planned_decode expand half (two-launch schedule)": entry(expand_ms, expand_bytes),
        "two-launch schedule total": entry(shrink_ms + expand_ms, total_bytes),
    }
    dom_name = "planned_decode (one launch)"
    dom = kernels[dom_name]
    traffic = traffic_bytes("decode_q")

    result = {
        "metric": METRIC,
        "value": round(step_gbs, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": timed_steps,
        "warmup": args.warmup,
        "ms_per_step": ms_per_step,
        "us_per_step": ms_per_step * 1e3,
        "tokens_per_s": host.tokens / (ms_per_step * 1e-3),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {
            "workload": HEADLINE_WORKLOAD,
            "tokens": host.tokens,
            "distinct_slots": len(used),
            "algorithmic_bytes_per_step": total_bytes,
            "replicas": args.replicas,
            "touched_bytes_per_rotation": args.replicas * touched,
            "timing": (f"median over {regions} regions of exactly {args.steps} steps, each a HIP graph replay "
                       f"timed with HIP events on the launch stream; each region starts at the replica after "
                       f"the previous region's last"),
            "path": "slot-planned shrink + expand, one launch (HipLoRABackend.apply_lora)",
            "handoff_fallback_chunks": fb,
        },
        "kernels": kernels,
        "roofline": {
            "kernel": dom_name,
            "bound": "hbm",
            "achieved": round(dom["GB/s"], 2),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(dom["GB/s"] / HBM_PEAK_GBS, 4),
            "traffic": traffic,
        },
    }

    if not args.no_other_configs:
        result["other_configs"] = other_configs()
    if not args.no_cpu_baseline:
        result["cpu_baseline"] = cpu_baseline(host, total_bytes, args.cpu_seconds)

    print(json.dumps(result), flush=True)
    return 0


def calibrate(args) -> int:
    """Floors of one launch at the headline size, and where the headline kernel's time goes.

    Loads the measurement library (``libmlora_calib.so``: the product's
    sources built with per-phase timestamps in the planned decode kernel,
    plus an empty and a streaming kernel) and prints one JSON line:

    * ``empty_kernel_us``: an empty kernel (1 and 1024 workgroups) per launch
      under HIP graph replay, 64 launches a graph;
    * ``stream_us``: one launch of 1024 workgroups reading the headline's
      11,534,336 algorithmic bytes, over rotating replicas (cold, at least
      600 MB a rotation) and from one buffer (hot, MALL-resident);
    * ``planned_decode_us``: the headline call (planned kernel, one launch)
      through the same library, graph-timed as the headline;
    * ``timeline``: per-phase quantiles (ns after the first workgroup
      starts) of the last call of 32 graph replays of 8 calls, cold
      replicas rotating as in the headline.
    """
    import ctypes
    import statistics

    import torch

    from multi_lora_amd import _ffi, synthetic
    from multi_lora_amd.build import CALIB_LIB
    from multi_lora_amd.kernels.lora_ops import _slices, seg_meta

    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    stream = torch.cuda.current_stream(dev)
    if not CALIB_LIB.exists():
        raise SystemExit(f"{CALIB_LIB} is not built (python -m multi_lora_amd.build)")
    lib = ctypes.CDLL(str(CALIB_LIB))
    vp, i32, i64 = ctypes.c_void_p, ctypes.c_int32, ctypes.c_int64
    lib.mlora_calib_empty.argtypes = [ctypes.c_int, vp, vp]
    lib.mlora_calib_stream.argtypes = [vp, i64, vp, ctypes.c_int, vp]
    lib.mlora_tl_clear.argtypes = [ctypes.c_int, vp]
    lib.mlora_tl_read.argtypes = [vp, ctypes.c_int]
    lib.mlora_last_error.restype = ctypes.c_char_p
    for name in ("mlora_apply_grouped", "mlora_grouped_workspace_bytes"):
        res, argt = _ffi._SIGNATURES[name]
        getattr(lib, name).restype = res
        getattr(lib, name).argtypes = argt

    def ok(rc, what):
        if rc != 0:
            raise RuntimeError(f"{what}: rc {rc} {lib.mlora_last_error().decode(errors='replace')}")

    sink = torch.zeros(4096, dtype=torch.int32, device=dev)
    result = {"metric": "launch floors and the planned decode kernel's timeline at the headline size",
              "workload": HEADLINE_WORKLOAD, "n_gpus": 1}

    # 1. The launch itself.
    empty = {}
    for blocks in (1, 1024):
        g = capture(torch, lambda i, b=blocks: ok(lib.mlora_calib_empty(b, sink.data_ptr(), _ffi.stream_ptr(dev)),
                                                  "empty"), 64)
        empty[f"{blocks}_workgroups"] = round(time_graph(torch, g, 64 * 50, 64, stream) * 1e3, 3)
    result["empty_kernel_us"] = empty

    # 2. One launch streaming the headline's bytes.
    host = synthetic.decode_q(device="cpu")
    nbytes = synthetic.algorithmic_bytes(host)
    n_rep = max(args.replicas, replicas_for(nbytes))
    bufs = [torch.full((nbytes,), i & 0x7F, dtype=torch.uint8, device=dev) for i in range(n_rep)]

    def stream_call(i):
        ok(lib.mlora_calib_stream(bufs[i % n_rep].data_ptr(), nbytes, sink.data_ptr(), 1024, _ffi.stream_ptr(dev)),
           "stream")

    per_rot = rotation_calls(n_rep)
    cold = RotatingTimer(torch, stream_call, n_rep, per_rot, stream).median(9)
    hot = time_graph(torch, capture(torch, lambda i: stream_call(0), 64), 64 * 20, 64, stream)
    result["stream_us"] = {"bytes": nbytes, "cold": round(cold * 1e3, 3), "hot": round(hot * 1e3, 3),
                           "cold_GB/s": round(nbytes / (cold * 1e-3) / 1e9, 1), "replicas": n_rep}
    del bufs

    # 3. The headline call through the same library.
    meta = synthetic.make_meta(host.seg_lens, host.seg_slots, host.slot_ranks, host.scalings, dev, torch.bfloat16)
    reps = [(host.x.to(dev), host.a_stacks[0].to(dev), host.b_stacks[0].to(dev), host.base.to(dev))
            for _ in range(args.replicas)]
    n_slots, r_max = host.a_stacks[0].shape[0], host.a_stacks[0].shape[1]
    in_dim, S = host.x.shape[1], host.tokens
    cmeta, keep = seg_meta(meta, dev, n_slots)
    slices = [_slices([a], [b], [0]) for _, a, b, _ in reps]
    ws_bytes = lib.mlora_grouped_workspace_bytes(in_dim, r_max, 1, S, n_slots, _ffi.MLORA_BF16, 1)
    ws = torch.zeros(ws_bytes, dtype=torch.uint8, device=dev)

    def decode_call(i):
        x, _, _, out = reps[i % len(reps)]
        ok(lib.mlora_apply_grouped(x.data_ptr(), x.stride(0), S, in_dim, slices[i % len(reps)], 1, r_max,
                                   out.data_ptr(), out.stride(0), ctypes.byref(cmeta), _ffi.MLORA_BF16,
                                   ws.data_ptr(), ws_bytes, 1, 3, _ffi.stream_ptr(dev)), "apply_grouped")

    timer = RotatingTimer(torch, decode_call, len(reps), args.steps, stream)
    result["planned_decode_us"] = round(timer.median(args.regions or 41) * 1e3, 3)

    # 4. Timeline: every workgroup writes its whole stamp record at its end,
    # so after a graph replay of 8 calls back to back the records are the
    # last call's, made in the timed protocol's conditions.
    e_grid = (int(meta.plan_entries) + 7) // 8 * 8
    kc, n_tiles = in_dim // 256, host.b_stacks[0].shape[1] // 256
    n_blk = (kc + n_tiles) * e_grid
    words = n_blk * 4 * 8
    buf = (ctypes.c_uint32 * words)()
    ph = {k: [] for k in ("s_start", "e_start", "s_entry", "s_data_wave", "s_reduced", "s_flag", "s_end", "e_entry", "e_requested",
                          "e_flags_seen", "e_sums", "e_y", "e_stored", "kernel_end")}
    crit = []
    tl_timer = RotatingTimer(torch, decode_call, len(reps), 8, stream)
    for it in range(32):
        ok(lib.mlora_tl_clear(words, _ffi.stream_ptr(dev)), "tl_clear")
        tl_timer.run(1)
        ok(lib.mlora_tl_read(ctypes.cast(buf, vp), words), "tl_read")
        t = torch.tensor(list(buf), dtype=torch.int64).view(n_blk, 4, 8)
        starts = t[:, :, 0][t[:, :, 0] > 0]
        # Low words of a 100 MHz counter: order them relative to one start,
        # modulo 2^32, then take the earliest start as time 0.
        ref0 = int(starts[0])
        wrap = lambda v: ((int(v) - ref0 + (1 << 31)) % (1 << 32)) - (1 << 31)  # noqa: E731
        t0 = min(wrap(v) for v in starts.tolist())
        rel = lambda v: (wrap(v) - t0) * 10  # noqa: E731  (10 ns ticks)
        flag_by_entry, seen_by_entry = {}, {}
        end = 0
        for b in range(n_blk):
            item, j = divmod(b, e_grid)
            w = t[b]
            if int(w[0, 1]) == 0:
                continue
            if item < kc:
                ph["s_start"].append(rel(w[0, 0]))
                ph["s_entry"].append(rel(w[0, 1]))
                ph["s_data_wave"] += [rel(w[q, 2]) for q in range(4) if int(w[q, 2]) > 0]
                ph["s_reduced"].append(rel(w[0, 3]))
                ph["s_flag"].append(rel(w[0, 4]))
                ph["s_end"].append(rel(w[0, 5]))
                flag_by_entry[j] = max(flag_by_entry.get(j, 0), rel(w[0, 4]))
                end = max(end, rel(w[0, 5]))
            else:
                ph["e_start"].append(rel(w[0, 0]))
                ph["e_entry"].append(rel(w[0, 1]))
                ph["e_requested"].append(rel(w[0, 2]))
                ph["e_flags_seen"].append(rel(w[0, 3]))
                ph["e_sums"].append(rel(w[0, 4]))
                ph["e_y"].append(rel(w[0, 5]))
                st = max(rel(w[q, 6]) for q in range(4))
                ph["e_stored"].append(st)
                seen_by_entry.setdefault(j, []).append(rel(w[0, 3]))
                end = max(end, st)
        ph["kernel_end"].append(end)
        crit += [statistics.median(v) - flag_by_entry[j] for j, v in seen_by_entry.items() if j in flag_by_entry]
    fb = int(ws[:4].view(torch.int32)[_ffi.WS_FALLBACKS].item())

    def q(v, f):
        v = sorted(v)
        return round(v[min(len(v) - 1, int(f * (len(v) - 1)))]) if v else None

    result["timeline_ns"] = {k: {"p10": q(v, 0.1), "p50": q(v, 0.5), "p90": q(v, 0.9), "max": q(v, 1.0)}
                             for k, v in ph.items()}
    result["timeline_ns"]["entry_last_flag_to_flags_seen"] = {"p50": q(crit, 0.5), "p90": q(crit, 0.9)}
    result["timeline_launches"] = 32
    result["handoff_fallback_chunks"] = fb
    result["phases"] = {
        "s_*": "shrink items: entry in, A and x in (each wave), four waves' sums in LDS, flag stored after the sums' "
               "acknowledgement, item done",
        "e_*": "expand items: entry in, B and output requested, every chunk flag seen, sums gathered, y in LDS, "
               "output stored and acknowledged (last wave)",
        "kernel_end": "last workgroup's end, ns after the first workgroup's start",
        "entry_last_flag_to_flags_seen": "per entry: median expand item's flags-seen minus the entry's last flag store",
    }
    print(json.dumps(result), flush=True)
    return 0


# The other configurations' calls, timed into the headline line (key
# "other_configs"): name -> (workload, what one step is).
OTHER_CONFIGS = {
    "c3_prefill_gate_up": ("prefill_gate_up", "HipLoRABackend.apply_lora_multi, gate|up (two slices)"),
    "c3_prefill_down": ("prefill_down", "HipLoRABackend.apply_lora_multi"),
    "c4_rmsnorm_qkv": ("decode_qkv", "rmsnorm_fwd, then HipLoRABackend.apply_lora_multi over q|k|v"),
    "c4_rmsnorm_qkv_fused": ("decode_qkv", "HipLoRABackend.rmsnorm_apply_lora_multi over q|k|v (the RMSNorm in the "
                                           "LoRA shrink's launch)"),
    "c5_qkv": ("c5_qkv", "HipLoRABackend.apply_lora_multi over q|k|v, one layer's call"),
    "c5_o": ("c5_o", "HipLoRABackend.apply_lora_multi, one layer's call"),
    "c5_gate_up": ("c5_gate_up", "HipLoRABackend.apply_lora_multi over gate|up, one layer's call"),
    "c5_down": ("c5_down", "HipLoRABackend.apply_lora_multi, one layer's call"),
}


def other_configs(regions: int = 7) -> dict:
    """Each other configuration's call as the backend makes it, under the
    headline's cold-replica protocol: replicas touching at least 600 MB in
    all, regions of whole rotations, median region."""
    import torch

    from multi_lora_amd import HipLoRABackend, synthetic
    from multi_lora_amd.kernels.rmsnorm import rmsnorm_fwd

    dev = torch.device("cuda", 0)
    stream = torch.cuda.current_stream(dev)
    res = {}
    for key, (name, what) in OTHER_CONFIGS.items():
        host = workload_host(name)
        meta = synthetic.make_meta(host.seg_lens, host.seg_slots, host.slot_ranks, host.scalings, dev,
                                   torch.bfloat16)
        n_rep = replicas_for(touched_bytes(host))
        reps = [(host.x.to(dev), [a.to(dev) for a in host.a_stacks], [b.to(dev) for b in host.b_stacks],
                 host.base.to(dev)) for _ in range(n_rep)]
        be = HipLoRABackend()
        be.set_kernel_input_metadata(meta)
        cols = host.col_offsets
        nbytes = synthetic.algorithmic_bytes(host)
        w = host.extra.get("norm_weight")
        if w is not None:
            w = w.to(dev)
            eps = host.extra["eps"]
            # unfused: x read by the RMSNorm, y written; fused: y written (x counted once, with the LoRA bytes)
            n_x = 1 if key.endswith("_fused") else 2
            nbytes += n_x * host.x.numel() * host.x.element_size() + w.numel() * w.element_size()

        def step(i, reps=reps, be=be, cols=cols, w=w, fused=key.endswith("_fused")):
            x, a, b, out = reps[i % len(reps)]
            if fused:
                be.rmsnorm_apply_lora_multi(x, w, eps, a, b, out, cols)
                return
            if w is not None:
                x = rmsnorm_fwd(x, w, eps)
            be.apply_lora_multi(x, a, b, out, cols)

        k = rotation_calls(n_rep)
        ms = RotatingTimer(torch, step, n_rep, k, stream).median(regions)
        fb, pe = be.linked_workspace.counters()
        if pe:
            raise RuntimeError(f"{key}: {pe} plan errors; timings are void")
        gbs = nbytes / (ms * 1e-3) / 1e9
        res[key] = {"us": round(ms * 1e3, 3), "algorithmic_bytes": nbytes, "GB/s": round(gbs, 1),
                    "frac": round(gbs / HBM_PEAK_GBS, 4), "tokens": host.tokens, "replicas": n_rep,
                    "calls_per_region": k, "step": what, "workload": OTHER_WORKLOADS[name]}
        del reps, be, meta, host
        torch.cuda.synchronize()
        torch.cuda.empty_cache()
    return res


def cpu_baseline(host, total_bytes: int, budget_s: float) -> dict:
    """The oracle's per-segment PyTorch path on the host cores (bf16, same inputs)."""
    import torch

    from oracle.lora_ref import TorchLoRABackend

    cores = cpu_cores()
    torch.set_num_threads(cores)
    be = TorchLoRABackend()
    be.set_kernel_input_metadata(host.meta)
    x, a, b = host.x, host.a_stacks[0], host.b_stacks[0]
    out = host.base.clone()
    for _ in range(3):
        be.apply_lora(x, a, b, out)
    times = []
    start = time.perf_counter()
    while time.perf_counter() - start < budget_s or len(times) < 20:
        t = time.perf_counter_ns()
        be.apply_lora(x, a, b, out)
        times.append(time.perf_counter_ns() - t)
        if len(times) >= 100000:
            break
    times.sort()
    med_s = times[len(times) // 2] * 1e-9
    return {
        "value": round(total_bytes / med_s / 1e9, 4),
        "unit": "GB/s",
        "us_per_step": med_s * 1e6,
        "cores": cores,
        "kind": "port",
        "cpu": cpu_model(),
        "sample": f"median of {len(times)} full 128-token shrink+expand calls (bf16, host tensors)",
    }


if __name__ == "__main__":
    sys.exit(main())
