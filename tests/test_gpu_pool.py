"""Pool upload through mlora_pool_scatter (GPU), bit-exact against the same
pool on the CPU (torch copies), which test_host_pool.py pins to the oracle.

Follows the reference's scatter semantics (multi_lora/kernels/scatter_bank.py:17-68):
rank prefixes of A rows / B columns are written, nothing else changes.
"""

import ctypes
import random

import pytest
import torch

from multi_lora_amd import AdapterWeights, LoRAMemoryPool, _ffi

pytestmark = pytest.mark.gpu


def adapter(seed, rank, dims, dtype, missing=()):
    g = torch.Generator().manual_seed(seed)
    mods = {}
    for k, (i, o) in dims.items():
        if k in missing:
            continue
        mods[k] = ((torch.randn(rank, i, generator=g)).to(dtype), (torch.randn(o, rank, generator=g)).to(dtype))
    return AdapterWeights(rank=rank, scaling=1.0 / rank, modules=mods)


def store(dims, ranks, dtype, seed0=0, missing_every=0):
    out = {}
    for i, r in enumerate(ranks):
        miss = (list(dims)[1],) if missing_every and i % missing_every == 0 else ()
        out[f"a{i}"] = adapter(seed0 + i, r, dims, dtype, miss)
    return out


def run_sequence(device, dims, ranks, dtype, k_slots, max_rank, seed, steps=25):
    """The same random batch sequence on a fresh pool; returns the pool."""
    # Separate adapter objects per pool: a pool releases the host copies it packs.
    st = store(dims, ranks, dtype, missing_every=3)
    pool = LoRAMemoryPool(k_slots, max_rank, torch.device(device), dtype)
    # The first adapter defines every key (pools allocate keys on first sight).
    pool.ensure_buffers(adapter(999, max_rank, dims, dtype))
    rng = random.Random(seed)
    names = list(st) + [None]
    for _ in range(steps):
        batch = list(dict.fromkeys(rng.choice(names) for _ in range(rng.randint(1, k_slots))))
        pool.prepare_lora_batch(batch, weight_store=st)
    if device != "cpu":
        torch.cuda.synchronize()
    return pool


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("dims,ranks,max_rank", [
    ({"q": (256, 256), "v": (256, 64), "o": (512, 256)}, [8, 16, 4, 16, 8, 16, 4], 16),   # 16-byte path
    ({"q": (37, 53), "v": (41, 7)}, [3, 5, 1, 6, 2], 6),                                   # element path
])
def test_gpu_upload_matches_cpu_pool(dev, dims, ranks, max_rank, dtype):
    gpu = run_sequence("cuda", dims, ranks, dtype, 4, max_rank, seed=7)
    cpu = run_sequence("cpu", dims, ranks, dtype, 4, max_rank, seed=7)
    assert dict(gpu.name_to_slot) == dict(cpu.name_to_slot)
    for key in dims:
        ga, gb = gpu.get_module_buffers(key)
        ca, cb = cpu.get_module_buffers(key)
        assert torch.equal(ga.cpu(), ca), key
        assert torch.equal(gb.cpu(), cb), key


def test_scatter_entry_point_direct(dev):
    """One staged bank, hand-built table, odd offsets; a slot outside the pool is skipped."""
    rank, max_rank, in_dim, out_dim, k_slots = 3, 4, 10, 6, 3
    a = torch.full((k_slots, max_rank, in_dim), -1.0, device=dev)
    b = torch.full((k_slots, out_dim, max_rank), -1.0, device=dev)
    a_off, b_off = 5, 5 + rank * in_dim + 2
    total = b_off + out_dim * rank
    stage = torch.arange(2 * total, dtype=torch.float32, device=dev).view(2, total)
    slots = torch.tensor([1, 7], dtype=torch.int32, device=dev)  # second one outside the pool
    key = _ffi.PoolKey(a.data_ptr(), a.stride(0), a_off, b.data_ptr(), b.stride(0), b.stride(1), b_off, in_dim,
                       out_dim)
    table = torch.frombuffer(bytearray(bytes(key)), dtype=torch.uint8).to(dev)
    rc = _ffi.lib().mlora_pool_scatter(stage.data_ptr(), stage.stride(0), 2, slots.data_ptr(), table.data_ptr(), 1,
                                       rank, k_slots, max(rank * in_dim, out_dim * rank), _ffi.MLORA_F32,
                                       _ffi.stream_ptr(dev))
    _ffi.check(rc, "mlora_pool_scatter")
    torch.cuda.synchronize()
    want_a = torch.full((k_slots, max_rank, in_dim), -1.0)
    want_b = torch.full((k_slots, out_dim, max_rank), -1.0)
    row = stage[0].cpu()
    want_a[1, :rank] = row[a_off:a_off + rank * in_dim].view(rank, in_dim)
    want_b[1, :, :rank] = row[b_off:b_off + out_dim * rank].view(out_dim, rank)
    assert torch.equal(a.cpu(), want_a) and torch.equal(b.cpu(), want_b)
    assert ctypes.sizeof(_ffi.PoolKey) == 64


def test_upload_into_an_evicted_slot_waits_for_the_compute_reading_it(dev):
    """Compute enqueued after a batch was prepared reads that batch's slots;
    preparing the next batch evicts one of them, and its upload (on the copy
    stream) must not land before that compute has read the slot."""
    dims = {"q_proj": (256, 128)}
    st = {"a": adapter(1, 8, dims, torch.float32), "b": adapter(2, 8, dims, torch.float32)}
    a_rows = st["a"].modules["q_proj"][0].clone()
    b_rows = st["b"].modules["q_proj"][0].clone()
    pool = LoRAMemoryPool(1, 8, dev, torch.float32)
    pool.prepare_lora_batch(["a"], weight_store=st)
    slot_a = pool.get_module_buffers("q_proj")[0][0]
    busy = torch.randn(2048, 2048, device=dev)
    for _ in range(30):  # keeps the compute stream busy for a while before the read below
        busy = torch.tanh(busy @ busy * 1e-3)
    seen = slot_a.clone()  # reads the slot after the long work
    pool.prepare_lora_batch(["b"], weight_store=st)  # evicts "a": slot 0 gets b's rows
    torch.cuda.synchronize()
    assert torch.equal(seen.cpu(), a_rows)
    assert torch.equal(pool.get_module_buffers("q_proj")[0][0].cpu(), b_rows)
    assert pool.get_slot_id("b") == 0 and "a" not in pool.name_to_slot


def test_pipelined_serving_equals_serialised(dev):
    """A serving loop that never synchronises between steps (the next batch is
    prepared, evicting and uploading, while the previous forward may still
    run) gives, step for step, the logits of the same batches run with a
    synchronisation after every step.  Three slots for six adapters, so
    nearly every step evicts."""
    from multi_lora_amd import MultiLoRAManager
    from multi_lora_amd.decoder import Decoder, DecoderConfig

    cfg = DecoderConfig()
    proj = ("self_attn.q_proj", "self_attn.k_proj", "self_attn.v_proj", "self_attn.o_proj", "mlp.gate_proj",
            "mlp.up_proj", "mlp.down_proj")

    def run(sync_each_step):
        torch.manual_seed(0)
        model = Decoder(cfg).to(dev, torch.float32).eval()
        adapters = {}
        for j in range(6):
            g = torch.Generator().manual_seed(100 + j)
            mods = {}
            for layer in range(cfg.num_hidden_layers):
                for p in proj:
                    lin = model.get_submodule(f"layers.{layer}.{p}")
                    mods[f"layers.{layer}.{p}"] = (torch.randn(8, lin.in_features, generator=g) * 0.05,
                                                   torch.randn(lin.out_features, 8, generator=g) * 0.05)
            adapters[f"a{j}"] = AdapterWeights(rank=8, scaling=2.0, modules=mods)
        mgr = MultiLoRAManager.from_adapters(model, adapters, max_loras_per_batch=3, max_lora_rank=8)
        rng = random.Random(7)
        ids = torch.randint(0, cfg.vocab_size, (4, 6), generator=torch.Generator().manual_seed(3)).to(dev)
        outs = []
        with torch.inference_mode():
            for _ in range(12):
                names = [f"a{rng.randrange(6)}" for _ in range(4)]
                while len(set(names)) > 3:
                    names[rng.randrange(4)] = names[0]
                out = mgr.forward_with_lora(input_ids=ids, lora_names=names, seq_lens=[6] * 4, use_cache=False)
                outs.append(out.logits.clone())
                if sync_each_step:
                    torch.cuda.synchronize()
        torch.cuda.synchronize()
        return [o.cpu() for o in outs]

    piped, serial = run(False), run(True)
    for k, (p_, s_) in enumerate(zip(piped, serial)):
        assert torch.equal(p_, s_), f"step {k} differs"
