"""One-call segment shrink + expand (mlora_apply_segments) on the GPU.

The call must equal the two-call path (mlora_shrink into a caller `mid`,
then mlora_expand) element for element, whether the expand reads `mid` or
adds up the shrink's split sums itself (split K, 16-bit data, r_max <= 64,
segments not all long), and must match the oracle like every other path.
"""

import pytest
import torch

from multi_lora_amd import HipLoRABackend
from multi_lora_amd.kernels.lora_ops import Workspace, apply_segments
from multi_lora_amd.synthetic import make_meta
from oracle.lora_ref import apply_f64
from tests.gpu_helpers import assert_tol_f64
from tests.test_gpu_lora import run_hip

pytestmark = pytest.mark.gpu


def case(dev, lens, slots, ranks, in_dim, outs, r_max, dtype, seed):
    g = torch.Generator().manual_seed(seed)
    n_slots = len(ranks)
    x = torch.randn(sum(lens), in_dim, generator=g).to(dtype)
    As = [(torch.randn(n_slots, r_max, in_dim, generator=g) * in_dim ** -0.5).to(dtype) for _ in outs]
    Bs = [(torch.randn(n_slots, o, r_max, generator=g) * 0.05).to(dtype) for o in outs]
    base = torch.randn(sum(lens), sum(outs), generator=g).to(dtype)
    cols = [sum(outs[:i]) for i in range(len(outs))]
    scal = [0.5 + 0.25 * i for i in range(n_slots)]
    return x, As, Bs, base, cols, make_meta(lens, slots, ranks, scal, "cpu", dtype), scal


@pytest.mark.parametrize("name,lens,slots,ranks,in_dim,outs,r_max,dtype", [
    # mixed batch, split K: the expand adds the split sums itself
    ("mixed", [70] + [1] * 40 + [130], [0] + [i % 5 for i in range(40)] + [3], [16, 16, 0, 9, 16], 4096,
     [512, 128, 128], 16, torch.bfloat16),
    ("mixed_r64", [90, 1, 1, 3, 40, 1], [0, 1, 2, 0, 3, 1], [64, 33, 0, 48], 8192, [256, 256], 64, torch.float16),
    ("decode_split", [1] * 24 + [5], [i % 6 for i in range(25)], [16, 8, 16, 0, 16, 12], 8192, [384], 16,
     torch.bfloat16),
    # long segments (streamed expand reads mid), fp32 (no split sums), K not split
    ("long", [150, 200, 130], [0, 1, 0], [16, 32], 4096, [1024, 256], 32, torch.bfloat16),
    ("fp32", [20, 1, 33], [0, 1, 0], [8, 16], 1024, [256], 16, torch.float32),
    ("short_k", [30, 2, 17], [1, 0, 1], [16, 16], 64, [128], 16, torch.bfloat16),
])
def test_one_call_equals_two_calls(dev, name, lens, slots, ranks, in_dim, outs, r_max, dtype):
    x, As, Bs, base, cols, meta_cpu, scal = case(dev, lens, slots, ranks, in_dim, outs, r_max, dtype, len(name))
    meta = make_meta(lens, slots, ranks, scal, dev, dtype)
    xd, Ad, Bd = x.to(dev), [a.to(dev) for a in As], [b.to(dev) for b in Bs]
    _, two = run_hip(xd, Ad, Bd, meta, base.to(dev), cols)
    one = base.to(dev).clone()
    apply_segments(xd, Ad, Bd, meta, one, cols, workspace=Workspace())
    torch.cuda.synchronize()
    assert torch.equal(one.cpu(), two), f"{name}: one-call result differs from shrink + expand"
    assert_tol_f64(one.cpu(), apply_f64(x, As, Bs, meta_cpu, base, cols), name)


def test_backend_mixed_batch_uses_one_call_and_replays_in_a_graph(dev):
    """The backend's apply_lora_multi on a mixed batch, eager and under HIP
    graph replay (several replays with a metadata rewrite in between), equals
    the two-call path each time."""
    lens = [64] + [1] * 30
    slots = [0] + [i % 4 for i in range(30)]
    ranks = [16, 16, 16, 16]
    x, As, Bs, base, cols, _, scal = case(dev, lens, slots, ranks, 4096, [1024, 256], 16, torch.bfloat16, 5)
    meta = make_meta(lens, slots, ranks, scal, dev, torch.bfloat16)
    xd, Ad, Bd = x.to(dev), [a.to(dev) for a in As], [b.to(dev) for b in Bs]
    be = HipLoRABackend()
    be.set_kernel_input_metadata(meta)
    out = base.to(dev).clone()
    be.apply_lora_multi(xd, Ad, Bd, out, cols)
    _, want = run_hip(xd, Ad, Bd, meta, base.to(dev), cols)
    assert torch.equal(out.cpu(), want)
    out.copy_(base.to(dev))
    graph = torch.cuda.CUDAGraph()
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        be.apply_lora_multi(xd, Ad, Bd, out, cols)  # warm-up outside the graph
    torch.cuda.current_stream().wait_stream(stream)
    torch.cuda.synchronize()
    with torch.cuda.graph(graph):
        be.apply_lora_multi(xd, Ad, Bd, out, cols)
    for rep in range(3):
        out.copy_(base.to(dev))
        if rep == 2:  # rewrite the slots in place: the replay must follow
            meta.weight_indices.copy_(torch.tensor([1] + [(i + 1) % 4 for i in range(30)], dtype=torch.int32))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        _, want = run_hip(xd, Ad, Bd, meta, base.to(dev), cols)
        assert torch.equal(out.cpu(), want), f"replay {rep}"
