"""Write the golden fixtures of the 1024->1024 fp32 CPU configuration (test data).

Inputs are drawn by ``multi_lora_amd.synthetic.cpu_small`` (seeded); this
script stores their SHA-256 digests and, computed here with plain numpy in
float64 one row at a time (independently of ``oracle/``), the shrink result
``mid`` and a fixed sample of the expanded output plus its row and column
sums.  A second fixture holds a small RMSNorm case, also in float64 numpy.

    python tests/golden/make_golden.py      # rewrites tests/golden/*.npz
"""

from __future__ import annotations

import hashlib
import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parents[1]))

OUT_COL_STEP = 16  # sampled output columns: 0, 16, 32, ...


def digest(a: np.ndarray) -> str:
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def lora_fixture() -> dict:
    from multi_lora_amd import synthetic

    wl = synthetic.cpu_small()
    x = wl.x.numpy()
    a = wl.a_stacks[0].numpy()
    b = wl.b_stacks[0].numpy()
    base = wl.base.numpy()
    indptr = np.cumsum([0] + wl.seg_lens)
    r_max = a.shape[1]
    mid = np.zeros((x.shape[0], r_max))
    out = base.astype(np.float64).copy()
    for s, slot in enumerate(wl.seg_slots):
        r, sc = wl.slot_ranks[slot], wl.scalings[slot]
        for t in range(indptr[s], indptr[s + 1]):
            y = a[slot, :r].astype(np.float64) @ x[t].astype(np.float64)
            mid[t, :r] = y
            out[t] += sc * (b[slot, :, :r].astype(np.float64) @ y)
    return {
        "digest_x": digest(x), "digest_a": digest(a), "digest_b": digest(b), "digest_base": digest(base),
        "seg_lens": np.array(wl.seg_lens, np.int32), "seg_slots": np.array(wl.seg_slots, np.int32),
        "slot_ranks": np.array(wl.slot_ranks, np.int32), "scalings": np.array(wl.scalings, np.float64),
        "mid": mid,
        "out_sample": out[:, ::OUT_COL_STEP],
        "out_row_sums": out.sum(axis=1),
        "out_col_sums": out.sum(axis=0),
    }


def rmsnorm_fixture() -> dict:
    g = np.random.default_rng(7)
    x = g.standard_normal((6, 96)).astype(np.float32) * np.array([1, 3, 0.1, 10, 1, 0.5], np.float32)[:, None]
    w = (1.0 + 0.1 * g.standard_normal(96)).astype(np.float32)
    eps = 1e-5
    x64 = x.astype(np.float64)
    y = x64 / np.sqrt((x64 * x64).mean(axis=1, keepdims=True) + eps) * w.astype(np.float64)
    return {"x": x, "w": w, "eps": np.array(eps), "y": y}


def main() -> None:
    np.savez(HERE / "cpu_small_lora.npz", **lora_fixture())
    np.savez(HERE / "rmsnorm_small.npz", **rmsnorm_fixture())
    print("wrote", HERE / "cpu_small_lora.npz", HERE / "rmsnorm_small.npz")


if __name__ == "__main__":
    main()
