"""Writes tests/golden/block_t16.npz: inputs (bf16 bit patterns) and float64
oracle outputs (stored as float32) of the block for B=1, T=16, C=256, H=1, N=64 with YaRN tables
(scale 4 over an original context of 8, temperature folded in).

The reference ships no golden vectors and cannot execute without a GPU, so
these are the oracle's own values (oracle/block.py through torch autograd in
float64). They lock the oracle against regressions and give the GPU path a
fixed known-answer case; they pin nothing about the reference beyond what
tests/test_oracle.py already pins.

Run from the repository root:  python tests/golden/make_block_fixture.py
"""
from __future__ import annotations

import sys
from pathlib import Path

import numpy as np
import torch

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))

from memory_efficient_attn_layer_amd.synthetic import Workload, make_inputs  # noqa: E402
from oracle import block as ob  # noqa: E402

FIXTURE = Path(__file__).resolve().with_name("block_t16.npz")
WORKLOAD = Workload(90, "golden B1 T16 C256 H1 N64 yarn4", 1, 16, 256, 1, 64, 4.0, 8)


def bits(t: torch.Tensor) -> np.ndarray:
    return t.contiguous().view(torch.int16).numpy().view(np.uint16)


def main() -> None:
    inp = make_inputs(WORKLOAD, seed=1234)
    g = ob.block_grads(inp, WORKLOAD.H, WORKLOAD.N, dtype=torch.float64)
    arrays = {f"in_{k}": bits(v) for k, v in inp.items()}
    arrays.update({f"out_{k}": v.numpy().astype(np.float32) for k, v in g.items()})
    arrays["shape"] = np.array([WORKLOAD.B, WORKLOAD.T, WORKLOAD.C, WORKLOAD.H, WORKLOAD.N])
    np.savez_compressed(FIXTURE, **arrays)
    print(f"wrote {FIXTURE} ({FIXTURE.stat().st_size} bytes)")


if __name__ == "__main__":
    main()
