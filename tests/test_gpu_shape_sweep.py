"""Block parity over a seeded sweep of irregular shapes.

The named parity cases pin chosen edge cases; this sweep draws sequence
lengths (short, ragged, tile multiples and tile multiples +- 1), head widths
32 to 256, head counts, model widths, batch sizes, YaRN scaling and the table
gradients at random from a fixed seed, so the whole-tile and clamped tile
paths of the attention kernels, their untested middle loops and their
diagonal tiles meet many combinations. Each case runs the fused block forward
and backward on the GPU and checks it against the fp32 oracle to the block's
stated tolerances (tests/parity_util.py).
"""
from __future__ import annotations

import random

import pytest

from memory_efficient_attn_layer_amd.synthetic import Workload
from tests.parity_util import check_block

pytestmark = pytest.mark.gpu


def _cases(seed: int = 20261202, n: int = 16):
    rng = random.Random(seed)
    out = []
    for i in range(n):
        N = rng.choice([32, 64, 64, 64, 128, 256])
        H = rng.choice([2, 4, 6]) if N == 32 else rng.choice([1, 2, 3, 4])
        C = rng.choice([128, 256, 384, 512]) if N < 256 else 256
        T = rng.choice([rng.randint(1, 200), rng.randint(200, 1300), 64 * rng.randint(1, 16),
                        128 * rng.randint(1, 8) + rng.randint(-1, 1)])
        T = max(T, 1)
        B = rng.randint(1, 3)
        yarn = rng.choice([1.0, 1.0, 4.0])
        tg = rng.random() < 0.5
        out.append(pytest.param(B, T, C, H, N, yarn, tg, 1000 + i,
                                id=f"B{B}-T{T}-C{C}-H{H}-N{N}-s{yarn:g}-{'tg' if tg else 'plain'}"))
    return out


@pytest.mark.parametrize("B,T,C,H,N,yarn,table_grad,seed", _cases())
def test_block_matches_oracle_on_seeded_shapes(B, T, C, H, N, yarn, table_grad, seed):
    w = Workload(99, f"sweep B{B} T{T} C{C} H{H} N{N}", B, T, C, H, N, yarn, (T // 4 or 1) if yarn > 1 else None)
    check_block(w, seed=seed, table_grad=table_grad)
