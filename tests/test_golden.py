"""The committed golden case (tests/golden/block_t16.npz, written by
tests/golden/make_block_fixture.py): the oracle reproduces it on the CPU, and
the HIP block matches it on the GPU within the block tolerances."""
from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import block as ob
from tests.parity_util import assert_grad_close, assert_out_close, gpu_block

FIXTURE = Path(__file__).resolve().parent / "golden" / "block_t16.npz"


def _load():
    d = np.load(FIXTURE)
    B, T, C, H, N = (int(v) for v in d["shape"])
    inp = {k[3:]: torch.from_numpy(d[k].view(np.int16).copy()).view(torch.bfloat16) for k in d if k.startswith("in_")}
    out = {k[4:]: torch.from_numpy(d[k]) for k in d if k.startswith("out_")}
    return inp, out, H, N


def test_oracle_reproduces_golden():
    inp, out, H, N = _load()
    g = ob.block_grads(inp, H, N, dtype=torch.float64)
    for k, ref in out.items():
        got = g[k].float()
        err = float((got - ref).abs().max() / ref.abs().max().clamp_min(1e-30))
        assert err < 1e-5, (k, err)


@pytest.mark.gpu
def test_gpu_block_matches_golden():
    inp, out, H, N = _load()
    got = gpu_block(inp, H, N)
    assert_out_close("y", got["y"], out["y"])
    for k in ("dx", "dwq", "dwk", "dwv", "dwg", "dwo", "df1", "df2"):
        assert_grad_close(k, got[k], out[k])
