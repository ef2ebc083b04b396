"""Synthetic workloads and the bench.py contract on the CPU (no GPU needed)."""
from __future__ import annotations

import json
import os
import subprocess
import sys

import pytest
import torch

from qflash_amd.workloads import CONFIGS, HEADLINE, make_inputs, outlier_tensor, swin_attn_mask

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_config_table_matches_the_benchmark_definition():
    shapes = {k: (c.Z, c.H, c.N, c.D) for k, c in CONFIGS.items()}
    assert shapes == {"cfg1": (8, 3, 197, 64), "cfg2": (64, 6, 197, 64), "cfg3": (64, 12, 577, 64),
                      "cfg4": (4096, 3, 49, 32), "cfg5": (8, 16, 4096, 64)}
    assert HEADLINE == "cfg3"
    c3 = CONFIGS["cfg3"]
    assert c3.ops == 65_456_504_832                   # 4*Z*H*N^2*D
    assert c3.bytes_min == 4 * 64 * 12 * 577 * 64
    c4 = CONFIGS["cfg4"]
    assert c4.images * c4.windows == c4.Z and c4.window ** 2 == c4.N


@pytest.mark.parametrize("H,D,n_out", [(3, 64, 4), (6, 64, 8), (12, 64, 15), (3, 32, 2), (16, 64, 20)])
def test_outlier_channel_counts(H, D, n_out):
    g = torch.Generator().manual_seed(0)
    x = outlier_tensor(g, 2, H, 40, D)
    assert x.shape == (2, H, 40, D) and not x.is_contiguous()   # token-major view
    tok = x.permute(0, 2, 1, 3).reshape(2, 40, H * D)
    big = (tok.abs().amax(dim=(0, 1)) > 6.0).sum().item()      # x8 channels stand out of N(0,1)
    assert abs(big - n_out) <= 1
    assert round(0.02 * H * D) == n_out or (n_out == 1)


def test_swin_mask_regions_and_bias():
    g = torch.Generator().manual_seed(3)
    m = swin_attn_mask(g, 3, 7, images=2, windows=4)
    assert m.shape == (8, 3, 49, 49)
    shifted = m[2] - m[0]   # window 2 of image 0 carries the 4-region mask, window 0 not
    vals = set(torch.unique(shifted.round()).tolist())
    assert vals == {0.0, -100.0}
    # token (row 3, col 3) and (row 4, col 4) lie in different regions: split at 4
    assert shifted[0, 3 * 7 + 3, 4 * 7 + 4] == -100.0
    assert shifted[0, 3 * 7 + 3, 0] == 0.0
    # the relative-position bias is identical for every window and image
    assert torch.equal(m[0], m[1]) and torch.equal(m[0], m[4])
    assert m[0].abs().max() < 0.2


def test_make_inputs_is_seeded_and_typed():
    a = make_inputs(CONFIGS["cfg1"], 0)
    b = make_inputs(CONFIGS["cfg1"], 0)
    assert all(torch.equal(x, y) for x, y in zip(a[:3], b[:3])) and a[3] is None
    q2 = make_inputs(CONFIGS["cfg2"], 1)[0]
    assert q2.dtype == torch.float16 and q2.shape == (64, 6, 197, 64)


def _bench(*args):
    return subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), *args], capture_output=True, text=True,
                          cwd=ROOT, timeout=300)


def test_bench_refuses_more_than_one_gpu():
    r = _bench("--gpus", "2")
    assert r.returncode == 2 and "one GPU" in r.stderr and r.stdout == ""


def test_bench_without_gpu_fails_loudly():
    if torch.cuda.is_available():
        pytest.skip("a GPU is visible")
    r = _bench("--steps", "1", "--warmup", "0")
    assert r.returncode != 0 and "no GPU" in r.stderr


def test_bench_reads_the_committed_traffic_summary():
    sys.path.insert(0, ROOT)
    import bench
    t = bench.read_traffic()
    if not os.path.exists(bench.TRAFFIC_SUMMARY):
        assert t is None
    else:
        assert t is not None and t > 0
    json.dumps({"traffic": t})
