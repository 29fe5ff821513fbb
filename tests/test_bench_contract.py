"""CPU checks of bench.py's contract and roofline accounting (no GPU).

* ``--gpus N`` with N > 1 exits with status 2 and says that this build
  measures one GPU (the driver's multi-GPU launch must not be mistaken for a
  result);
* ``roofline_of`` takes the MFMA roofline when a kernel's arithmetic
  intensity over its compulsory bytes is above the ridge point of the peaks
  (2.5 PFLOP/s over 8 TB/s = 312.5 FLOP/B) and the HBM one below it, with
  ``frac`` the achieved rate over that roofline's peak -- checked on the c3
  selection dK/dV at its measured launch time (the bench line's figures) and
  on the same kernel given 100x fewer FLOPs, which puts it below the ridge.
"""

import os
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_more_than_one_gpu_is_refused():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"], capture_output=True,
                       text=True, timeout=120, cwd=ROOT)
    assert r.returncode == 2
    assert "one GPU" in r.stderr
    assert r.stdout.strip() == ""


def _c3_sel_dkdv(flops, launch_s):
    import bench
    w = bench.WORKLOADS["c3"]
    pairs = 2066432   # (query, selected block) pairs of a c3 step with its seeded inputs (bench line)
    return bench.roofline_of(w, "dkdv[sel]", flops, launch_s, 2.6047e10, None, pairs)


def test_roofline_bound_follows_the_intensity():
    ent = _c3_sel_dkdv(2.7059e12, 5.2525e-3)
    # compulsory bytes: Q, dO and dQ rows of every query row (3 x 64 x 32768 x 128 x 2 B), the two row
    # statistics (2 x 64 x 32768 x 4 B), and per key K, V, K^T read in bf16 and dK, dV written in float32
    # (4 x 32768 keys x (3 x 128 x 2 + 2 x 128 x 4) B)
    comp = 3 * 64 * 32768 * 128 * 2 + 2 * 64 * 32768 * 4 + 4 * 32768 * (3 * 128 * 2 + 2 * 128 * 4)
    assert ent["compulsory_bytes"] == comp
    assert ent["ridge_flop_per_byte"] == pytest.approx(312.5)
    assert ent["bound"] == "mfma" and ent["unit"] == "TFLOP/s"
    assert ent["frac"] == pytest.approx(2.7059e12 / 5.2525e-3 / 2.5e15, abs=1e-4)
    assert ent["traffic_ratio"] == pytest.approx(2.6047e10 / comp, abs=0.01)
    low = _c3_sel_dkdv(2.7059e10, 5.2525e-3)   # 14.5 FLOP/B: below the ridge
    assert low["bound"] == "hbm" and low["unit"] == "GB/s"
    assert low["frac"] == pytest.approx(comp / 5.2525e-3 / 8e12, abs=1e-4)
