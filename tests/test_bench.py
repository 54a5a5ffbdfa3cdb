"""Host-side checks of bench.py (no GPU): the byte accounting behind
roofline.achieved for every workload, the tokens/s and roofline arithmetic,
the committed HBM-traffic figures it reports, and the refusal of more than
one GPU."""
import os
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)

import bench  # noqa: E402
from orthossm_amd.synthetic import CONFIGS  # noqa: E402


# Algorithmic bytes of one step, from the shapes: every input read once and
# every output written once (x, out; coefficients, damping, lambda; g; the
# EMA state in and out per launch; the gradient; the full path's momentum
# and LUT).
@pytest.mark.parametrize("name,want", [
    ("headline", 2 * 4 * 16384 * 512 * 4 + 4 * 8 * 8 * 64 * 4 + 2 * 8 * 4 + 2 * 4 * 512 * 4),
    ("streaming", 2 * 262144 * 512 * 4 + 8 * 8 * 64 * 4 + 2 * 8 * 4 + 16 * 2 * 512 * 4),
    ("dynamic", 2 * 8 * 32768 * 1024 * 4 + 8 * 8 * 8 * 128 * 4 + 2 * 8 * 4 + 8 * 32768 * 8 * 4 + 2 * 8 * 1024 * 4),
    ("bf16_ttt", 2 * 16 * 65536 * 512 * 2 + 2 * 16 * 8 * 8 * 64 * 4 + 2 * 8 * 4 + 2 * 16 * 512 * 4),
    ("backward", 4 * 4 * 16384 * 512 * 4 + 2 * 4 * 8 * 8 * 64 * 4 + 2 * 8 * 4 + 2 * 4 * 512 * 4),
    ("v10_full", 2 * 4 * 16384 * 512 * 4 + 4 * 4 * 8 * 8 * 64 * 4 + 2 * 8 * 4 + 8 * 256 * 4),
])
def test_algorithmic_bytes(name, want):
    assert bench.algorithmic_bytes(CONFIGS[name]) == want


def test_headline_bytes_match_the_profiles():
    # the figure the headline profile and roofline.algorithmic_bytes quote
    assert bench.algorithmic_bytes(CONFIGS["headline"]) == 268517440


def test_launch_figures():
    cfg = CONFIGS["streaming"]
    f = bench.launch_figures(cfg, 0.256)
    assert f["launches_per_step"] == 16
    assert f["kernel_ms_mean"] == pytest.approx(0.016)
    assert f["value"] == pytest.approx(cfg.B * cfg.S / 0.256e-3)
    assert f["achieved"] == pytest.approx(bench.algorithmic_bytes(cfg) / 16 / 0.016e-3 / 1e9)
    assert f["frac"] == pytest.approx(f["achieved"] / bench.HBM_PEAK_GBS)


@pytest.mark.parametrize("name", [n for n in CONFIGS if n != "cpu_ref"])
def test_traffic_figures_present(name):
    t = bench.measured_traffic(name)
    assert t is not None and t > 0.9 * bench.algorithmic_bytes(CONFIGS[name]) / (
        CONFIGS[name].S // CONFIGS[name].chunk if CONFIGS[name].chunk else 1)


def test_more_than_one_gpu_is_refused():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"], capture_output=True,
                       text=True, timeout=300)
    assert r.returncode == 2
    assert "one GPU" in r.stderr
