"""Host-side pieces of bench.py that run without a GPU: the amd-smi telemetry
parser (on a stand-in tool that prints amd-smi's `metric -p -c --json`
layout) and the one-GPU contract of --gpus."""
import os
import stat
import subprocess
import sys

import bench

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))

SMI_JSON = """{
  "gpu_data": [
    {"gpu": 0,
     "power": {"socket_power": {"value": 1210, "unit": "W"}, "gfx_voltage": "N/A"},
     "clock": {"gfx_0": {"clk": {"value": 1800, "unit": "MHz"}, "min_clk": {"value": 500, "unit": "MHz"}},
               "gfx_1": {"clk": {"value": 1700, "unit": "MHz"}},
               "gfx_2": {"clk": "N/A"},
               "mem_0": {"clk": {"value": 1900, "unit": "MHz"}},
               "fclk_0": {"clk": {"value": 2000, "unit": "MHz"}}}},
    {"gpu": 1,
     "power": {"socket_power": "N/A"},
     "clock": {}}
  ]
}"""


def test_smi_sample_parses_power_and_clocks(tmp_path):
    tool = tmp_path / "amd-smi"
    tool.write_text("#!/bin/sh\necho 'a warning line before the JSON'\ncat <<'EOF'\n" + SMI_JSON + "\nEOF\n")
    tool.chmod(tool.stat().st_mode | stat.S_IEXEC)
    got = bench._smi_sample(str(tool))
    assert len(got) == 2
    assert got[0] == {"power_w": 1210.0, "gfx_mhz": 1750.0, "mem_mhz": 1900.0}
    assert got[1] == {"power_w": None, "gfx_mhz": None, "mem_mhz": None}


def test_gpus_above_one_exit_with_a_message():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"],
                       capture_output=True, text=True, timeout=120)
    assert r.returncode == 2 and "one GPU" in r.stderr and r.stdout == ""


def test_telemetry_is_null_without_amd_smi(monkeypatch):
    monkeypatch.setattr(bench.shutil, "which", lambda name: None)
    monkeypatch.setattr(bench.os.path, "exists", lambda p: False)
    assert bench.telemetry(case=None, dev=None) is None
