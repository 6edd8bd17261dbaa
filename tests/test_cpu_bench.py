"""CPU suite: bench.py's host-side helpers (no GPU): the amd-smi report
parser behind --sustain, the committed HBM-traffic figure it reads for the
roofline, and the refusal of more than one GPU."""
import os
import subprocess
import sys

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, REPO)

import bench  # noqa: E402

# the shape of `amd-smi metric -g 0 --power --clock` on an MI355X under load
# (GFX_2 .. GFX_6, the other video clocks and SOCCLK trimmed)
REPORT = """GPU: 0
    POWER:
        SOCKET_POWER: 1376 W
        GFX_VOLTAGE: N/A
        THROTTLE_STATUS: N/A
    CLOCK:
        GFX_0:
            CLK: 2043 MHz
            MIN_CLK: 500 MHz
            MAX_CLK: 2400 MHz
            CLK_LOCKED: DISABLED
            DEEP_SLEEP: DISABLED
        GFX_1:
            CLK: 1987 MHz
            MIN_CLK: 500 MHz
            MAX_CLK: 2400 MHz
            CLK_LOCKED: DISABLED
            DEEP_SLEEP: DISABLED
        GFX_7:
            CLK: 2017 MHz
            MIN_CLK: 500 MHz
            MAX_CLK: 2400 MHz
        MEM_0:
            CLK: 2000 MHz
            MIN_CLK: 2000 MHz
        VCLK_0:
            CLK: 59 MHz
"""


def test_parse_smi_report():
    s = bench.parse_smi(REPORT)
    assert s["socket_W"] == 1376.0
    # one clock per GFX entry, in order; MIN/MAX lines and other clocks are not taken
    assert s["gfx_MHz"] == [2043.0, 1987.0, 2017.0]
    assert s["mem_MHz"] == 2000.0


def test_parse_smi_without_power():
    assert bench.parse_smi(REPORT.replace("1376 W", "N/A")) is None
    assert bench.parse_smi("") is None


def test_parse_smi_without_memory_clock():
    s = bench.parse_smi(REPORT.split("        MEM_0:")[0])
    assert s["mem_MHz"] is None and len(s["gfx_MHz"]) == 3


def test_traffic_figure_is_committed():
    t = bench.read_traffic()
    assert t is not None and 8.0e8 < t < 1.0e9  # gate_up at config 3: about 894 MB per launch


def test_more_than_one_gpu_is_refused():
    r = subprocess.run([sys.executable, os.path.join(REPO, "bench.py"), "--gpus", "2"], capture_output=True,
                       text=True, timeout=120)
    assert r.returncode == 2
    assert "one GPU" in r.stderr
