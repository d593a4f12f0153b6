"""The rocprofv3 summaries under profiles/: every program their commands run is a
file of this repository, and the machine-readable HBM traffic block that bench.py
reports as `roofline.traffic` parses and covers the five graded configurations
with at least their algorithmic bytes."""
import re
import subprocess
from pathlib import Path

ROOT = Path(__file__).resolve().parents[1]
PROFILES = ROOT / "profiles"


def _repo_files():
    r = subprocess.run(["git", "ls-files"], cwd=ROOT, capture_output=True, text=True)
    return set(r.stdout.split()) if r.returncode == 0 else None


def test_profile_commands_run_repository_files():
    tracked = _repo_files()
    programs = set()
    for md in PROFILES.glob("*.md"):
        programs |= set(re.findall(r"python3 \$R/(\S+)", md.read_text()))
    assert programs, "no commands found in profiles/*.md"
    for prog in sorted(programs):
        assert (ROOT / prog).is_file(), prog
        if tracked is not None:
            assert prog in tracked, f"{prog} is not committed"


def test_traffic_block_parses_and_covers_the_graded_configs():
    import bench
    traffic = bench.measured_traffic()
    assert traffic is not None
    # algorithmic bytes per call (inputs read once, outputs written once)
    floor = {"silu": 8 * 2048 * 8192, "adamw": 28 * (1 << 27),
             "rmsnorm_matmul": 2 * (4096 * 4096 + 4096 * 11008 + 4096 * 11008),
             "swiglu": 2 * (2048 * 4096 + 3 * 4096 * 14336 + 2048 * 4096),
             "gqa": 2 * (4 * 4096 * 32 * 128 * 2 + 2 * 4 * 4096 * 8 * 128)}
    for name, least in floor.items():
        assert traffic[name] >= 0.99 * least, (name, traffic[name], least)
