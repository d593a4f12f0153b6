"""Host replay of every global access and of the K/V ring schedule of the bf16
GQA kernel (no GPU).

tests/gqa_replay.hip walks each workgroup, block, wave and lane of a
kda_gqa_fwd_bf16 launch through the geometry and schedule functions the kernel
itself computes its addresses with (kda-for-trainium_amd/csrc/attention_geom.h),
in the kernel's DMA schedule, and checks that q loads, K/V tile DMA sources (after
the clamp of rows past the sequence), LDS destinations and output stores stay
inside their buffers, that no 32-bit DMA offset wraps, that the persistent
(causal) schedule runs every block once and every output element is stored
exactly once, and that every read of the K/V ring finds the right block's tile,
landed, and is never overtaken by a DMA into its slot -- including the prefetch
of a block's first tiles by the previous block, and the next block's q rows that
the last iteration stages in LDS (sources inside q, no offset wrap, slots untouched
until read).
Shapes: the causal graded configuration (at the launcher's grid and at smaller
ones, so that workgroups run several blocks), ragged and partial-tile shapes (B2
S333 Hq8 Hkv2 among them), every heads-per-workgroup case, both output layouts,
and the largest kv-head count the launcher accepts, next to the first it refuses.
Four deliberately wrong schedules show that the ring checks fail when they should."""
import shutil
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
HIPCC = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"


@pytest.fixture(scope="module")
def replay(tmp_path_factory):
    if not Path(HIPCC).exists():
        pytest.skip("hipcc not found")
    exe = tmp_path_factory.mktemp("replay") / "gqa_replay"
    subprocess.run([HIPCC, "--offload-arch=gfx950", "--offload-host-only", "-O2", "-std=c++17",
                    f"-I{ROOT / 'kda-for-trainium_amd' / 'csrc'}", f"-I{ROOT / 'include'}",
                    str(ROOT / "tests" / "gqa_replay.hip"), "-o", str(exe)],
                   check=True, capture_output=True, text=True)
    return exe


def run(exe, b, s, hq, hkv, causal, layout="bshd", grid=0, mistake=0):
    r = subprocess.run([str(exe), str(b), str(s), str(hq), str(hkv), str(int(causal)), layout,
                        str(grid), str(mistake)],
                       capture_output=True, text=True, timeout=300)
    return r.returncode, r.stdout


@pytest.mark.parametrize("b,s,hq,hkv,causal,layout", [
    (4, 4096, 32, 8, True, "bshd"),     # the graded causal configuration
    (4, 4096, 32, 8, False, "bshd"),
    (1, 4096, 16, 8, False, "bhsd"),    # NKIBench gqa_full's layout
    (2, 333, 8, 2, True, "bshd"),       # partial last key tile, clamped DMA rows
    (2, 333, 8, 2, True, "bhsd"),
    (2, 333, 8, 2, False, "bshd"),
    (1, 1, 4, 4, True, "bshd"),
    (1, 64, 4, 1, True, "bshd"),
    (1, 200, 16, 2, True, "bshd"),      # 8 heads per workgroup
    (1, 517, 6, 2, True, "bshd"),       # G = 3: one head per workgroup, 3 workgroups per kv head
    (3, 96, 8, 1, False, "bhsd"),
    (1, 300, 64, 8, True, "bhsd"),
])
def test_every_access_in_bounds(replay, b, s, hq, hkv, causal, layout):
    rc, out = run(replay, b, s, hq, hkv, causal, layout)
    print(out)
    assert rc == 0 and out.startswith("ok "), out


@pytest.mark.parametrize("b,s,hq,hkv,grid", [
    (4, 4096, 32, 8, 1),      # one workgroup runs all 2048 blocks
    (4, 4096, 32, 8, 100),
    (2, 333, 8, 2, 1),        # blocks of 1 to 6 tiles: prefetch of fewer than 3 tiles
    (2, 333, 8, 2, 3),
    (1, 130, 4, 4, 2),        # 1-, 2- and 3-tile blocks
    (1, 517, 6, 2, 5),
])
def test_persistent_schedule_at_other_grids(replay, b, s, hq, hkv, grid):
    rc, out = run(replay, b, s, hq, hkv, True, grid=grid)
    print(out)
    assert rc == 0 and out.startswith("ok "), out


@pytest.mark.parametrize("mistake", [1, 2, 3, 4])
def test_ring_checks_catch_a_wrong_schedule(replay, mistake):
    """A prologue that skips tiles the previous block did not prefetch, a K DMA one
    slot early, a prologue that does not wait for its own DMAs, and q rows staged
    over the next block's prefetched K(2) are all reported as ring violations."""
    rc, out = run(replay, 2, 333, 8, 2, True, grid=3, mistake=mistake)
    assert rc == 1 and "VIOLATION ring" in out, out


def test_dma_offsets_at_the_kv_head_limit(replay):
    """Full 64-row tiles at Hkv = 266305 (the launcher's largest) do not wrap the
    32-bit DMA offsets; at 266306 (which it refuses) they do."""
    rc, out = run(replay, 1, 64, 266305, 266305, True)
    assert rc == 0 and out.startswith("ok "), out
    rc, out = run(replay, 1, 64, 266306, 266306, True)
    assert rc == 1 and "32-bit offset wraps" in out, out
