"""GPU: the C ABI from a C99 host program (tests/c_host/silu_host.c, built by
__graft_entry__.build() with the C compiler): hipMalloc'd buffers, a HIP stream
of its own, kda_silu_f32, and the result checked on the host against
x / (1 + exp(-x)) in double (every element within 4e-6 relative), for a size with a scalar tail
and one that is a whole number of 16-byte vectors."""
import subprocess
from pathlib import Path

import pytest

pytestmark = pytest.mark.gpu
EXE = Path(__file__).resolve().parent / "c_host" / "silu_host"


@pytest.mark.parametrize("n", [(1 << 20) + 3, 2048 * 8192])
def test_c_host_silu(n):
    assert EXE.exists(), f"{EXE} is missing: run __graft_entry__.build()"
    r = subprocess.run([str(EXE), str(n)], capture_output=True, text=True, timeout=120)
    print(r.stdout, r.stderr, flush=True)
    assert r.returncode == 0, r.stdout + r.stderr
    assert f"silu n={n}: worst relative error" in r.stdout
