"""The C ABI's argument validation under AddressSanitizer and UBSan (host code).

`make -C kda-for-trainium_amd/csrc asan` builds the library with host-side
sanitizers (device code unchanged; `__graft_entry__.build()` builds it).  A
subprocess preloads the sanitizer runtime and calls every entry point declared
in include/kda.h with invalid arguments: null pointers, negative and oversized
(2^40) sizes, misaligned pointers, unknown operator ids, and once with every size
zero (an empty problem, which may succeed).  Each invalid call must return an
error status before any launch (no GPU is needed), and the process must end
without a sanitizer report.
"""
import glob
import os
import subprocess
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
ASAN_LIB = ROOT / "kda-for-trainium_amd" / "csrc" / "_build_asan" / "libkda_hostasan.so"


def _runtime():
    hits = sorted(glob.glob("/opt/rocm*/lib/llvm/lib/clang/*/lib/linux/libclang_rt.asan-x86_64.so"))
    return hits[-1] if hits else None


_DRIVER = r"""
import ctypes, sys
sys.path.insert(0, sys.argv[2])
from kda import _lib
L = ctypes.CDLL(sys.argv[1])
L.kda_last_error.restype = ctypes.c_char_p
bad = 0
def value(t, case):
    if t is _lib._p:
        return None if case != 3 else 1          # null, or a misaligned non-null address
    if t is _lib._i64:
        return {0: -1, 1: 0, 2: 1 << 40, 3: 8}[case]
    if t is _lib._int:
        return {0: -1, 1: 99, 2: 1 << 30, 3: 1}[case]
    return {0: -1.0, 1: 0.0, 2: float("nan"), 3: 1.0}[case]
for name, types in _lib.SIGNATURES.items():
    f = getattr(L, name)
    f.argtypes = types
    f.restype = _lib.RESTYPES.get(name, ctypes.c_int)
    for case in range(4):
        args = [value(t, case) for t in types]
        rc = f(*args)
        if case == 1:                              # all sizes 0: an empty problem may succeed
            continue
        ok = (rc == -1) if name == "kda_workspace_size" else (rc != 0)
        if name == "kda_workspace_size" and case == 3:
            ok = rc >= 0                           # op 1 at sizes 8: a real size
        if not ok:
            bad += 1
            print(f"{name} case {case}: returned {rc}", flush=True)
        elif name != "kda_workspace_size" and not L.kda_last_error():
            bad += 1
            print(f"{name} case {case}: error without a message", flush=True)
# Real shapes whose largest sizes multiply past 2^40 have positive workspace sizes,
# and their entry points refuse a missing workspace before any launch.
ws = L.kda_workspace_size
ws.argtypes = _lib.SIGNATURES["kda_workspace_size"]
ws.restype = ctypes.c_int64
for op, dims in ((_lib.OP_MATMUL_F32, (1, 8192, 8192, 28672, 0)),
                 (_lib.OP_RMSNORM_MATMUL_BF16, (1, 4096, 4096, 128256, 0)),
                 (_lib.OP_RMSNORM_MATMUL_BF16, (1, 4096, 4096, 65544, 0))):
    if ws(op, *dims) <= 0:
        bad += 1
        print(f"workspace size of op {op} at {dims}: {ws(op, *dims)}", flush=True)
fake = 1 << 20
for name, args in (("kda_matmul_f32", (fake, fake, fake, 8192, 8192, 28672, None, 0, None)),
                   ("kda_rmsnorm_matmul_bf16", (fake, fake, fake, fake, 4096, 4096, 128256, 1e-6,
                                                None, 0, None))):
    f = getattr(L, name)
    if f(*args) == 0:
        bad += 1
        print(f"{name} accepted a null workspace", flush=True)
print(f"checked {len(_lib.SIGNATURES)} entry points, {bad} problems", flush=True)
sys.exit(1 if bad else 0)
"""


@pytest.mark.skipif(not ASAN_LIB.exists(), reason="host-sanitizer build absent (make asan)")
def test_validation_paths_are_sanitizer_clean():
    rt = _runtime()
    if rt is None:
        pytest.skip("clang ASan runtime not found")
    env = dict(os.environ, LD_PRELOAD=rt, ASAN_OPTIONS="detect_leaks=0:abort_on_error=1",
               UBSAN_OPTIONS="halt_on_error=1:print_stacktrace=1", HIP_VISIBLE_DEVICES="")
    r = subprocess.run([sys.executable, "-c", _DRIVER, str(ASAN_LIB), str(ROOT / "kda-for-trainium_amd")],
                       env=env, capture_output=True, text=True, timeout=300)
    out = r.stdout + r.stderr
    assert "AddressSanitizer" not in out and "runtime error" not in out, out[-3000:]
    assert r.returncode == 0, out[-3000:]
    assert "0 problems" in r.stdout
