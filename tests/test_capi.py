"""The C ABI: libkda.so loads, exports every symbol include/kda.h declares, the
ctypes table matches the header, and argument validation fails cleanly.  CPU only:
the calls below are rejected before any HIP call is made."""
import ctypes
import re
import subprocess
from pathlib import Path

import pytest

from kda import _lib

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "kda.h"


def declared_functions():
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    return sorted(set(re.findall(r"^\s*(?:int|int64_t|const char\*)\s+(kda_\w+)\s*\(", text, flags=re.M)))


def test_header_declares_entry_points():
    names = declared_functions()
    assert "kda_version" in names and "kda_last_error" in names and len(names) >= 5


def test_library_exports_every_declared_symbol():
    out = subprocess.run(["nm", "-D", "--defined-only", str(_lib.LIB_PATH)],
                         capture_output=True, text=True, check=True).stdout
    exported = set(re.findall(r"\bT (kda_\w+)", out))
    missing = [n for n in declared_functions() if n not in exported]
    assert not missing, missing


def test_ctypes_table_matches_header():
    header = set(declared_functions()) - {"kda_version", "kda_last_error"}
    assert header == set(_lib.SIGNATURES), header ^ set(_lib.SIGNATURES)


def test_version_and_load():
    assert _lib.version() == 100
    assert _lib.lib().kda_last_error() == b""


def test_invalid_arguments_rejected_without_launch():
    with pytest.raises(ValueError, match="n=-1"):
        _lib.call("kda_silu_f32", None, None, -1, None)
    with pytest.raises(ValueError, match="even D"):
        _lib.call("kda_rope_f32", None, None, None, None, 3, 8, None)
    with pytest.raises(ValueError, match="step"):
        _lib.call("kda_adamw_f32", None, None, None, None, None, None, None, 8,
                  1e-3, 0.9, 0.999, 1e-8, 0.0, 0, None)
    with pytest.raises(ValueError, match="null pointer"):
        _lib.call("kda_silu_f32", None, None, 16, None)


def test_workspace_sizes_are_host_arithmetic():
    """Size queries touch no device: the documented closed forms, and -1 for an
    unknown op or a negative size."""
    q = lambda *a: _lib.query("kda_workspace_size", *a)
    m, k, f = 2048, 4096, 14336
    assert q(_lib.OP_SWIGLU_BF16, 1, m, k, f, 0) == 8 * m * k          # down-GEMM fp32 partials
    assert q(_lib.OP_RMSNORM_MATMUL_BF16, 1, 4096, 4096, 11008, 0) == 2 * 4096 * 4096 + 4 * 4096
    assert q(_lib.OP_SWIGLU_BF16, 1, m, k, f, 0) == q(_lib.OP_SWIGLU_BF16, 1, m, k, 2 * f, 0)
    assert q(_lib.OP_ADD_RMSNORM_MATMUL_BF16, 1, 4096, 4096, 11008, 0) == 2 * 4096 * 4096 + 4 * 4096
    assert q(_lib.OP_MATMUL_ADD_RMSNORM_BF16, 1, 4096, 4096, 11008, 0) == 4 * 4096 * (11008 // 32)
    assert q(_lib.OP_MATMUL_ADD_RMSNORM_BF16, 1, 7, 4096, 40, 0) == 4 * 7 * 2
    assert q(99, 1, 1, 1, 1, 0) == -1
    assert q(_lib.OP_MATMUL_F32, 1, -1, 32, 32, 0) == -1
    assert q(_lib.OP_MATMUL_F32, 1, 1 << 40, 1 << 40, 8, 0) == -1     # overflows int64: no size
    assert q(_lib.OP_BMM_SOFTMAX_F32, 1 << 30, 0, 64, 1 << 30, 0) == -1
    assert q(_lib.OP_GQA_F32, 1 << 40, 1 << 40, 8, 8, 0) == -1


def _pad(x):
    return (x + 255) // 256 * 256


def test_workspace_sizes_of_large_real_shapes():
    """Shapes whose three largest sizes multiply past 2^40 still have a workspace:
    each size term is checked on its own, so only a term that overflows int64 gives -1."""
    q = lambda *a: _lib.query("kda_workspace_size", *a)
    m, k, n = 8192, 8192, 28672                                        # fp32 split planes: 2*(2MK + 2KN)
    assert q(_lib.OP_MATMUL_F32, 1, m, k, n, 0) == 2 * _pad(2 * m * k) + 2 * 2 * k * n
    assert q(_lib.OP_RMSNORM_MATMUL_BF16, 1, 4096, 4096, 128256, 0) == 2 * 4096 * 4096 + 4 * 4096
    assert q(_lib.OP_RMSNORM_MATMUL_BF16, 1, 4096, 4096, 65544, 0) == 2 * 4096 * 4096 + 4 * 4096
    assert q(_lib.OP_SWIGLU_BF16, 1, 8192, 8192, 1 << 20, 0) == 8 * 8192 * 8192
    assert q(_lib.OP_MATMUL_ADD_RMSNORM_BF16, 1, 1 << 20, 4096, 1 << 20, 0) == 4 * (1 << 20) * (1 << 15)
    assert q(_lib.OP_GQA_F32, 64, 1 << 20, 32, 8, 0) > 4 * 2 * 64 * (1 << 20) * 8 * 128
    # near the int64 limit: 8 * M * K bytes of partials
    assert q(_lib.OP_SWIGLU_BF16, 1, 1, 1, 0, 0) == 8
    assert q(_lib.OP_SWIGLU_BF16, 1, 1 << 30, 1 << 29, 8, 0) == 1 << 62
    assert q(_lib.OP_SWIGLU_BF16, 1, 1 << 30, 1 << 30, 8, 0) == -1      # 2^63 bytes overflow


def test_missing_workspace_refused_at_large_shapes():
    """A null workspace is refused before any launch at sizes whose workspace is
    large (no GPU is touched: the calls fail in argument validation)."""
    fake = 1 << 20                                                      # aligned, never dereferenced
    m, k, n = 8192, 8192, 28672
    with pytest.raises(ValueError, match="workspace"):
        _lib.call("kda_matmul_f32", fake, fake, fake, m, k, n, None, 0, None)
    with pytest.raises(ValueError, match="workspace"):
        _lib.call("kda_matmul_f32", fake, fake, fake, m, k, n, fake, 1 << 20, None)
    with pytest.raises(ValueError, match="workspace"):
        _lib.call("kda_rmsnorm_matmul_bf16", fake, fake, fake, fake, 4096, 4096, 128256, 1e-6,
                  None, 0, None)


def test_gqa_bf16_rejects_kv_heads_beyond_32bit_dma_offsets():
    """A key tile's 64 rows are addressed with 32-bit per-lane byte offsets
    (row * Hkv*256 + chunk start, at most 63 * Hkv*256 + 240): Hkv = 266306 would
    wrap them, 266305 is the largest that fits (tests/test_gqa_addresses.py replays
    both).  Refused before any launch (the pointers are never dereferenced)."""
    fake = 1 << 20
    for hkv in (266306, 1 << 20):
        with pytest.raises(ValueError, match="32-bit DMA offsets"):
            _lib.call("kda_gqa_fwd_bf16", fake, fake, fake, fake, 1, 64, hkv, hkv, 128, 0.088, 1,
                      0, 0, 0, None)


def test_gqa_bf16_causal_rejects_query_heads_beyond_32bit_staging_offsets():
    """Causal launches stage a wave's next 32 q rows by DMA with 32-bit per-lane
    offsets (at most 31 * Hq*256 + 240 bytes): Hq = 541201 is refused before any
    launch (541200 is the largest that fits); the pointers are never dereferenced."""
    fake = 1 << 20
    with pytest.raises(ValueError, match="staged q rows"):
        _lib.call("kda_gqa_fwd_bf16", fake, fake, fake, fake, 1, 64, 541201, 1, 128, 0.088, 1,
                  0, 0, 0, None)


def test_header_is_strict_c99(tmp_path):
    """include/kda.h compiles as ISO C99 on its own, warnings as errors."""
    src = tmp_path / "use_header.c"
    src.write_text('#include "kda.h"\nint main(void) { return kda_version() == 100 ? 0 : 1; }\n')
    subprocess.run(["gcc", "-std=c99", "-pedantic", "-Wall", "-Wextra", "-Werror", "-fsyntax-only",
                    f"-I{ROOT / 'include'}", str(src)], check=True)


def test_c_host_program_validation(tmp_path):
    """The C99 host program (tests/c_host/silu_host.c), compiled with the C
    compiler and linked against libkda.so and the HIP runtime, gets the status codes
    and messages of failed validation from C; no GPU is touched."""
    import __graft_entry__ as entry
    exe = tmp_path / "silu_host"
    cmd = [str(exe) if a == str(entry.C_HOST / "silu_host") else a for a in entry.C_HOST_BUILD]
    cmd = [a.replace("$ORIGIN/../../kda-for-trainium_amd/kda", str(_lib.LIB_PATH.parent)) for a in cmd]
    subprocess.run(cmd, check=True)
    r = subprocess.run([str(exe), "--validate"], capture_output=True, text=True,
                       env={**__import__("os").environ, "HIP_VISIBLE_DEVICES": ""})
    assert r.returncode == 0, r.stdout + r.stderr
    assert "rc=1 msg='silu: n=-1 < 0'" in r.stdout and "rc=0 msg=''" in r.stdout


def test_ops_reject_cpu_tensors():
    import torch
    from kda import ops
    with pytest.raises(ValueError, match="GPU tensor"):
        ops.silu(torch.zeros(4))
