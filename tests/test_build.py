"""Device code built with the library's flags contains no packed-fp32 VALU
instructions and no scalar-cache writes (CPU only: compiles to gfx950
assembly and scans it)."""
import re
import subprocess

import pytest

from kunserve_amd import build as kb

FORBIDDEN = [
    r"\bv_pk_(add|mul|fma)_f32\b",                      # packed fp32
    r"\bs_(store|buffer_store|scratch_store)_\w+",      # scalar memory stores
    r"\bs_(buffer_)?atomic_\w+",                        # scalar atomics
    r"\bs_dcache_(wb|discard)\w*",                      # scalar cache write-back/discard
]


@pytest.mark.parametrize("src", kb.sources(), ids=lambda p: p.name)
def test_device_code_has_no_forbidden_instructions(src, tmp_path):
    out = tmp_path / (src.stem + ".s")
    cmd = [kb.hipcc(), *kb.flags_for(src), "--cuda-device-only", "-S", str(src), "-o", str(out)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    assert proc.returncode == 0, proc.stderr[-2000:]
    asm = out.read_text()
    assert "v_mfma" in asm or "mfma" not in src.read_text()
    for pat in FORBIDDEN:
        hits = sorted(set(m.group(0) for m in re.finditer(pat, asm)))
        assert not hits, f"{src.name}: {hits}"
