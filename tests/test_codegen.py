"""Code-generation invariants of the gfx950 main loop, checked on the CPU from hipcc's assembly.

Every MFMA must issue with the whole wave active. Its operands are spread over all 64 lanes (a
V^T row sits in one lane, a query column in two), so an MFMA under a partial EXEC mask silently
drops the inactive lanes' operand rows. The compiler is free to sink an MFMA whose result is only
used inside a divergent branch (the epilogue's `qrow < N` store) into that branch, which once
broke every ragged non-causal call; the kernel source prevents it, and this test keeps it so.
"""
import os
import re
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "sageattention-rdna4_amd")
sys.path.insert(0, PKG)


def _assembly(source):
    import build_lib
    if not os.path.exists(build_lib.HIPCC):
        pytest.skip("hipcc not available")
    flags = [f for f in build_lib.COMMON_FLAGS if f not in ("-fPIC",)]
    flags += build_lib.FILE_FLAGS.get(os.path.basename(source), [])
    res = subprocess.run([build_lib.HIPCC] + flags + ["--cuda-device-only", "-S", "-o", "-", source],
                         capture_output=True, text=True)
    assert res.returncode == 0, res.stderr[-2000:]
    return res.stdout


def masked_mfmas(asm):
    """MFMAs that sit between an `s_and_saveexec_b64` and the `s_or_b64 exec, exec, ...` that
    restores EXEC (the structured if/else shape the compiler emits for divergent branches)."""
    bad = []
    for name in re.findall(r"^(_Z\w+):", asm, re.M):
        start = asm.index(name + ":")
        end = asm.index(".Lfunc_end", start)
        depth = 0
        for line in asm[start:end].split("\n"):
            t = line.strip()
            if t.startswith("s_and_saveexec_b64"):
                depth += 1
            elif t.startswith("s_or_b64 exec, exec,"):
                depth = max(0, depth - 1)
            if "v_mfma" in t and depth > 0:
                bad.append((name, t))
    return bad


def test_detector_flags_a_masked_mfma():
    asm = ("_Zk:\n s_and_saveexec_b64 s[2:3], vcc\n v_mfma_f32_32x32x8_f16 v[0:15], v[16:17], "
           "v[18:19], v[0:15]\n s_or_b64 exec, exec, s[2:3]\n.Lfunc_end0:\n")
    assert len(masked_mfmas(asm)) == 1
    assert masked_mfmas(asm.replace(" s_and_saveexec_b64 s[2:3], vcc\n", "")) == []


def test_main_loop_mfmas_run_with_the_whole_wave():
    asm = _assembly(os.path.join(PKG, "csrc", "attn_fwd.hip"))
    assert "v_mfma" in asm
    bad = masked_mfmas(asm)
    assert not bad, bad[:4]
