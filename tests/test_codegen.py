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


_LABEL = re.compile(r"^(\.LBB\w+):")
_BRANCH = re.compile(r"^s_(c?branch)\w*\s+(\.LBB\w+)")


def _blocks(lines):
    """Split a function's lines into basic blocks: (label or None, [instructions])."""
    blocks, cur = [], [None, []]
    for line in lines:
        t = line.split(";")[0].strip()
        m = _LABEL.match(t)
        if m:
            if cur[0] is not None or cur[1]:
                blocks.append(cur)
            cur = [m.group(1), []]
            continue
        if not t or t.startswith("."):
            continue
        cur[1].append(t)
        if t.startswith(("s_branch", "s_cbranch", "s_endpgm", "s_setpc")):
            blocks.append(cur)
            cur = [None, []]
    if cur[0] is not None or cur[1]:
        blocks.append(cur)
    return blocks


def masked_mfmas(asm):
    """MFMAs that can run inside a divergent region: after an `s_and_saveexec_b64` and before the
    `s_or_b64 exec, exec, ...` that restores EXEC (the structured if/else shape the compiler emits
    for divergent branches). The region depth is propagated over the control-flow graph (blocks
    split at labels and branches, edges for branches and fall-through), so out-of-line blocks the
    compiler places after `s_endpgm` get the depth of the code that branches to them."""
    bad = []
    for name in re.findall(r"^(_Z\w+):", asm, re.M):
        start = asm.index(name + ":")
        end = asm.index(".Lfunc_end", start)
        blocks = _blocks(asm[start:end].split("\n")[1:])
        index = {lab: i for i, (lab, _) in enumerate(blocks) if lab}
        succ = []
        for i, (_, ins) in enumerate(blocks):
            last = ins[-1] if ins else ""
            m = _BRANCH.match(last)
            s = []
            if m:
                s.append(index[m.group(2)])
            if not last.startswith(("s_branch", "s_endpgm", "s_setpc")) and i + 1 < len(blocks):
                s.append(i + 1)
            succ.append(s)
        entry = [None] * len(blocks)
        entry[0] = 0
        work = [0]
        while work:
            i = work.pop()
            d = entry[i]
            for t in blocks[i][1]:
                if t.startswith("s_and_saveexec_b64"):
                    d += 1
                elif t.startswith("s_or_b64 exec, exec,"):
                    d = max(0, d - 1)
            for k in succ[i]:
                nd = min(d, 8)
                if entry[k] is None or nd > entry[k]:
                    entry[k] = nd
                    work.append(k)
        for i, (_, ins) in enumerate(blocks):
            if entry[i] is None:
                continue
            d = entry[i]
            for t in ins:
                if t.startswith("s_and_saveexec_b64"):
                    d += 1
                elif t.startswith("s_or_b64 exec, exec,"):
                    d = max(0, d - 1)
                if "v_mfma" in t and d > 0:
                    bad.append((name, t))
    return bad


def test_detector_flags_a_masked_mfma():
    asm = ("_Zk:\n s_and_saveexec_b64 s[2:3], vcc\n v_mfma_f32_32x32x8_f16 v[0:15], v[16:17], "
           "v[18:19], v[0:15]\n s_or_b64 exec, exec, s[2:3]\n.Lfunc_end0:\n")
    assert len(masked_mfmas(asm)) == 1
    assert masked_mfmas(asm.replace(" s_and_saveexec_b64 s[2:3], vcc\n", "")) == []


def test_detector_follows_out_of_line_blocks():
    # an MFMA block placed after s_endpgm: reached from uniform code it runs with the whole wave,
    # reached from inside a divergent region it does not
    uniform = ("_Zk:\n s_cbranch_vccz .LBB0_3\n s_and_saveexec_b64 s[2:3], vcc\n"
               " s_cbranch_execz .LBB0_2\n v_add_f32 v0, v1, v2\n.LBB0_2:\n"
               " s_or_b64 exec, exec, s[2:3]\n s_endpgm\n.LBB0_3:\n"
               " v_mfma_f32_32x32x8_f16 v[0:15], v[16:17], v[18:19], v[0:15]\n s_branch .LBB0_2\n"
               ".Lfunc_end0:\n")
    assert masked_mfmas(uniform) == []
    divergent = uniform.replace(" s_cbranch_vccz .LBB0_3\n s_and_saveexec_b64 s[2:3], vcc\n"
                                " s_cbranch_execz .LBB0_2\n",
                                " s_and_saveexec_b64 s[2:3], vcc\n s_cbranch_execz .LBB0_3\n")
    assert len(masked_mfmas(divergent)) == 1


@pytest.mark.parametrize("source", ["attn_fwd.hip", "attn_fwd_pp.hip"])
def test_main_loop_mfmas_run_with_the_whole_wave(source):
    asm = _assembly(os.path.join(PKG, "csrc", source))
    assert "v_mfma" in asm
    bad = masked_mfmas(asm)
    assert not bad, bad[:4]
