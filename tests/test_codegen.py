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


@pytest.mark.parametrize("source", ["attn_fwd.hip", "attn_fwd_pp.hip", "attn_fwd_pl.hip"])
def test_main_loop_mfmas_run_with_the_whole_wave(source):
    asm = _assembly(os.path.join(PKG, "csrc", source))
    assert "v_mfma" in asm
    bad = masked_mfmas(asm)
    assert not bad, bad[:4]


# ---------------------------------------------------------------------------------------------
# MFMA results read too early. The hardware does not hold back every read of an MFMA's result
# until the result is written: software has to leave a gap after the MFMA issues. The compiler
# pads by its own table (18-20 wait states after v_mfma_scale_f32_32x32x64_f8f6f4), and on gfx950
# that was measured short: in a main-loop variant whose last P.V MFMA was followed by register
# copies 18 wait states later, and in another whose spill code stored a fresh accumulator 20
# wait states after the MFMA, registers 14-15 of the tile came back stale, nondeterministically.
# The kernels therefore keep every non-MFMA read of an MFMA result at least the MFMA's full
# duration away: 64 cycles for the 32x32x64 fp8 MFMA (16 passes of 4), 32 for the 32x32x32 int8
# one. Distances are counted conservatively along every control-flow path: s_nop N is N+1 cycles,
# any non-MFMA instruction 1, and an MFMA the same wave issues after an earlier one the earlier
# one's duration less 8 (a wave's next MFMA issues only once the matrix core has taken the
# previous one's work: measured, four independent MFMAs followed by VALU work hold that work back
# by three MFMA durations).
# ---------------------------------------------------------------------------------------------
_REG = re.compile(r"\b([va])(?:(\d+)|\[(\d+):(\d+)\])")


def _regs(text):
    out = set()
    for m in _REG.finditer(text):
        bank = m.group(1)
        if m.group(2) is not None:
            out.add((bank, int(m.group(2))))
        else:
            out.update((bank, r) for r in range(int(m.group(3)), int(m.group(4)) + 1))
    return out


def _operands(ins):
    parts = ins.split(None, 1)
    if len(parts) < 2:
        return parts[0], []
    ops = []
    depth = 0
    cur = ""
    for ch in parts[1]:
        if ch == "," and depth == 0:
            ops.append(cur.strip())
            cur = ""
            continue
        depth += ch == "["
        depth -= ch == "]"
        cur += ch
    if cur.strip():
        ops.append(cur.strip())
    return parts[0], ops


def _mfma_cycles(mnem):
    m = re.search(r"(\d+)x(\d+)x(\d+)", mnem)
    if not m:
        return 32
    mm, nn, kk = (int(x) for x in m.groups())
    # matrix-core cycles at the gfx950 rates: 32x32x32 int8 and 32x32x64 fp8 take 32 and 64
    # cycles; the scale factor per shape is M*N*K / 1024 for 8-bit operands, M*N*K / 512 for 16-bit
    per = 512 if ("bf16" in mnem or "f16" in mnem) and "f8" not in mnem else 1024
    return max(16, mm * nn * kk // per)


def _sources_and_dests(mnem, ops):
    """(read registers, written registers) of one instruction (VGPR/AGPR only)."""
    if not ops:
        return set(), set()
    store_like = ("store" in mnem or mnem.startswith(("ds_write", "ds_add", "global_load_lds",
                                                      "buffer_load_dword_lds", "v_cmp", "v_cmpx",
                                                      "v_readlane", "v_readfirstlane",
                                                      "s_")))
    if mnem.startswith("v_permlane") and "swap" in mnem:
        both = _regs(ops[0]) | _regs(ops[1])
        return both, both
    if store_like:
        src = set()
        for o in ops:
            src |= _regs(o)
        return src, set()
    src = set()
    for o in ops[1:]:
        src |= _regs(o)
    return src, _regs(ops[0])


def early_mfma_reads(asm, min_f8=64, min_other=32):
    """(kernel, mfma, reader, cycles) for every read of an MFMA result by a non-MFMA instruction
    (or by an MFMA as its A/B operand) closer than the MFMA's full duration along some path."""
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
        parsed = [[_operands(t) for t in ins] for _, ins in blocks]
        for bi, ins in enumerate(parsed):
            for ii, (mnem, ops) in enumerate(ins):
                if not mnem.startswith("v_mfma"):
                    continue
                dst = _regs(ops[0])
                need = min_f8 if "f8f6f4" in mnem and "32x32x64" in mnem else min_other
                # walk forward: (block, index, cycles so far, registers still holding the result)
                seen = {}
                work = [(bi, ii + 1, 0, frozenset(dst), _mfma_cycles(mnem))]
                while work:
                    b, i, c, live, prev = work.pop()
                    while c < need and live:
                        if i >= len(parsed[b]):
                            for k in succ[b]:
                                key = (k, live)
                                if seen.get(key, 1 << 30) > c:
                                    seen[key] = c
                                    work.append((k, 0, c, live, prev))
                            break
                        mn, op = parsed[b][i]
                        src, wr = _sources_and_dests(mn, op)
                        if mn.startswith("v_mfma"):
                            a_b = set()
                            for o in op[1:3]:
                                a_b |= _regs(o)
                            if a_b & live:
                                bad.append((name, blocks[bi][1][ii], blocks[b][1][i], c))
                                break
                            if len(op) > 3 and _regs(op[3]) & live and _regs(op[0]) == _regs(op[3]):
                                live = live - _regs(op[0])     # accumulation chain: superseded
                            c += max(8, prev - 8)
                            prev = _mfma_cycles(mn)
                        else:
                            if src & live:
                                bad.append((name, blocks[bi][1][ii], blocks[b][1][i], c))
                                break
                            live = live - wr
                            m = re.match(r"s_nop\s+(\d+)", blocks[b][1][i])
                            c += int(m.group(1)) + 1 if m else 1
                        i += 1
    return bad


def test_detector_flags_an_early_read():
    asm = ("_Zk:\n v_mfma_scale_f32_32x32x64_f8f6f4 v[0:15], v[16:23], v[24:31], 0, v1, v1\n"
           " s_nop 15\n s_nop 3\n v_add_f32 v40, v15, v15\n s_endpgm\n.Lfunc_end0:\n")
    assert len(early_mfma_reads(asm)) == 1
    fenced = asm.replace(" s_nop 3\n", " s_nop 15\n s_nop 15\n s_nop 15\n")
    assert early_mfma_reads(fenced) == []
    # reached only through a loop back-edge after enough other work
    looped = ("_Zk:\n.LBB0_1:\n v_add_f32 v40, v15, v15\n"
              " v_mfma_i32_32x32x32_i8 v[0:15], v[16:19], v[20:23], 0\n"
              + " v_mov_b32 v41, v42\n" * 40 + " s_cbranch_scc1 .LBB0_1\n s_endpgm\n.Lfunc_end0:\n")
    assert early_mfma_reads(looped) == []
    assert len(early_mfma_reads(looped.replace(" v_mov_b32 v41, v42\n" * 40, ""))) == 1
    # an overwrite ends the result's life; an accumulation chain supersedes it
    over = asm.replace(" v_add_f32 v40, v15, v15\n", " v_mov_b32 v15, 0\n v_add_f32 v40, v15, v15\n")
    assert early_mfma_reads(over) == []


@pytest.mark.parametrize("source", ["attn_fwd.hip", "attn_fwd_pp.hip", "attn_fwd_pl.hip"])
def test_mfma_results_are_read_after_the_mfma_completes(source):
    asm = _assembly(os.path.join(PKG, "csrc", source))
    bad = early_mfma_reads(asm)
    assert not bad, bad[:6]


def _kernel_resources(asm):
    """(kernel name, VGPRs, spilled VGPRs, scratch bytes per lane) for every kernel in hipcc's
    metadata."""
    out = []
    for m in re.finditer(r"^\s+- \.agpr_count:.*?(?=^\s+- \.agpr_count:|^\.end_amdgpu_metadata)",
                         asm, re.S | re.M):
        block = m.group(0)
        name = re.search(r"^\s+\.name:\s+(\S+)", block, re.M).group(1)
        vg = int(re.search(r"^\s+\.vgpr_count:\s+(\d+)", block, re.M).group(1))
        vs = int(re.search(r"^\s+\.vgpr_spill_count:\s+(\d+)", block, re.M).group(1))
        ps = int(re.search(r"^\s+\.private_segment_fixed_size:\s+(\d+)", block, re.M).group(1))
        out.append((name, vg, vs, ps))
    return out


@pytest.mark.parametrize("source", ["attn_fwd.hip", "attn_fwd_pp.hip", "attn_fwd_pl.hip",
                                    "prologue.hip"])
def test_no_kernel_spills_registers(source):
    # the register budget is a gate: no instantiation of any kernel spills VGPRs or uses scratch
    # memory at all (SGPRs parked in VGPR lanes, v_writelane, cost no memory traffic and are
    # allowed)
    res = _kernel_resources(_assembly(os.path.join(PKG, "csrc", source)))
    assert res, "no kernel metadata found"
    spilled = [r for r in res if r[2] or r[3]]
    assert not spilled, spilled
    assert max(r[1] for r in res) <= 256


def test_resource_parser_sees_a_spill():
    meta = ("  - .agpr_count:     0\n    .name:           _Zk\n    .private_segment_fixed_size: 12\n"
            "    .vgpr_count:     168\n    .vgpr_spill_count: 3\n.end_amdgpu_metadata\n")
    assert _kernel_resources(meta) == [("_Zk", 168, 3, 12)]
