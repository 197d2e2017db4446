"""Code-generation invariants of the gfx950 main loop, checked on the CPU from hipcc's assembly.

Every MFMA must issue with the whole wave active. Its operands are spread over all 64 lanes (a
V^T row sits in one lane, a query column in two), so an MFMA under a partial EXEC mask silently
drops the inactive lanes' operand rows. The compiler is free to sink an MFMA whose result is only
used inside a divergent branch (the epilogue's `qrow < N` store) into that branch, which once
broke every ragged non-causal call; the kernel source prevents it, and this test keeps it so.
"""
import functools
import os
import re
import shutil
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "sageattention-rdna4_amd")
sys.path.insert(0, PKG)


@functools.lru_cache(maxsize=None)
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


# ---------------------------------------------------------------------------------------------
# Barrier liveness. A workgroup whose waves execute different numbers of `s_barrier` hangs the
# GPU. In the ping-pong kernel each wave computes up to its own causal diagonal (w_end differs by
# wave) and then only stages, keeping 2 barriers per 64-key block, so the totals agree only by
# construction. `asm_sim` interprets each kernel's assembly per wave for concrete arguments
# (scalar control flow exactly; data-dependent branches both ways, which must agree on their
# barrier count) and counts the barriers each wave executes; every wave must execute the same
# number, on shapes that cover causal and non-causal grids, ragged tails, grouped K/V heads, a
# key length of its own and the optional outputs.
# ---------------------------------------------------------------------------------------------
import asm_sim  # noqa: E402

_FAKE = 0x20000000                     # device addresses the interpreter never dereferences


def _fake(i):
    return _FAKE + (i << 24)


def _cdiv(a, b):
    return (a + b - 1) // b


def _template(name):
    """(bf16, qk_int8, causal, head_dim, key split) of a main-loop kernel's mangled name."""
    m = re.search(r"I(DF16_|DF16b)Lb([01])ELb([01])E(?:Li(\d+)E)?(?:Lb([01])E)?", name)
    return m.group(1) == "DF16b", m.group(2) == "1", m.group(3) == "1", \
        int(m.group(4)) if m.group(4) else 128, m.group(5) == "1"


def _attn_args(family, N, Nk, H, H_kv, D, lse=False, vmean=False, split=False):
    """Kernel arguments in signature order, as the launchers in attn_fwd*.hip form them (B = 1,
    contiguous HND), and the number of workgroups."""
    bm = 256 if family == "pp" else 64 if split else 128
    num_qt = _cdiv(N, bm)
    total = num_qt * H
    strides = [H * N * D, N * D, D] * 2
    tail = [H, H_kv, H // H_kv, N, Nk, _cdiv(Nk, 64) * 64, num_qt, total // 8 * 8, 0.088,
            _fake(9) if lse else 0, _fake(10) if lse else 0, _fake(11) if vmean else 0]
    if family == "pl":
        plane = 2 * _cdiv(Nk, 64) * 64
        head = [_fake(0), _fake(1), _fake(2), plane, 128, _fake(2) + 256, plane, 128, 1.0,
                _fake(3), _fake(4), _fake(5)]
    else:
        head = [_fake(0), _fake(1), _fake(2), _fake(3), _fake(4), _fake(5)]
    return head + strides + tail, total


# (N, N_kv, H, H_kv, lse, vmean): causal calls use N == N_kv
_CAUSAL_SHAPES = [(1, 1, 1, 1, False, False), (200, 200, 2, 1, True, False),
                  (777, 777, 1, 1, False, True)]
_NONCAUSAL_SHAPES = [(1, 1, 1, 1, False, False), (300, 777, 4, 2, True, True),
                     (777, 65, 1, 1, False, False), (513, 512, 1, 1, False, False),
                     (100, 129, 1, 1, False, False), (100, 200, 1, 1, True, False)]


def _pick(total):
    ids = sorted({0, 1, total // 2, total - 2, total - 1} & set(range(total)))
    return ids


def _main_loop_cases(asm):
    for name in asm_sim.kernel_functions(asm):
        fam = ("pp" if "attn_fwd_pp_kernel" in name else "pl" if "attn_fwd_pl_kernel" in name
               else "q" if "attn_fwd_kernel" in name else None)
        if fam is None:
            continue
        _, _, causal, D, split = _template(name)
        for N, Nk, H, H_kv, lse, vm in (_CAUSAL_SHAPES if causal else _NONCAUSAL_SHAPES):
            vals, total = _attn_args(fam, N, Nk, H, H_kv, D, lse, vm, split)
            for wg in _pick(total):
                yield name, vals, wg, (N, Nk, H, H_kv, wg)


@pytest.mark.parametrize("source", ["attn_fwd.hip", "attn_fwd_pp.hip", "attn_fwd_pl.hip"])
def test_every_wave_of_a_main_loop_block_executes_the_same_barriers(source):
    asm = _assembly(os.path.join(PKG, "csrc", source))
    seen = split = 0
    for name, vals, wg, case in _main_loop_cases(asm):
        counts, _ = asm_sim.barrier_counts(asm, name, vals, wg)
        assert len(set(counts)) == 1 and counts[0] > 0, (name, case, counts)
        seen += 1
        split += _template(name)[4]
    assert seen >= 20
    # the key-split forms (head_dim 64, three dtype forms), key groups of 0 to 7 blocks each
    assert split >= (60 if source == "attn_fwd_pl.hip" else 0)


def _prologue_geom(BH, N, N_pad, step):
    # prologue_geom (prologue.hip): one round of resident blocks on 256 CUs, 3 stats blocks and
    # 8 quant blocks per CU
    per = lambda slots: slots // BH if BH < slots else 1  # noqa: E731
    nc = _cdiv(N, 64) * 64
    r1 = _cdiv(_cdiv(nc, per(256 * 3)), step) * step
    r2 = _cdiv(_cdiv(N_pad, per(256 * 8)), 64) * 64
    return r1, _cdiv(nc, r1), r2, _cdiv(N_pad, r2)


def test_every_wave_of_a_prologue_block_executes_the_same_barriers():
    asm = _assembly(os.path.join(PKG, "csrc", "prologue.hip"))
    seen = 0
    for name in asm_sim.kernel_functions(asm):
        m = re.search(r"(kv_stats_kernel|k_quant_kernel)I(DF16_|DF16b)L(b|i)([0-9])ELi(\d+)E",
                      name)
        if not m:
            continue
        D = int(m.group(5))
        step = 8 * (256 // (D // 8))
        for BH, N, extra_pad in ((2, 777, 0), (1, 5000, 128), (800, 64, 0)):
            n_pad = _cdiv(N, 64) * 64 + extra_pad
            r1, c1, r2, c2 = _prologue_geom(BH, N, n_pad, step)
            st = [BH * N * D, N * D, D]
            if m.group(1) == "kv_stats_kernel":
                vals = [_fake(0), _fake(1), _fake(2), _fake(3), _fake(4), _fake(5), _fake(6),
                        _fake(7), BH, N, n_pad, r1, c1] + st + st + [1]
                total = c1 * BH
            else:
                vals = [_fake(0), _fake(1), _fake(2), _fake(3), _fake(4), _fake(5), _fake(6),
                        _fake(7), _fake(8), BH, N, n_pad, r2, c2, c1] + st + [1, 1]
                total = c2 * BH
            for wg in _pick(total):
                counts, _ = asm_sim.barrier_counts(asm, name, vals, wg)
                assert len(set(counts)) == 1 and counts[0] > 0, (name, BH, N, wg, counts)
                seen += 1
    assert seen >= 50


def _mutated_assembly(tmp_path, source, old, new, compile_source=None):
    """hipcc -S of `compile_source` (default `source`) in a copy of csrc/ in which `old` is
    replaced by `new` in `source`."""
    import build_lib
    src = tmp_path / "csrc"
    shutil.copytree(os.path.join(PKG, "csrc"), src)
    inc = tmp_path / "include"
    shutil.copytree(os.path.join(ROOT, "include"), inc)
    path = src / source
    text = path.read_text()
    assert old in text
    path.write_text(text.replace(old, new))
    target = compile_source or source
    flags = [f for f in build_lib.COMMON_FLAGS if f not in ("-fPIC",)]
    flags += build_lib.FILE_FLAGS.get(target, [])
    res = subprocess.run([build_lib.HIPCC] + flags + ["--cuda-device-only", "-S", "-o", "-",
                                                      str(src / target)],
                         capture_output=True, text=True)
    assert res.returncode == 0, res.stderr[-2000:]
    return res.stdout


def _pp_causal_int8(asm):
    return next(n for n in asm_sim.kernel_functions(asm)
                if "attn_fwd_pp_kernel" in n and _template(n)[1:3] == (True, True))


def test_barrier_check_flags_a_staging_tail_that_starts_one_block_late(tmp_path):
    # Planted in a copy of the ping-pong: the staging-only blocks after a wave's diagonal start
    # one block late, so the waves whose diagonal ends early execute two barriers fewer.
    asm = _mutated_assembly(tmp_path, "attn_fwd_pp.hip", "for (j = w_end; j < j_end; ++j) {",
                            "for (j = w_end + 1; j < j_end; ++j) {")
    name = _pp_causal_int8(asm)
    # the last q-tile (rows 768..1023, run first): the waves' diagonals end at blocks 13 .. 16
    vals, total = _attn_args("pp", 1024, 1024, 1, 1, 128)
    counts, _ = asm_sim.barrier_counts(asm, name, vals, 0)
    assert len(set(counts)) > 1, counts
    good = _assembly(os.path.join(PKG, "csrc", "attn_fwd_pp.hip"))
    counts, _ = asm_sim.barrier_counts(good, _pp_causal_int8(good), vals, 0)
    assert len(set(counts)) == 1, counts


def test_barrier_check_flags_a_barrier_under_a_data_dependent_branch(tmp_path):
    # Planted: a barrier inside the accumulator rescale, which a wave runs only when some lane's
    # running maximum moved -- a data-dependent count.
    asm = _mutated_assembly(tmp_path, "attn_common.h",
                            "  if (__any(alpha != 1.0f)) {\n",
                            "  if (__any(alpha != 1.0f)) {\n    __syncthreads();\n",
                            compile_source="attn_fwd_pp.hip")
    with pytest.raises(asm_sim.DataDependentBarrier):
        for name, vals, wg, _ in _main_loop_cases(asm):
            asm_sim.barrier_counts(asm, name, vals, wg)


def test_interpreter_follows_scalar_control_flow():
    # a counted loop whose trip count comes from a kernel argument, a wave-dependent branch and a
    # data-dependent one (a global load) around barrier-free code
    asm = """_Zk:
 s_load_dword s4, s[0:1], 0x0
 v_lshrrev_b32_e32 v1, 6, v0
 v_readfirstlane_b32 s5, v1
 s_waitcnt lgkmcnt(0)
.LBB0_1:
 s_barrier
 s_add_i32 s4, s4, -1
 s_cmp_lg_u32 s4, 0
 s_cbranch_scc1 .LBB0_1
 s_cmp_eq_u32 s5, 1
 s_cbranch_scc1 .LBB0_3
 global_load_dword v2, v1, s[0:1]
 s_waitcnt vmcnt(0)
 v_cmp_eq_u32_e32 vcc, 0, v2
 s_cbranch_vccnz .LBB0_3
 v_add_u32_e32 v3, v2, v2
.LBB0_3:
 s_barrier
 s_endpgm
.Lfunc_end0:
"""
    meta = """
  - .agpr_count:     0
    .args:
      - .offset:         0
        .size:           4
        .value_kind:     by_value
    .max_flat_workgroup_size: 128
    .name:           _Zk
.amdhsa_kernel _Zk
    .amdhsa_user_sgpr_count 2
    .amdhsa_user_sgpr_kernarg_segment_ptr 1
    .amdhsa_system_sgpr_workgroup_id_x 1
.end_amdhsa_kernel
"""
    counts, _ = asm_sim.barrier_counts(asm + meta, "_Zk", [5], 0)
    assert counts == [6, 6]
    bad = asm.replace(" v_add_u32_e32 v3, v2, v2\n", " s_barrier\n")
    with pytest.raises(asm_sim.DataDependentBarrier):
        asm_sim.barrier_counts(bad + meta, "_Zk", [5], 0)
    skewed = asm.replace(".LBB0_3:\n s_barrier\n", ".LBB0_3:\n")\
        .replace(" s_cbranch_scc1 .LBB0_3\n global_load", " s_cbranch_scc1 .LBB0_4\n global_load")\
        .replace(" s_endpgm\n", " s_endpgm\n.LBB0_4:\n s_barrier\n s_endpgm\n")
    counts, _ = asm_sim.barrier_counts(skewed + meta, "_Zk", [5], 0)
    assert counts == [5, 6]
    # s_bitset1 / s_bitset0 set and clear one bit of the destination, keeping the rest: the trip
    # count becomes 5 | (1 << 3) = 13, then 13 & ~(1 << 0) = 12, and the final barrier makes 13
    bits = asm.replace(" s_waitcnt lgkmcnt(0)\n", " s_waitcnt lgkmcnt(0)\n s_bitset1_b32 s4, 3\n"
                       " s_mov_b32 s6, 0\n s_bitset0_b32 s4, s6\n")
    counts, _ = asm_sim.barrier_counts(bits + meta, "_Zk", [5], 0)
    assert counts == [13, 13]


# ---------------------------------------------------------------------------------------------
# The hot loop's instruction budget (the reference's method: count instructions per matrix
# instruction in the hot loop against a budget). The interpreter counts the vector ALU
# instructions each wave executes, along the cheaper side of every data-dependent branch (the
# accumulator rescale runs only when a row maximum moves), so the difference between two key
# lengths is the per-block cost of the steady state. Per 64-key block of one wave (32 queries):
# 12 MFMAs with int8 Q.K (8 for S^T, 4 for P.V), 8 with e4m3 Q.K; the VALU count is held to the
# committed budget, so a change that should cut it and does not is caught before it is timed.
# ---------------------------------------------------------------------------------------------
# qk_int8 -> VALU per wave and 64-key block, in all and in the softmax phase (the longer of the
# two phases between barriers: the ping-pong's critical path)
PP_VALU_BUDGET = {True: 244, False: 212}
PP_SOFTMAX_PHASE_BUDGET = {True: 228, False: 212}


def pp_block_costs(asm, name):
    """Per wave: (VALU, MFMA) per 64-key block of the ping-pong in its steady state (one q-tile,
    non-causal, 8 more key blocks), and the VALU of its longest steady-state phase."""
    res, phase = [], []
    for nk in (640, 1152):
        vals, _ = _attn_args("pp", 256, nk, 1, 1, 128)
        _, states = asm_sim.barrier_counts(asm, name, vals, 0)
        res.append([(s.valu, s.mfma) for s in states])
        phase = [max(v for v, _ in s.phases()[4:-4]) for s in states]
    per_block = [((b[0] - a[0]) / 8.0, (b[1] - a[1]) / 8.0) for a, b in zip(*res)]
    return per_block, phase


@pytest.mark.parametrize("qk_int8", [True, False])
def test_ping_pong_instruction_budget(qk_int8):
    asm = _assembly(os.path.join(PKG, "csrc", "attn_fwd_pp.hip"))
    name = next(n for n in asm_sim.kernel_functions(asm)
                if "attn_fwd_pp_kernel" in n and _template(n)[1:3] == (qk_int8, False)
                and not _template(n)[0])
    costs, phase = pp_block_costs(asm, name)
    assert all(m == (12 if qk_int8 else 8) for _, m in costs), costs
    worst = max(v for v, _ in costs)
    assert worst <= PP_VALU_BUDGET[qk_int8], (worst, costs)
    assert max(phase) <= PP_SOFTMAX_PHASE_BUDGET[qk_int8], phase
