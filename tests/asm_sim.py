"""A control-flow interpreter of gfx950 kernel assembly (hipcc -S), for barrier-count checks on the
CPU. Test infrastructure only.

A workgroup hangs when its waves do not all execute the same number of `s_barrier` instructions.
`barrier_counts` runs one kernel's assembly once per wave of a workgroup, for concrete kernel
arguments and a concrete workgroup id, and returns how many barriers each wave executed:

* scalar instructions (SALU, scalar branches, `s_load` from the kernel-argument segment) and the
  vector instructions that feed control flow (lane-id arithmetic, compares, `v_readfirstlane`,
  SGPR spills to VGPR lanes, the float-reciprocal integer division idiom) are interpreted
  exactly, lane by lane;
* every other value -- loads from memory or LDS, MFMA results, DPP, anything not implemented --
  is UNKNOWN, and so is everything computed from it;
* a branch on an UNKNOWN condition (data-dependent, e.g. "skip the rescale when no lane needs
  it") is followed both ways up to its immediate post-dominator; both paths must execute the
  same number of barriers (else `DataDependentBarrier`), and their states are merged (values
  that differ become UNKNOWN);
* a wave that does not reach `s_endpgm` within the step budget raises `NoTermination`.

The model decides nothing about memory or arithmetic results, only which blocks each wave runs.
"""
import re
import struct

import numpy as np

LANES = 64
M32 = 0xFFFFFFFF
FULL = (1 << LANES) - 1
KERNARG = 0x10000000          # the modelled address of the kernel-argument segment


class DataDependentBarrier(Exception):
    pass


class NoTermination(Exception):
    pass


class Unsupported(Exception):
    pass


# ----------------------------------------------------------------------------------- parsing
_LABEL = re.compile(r"^(\.LBB\w+):")
_SPECIAL = {"vcc": (106, 2), "vcc_lo": (106, 1), "vcc_hi": (107, 1), "exec": (126, 2),
            "exec_lo": (126, 1), "exec_hi": (127, 1), "m0": (124, 1), "flat_scratch": (102, 2)}


def _f2u(x):
    return struct.unpack("<I", struct.pack("<f", float(x)))[0]


class Op:
    """One operand: kind 's' (SGPR base, count), 'v' (VGPRs), 'a' (AGPRs), 'imm', 'scc' or
    'other' (not modelled); `mod` marks a neg/abs modifier."""
    __slots__ = ("kind", "base", "n", "val", "mod")

    def __init__(self, kind, base=0, n=1, val=None, mod=False):
        self.kind, self.base, self.n, self.val, self.mod = kind, base, n, val, mod


def parse_operand(t):
    t = t.strip()
    mod = False
    if t.startswith(("|", "-|", "neg(", "abs(", "-v", "-s")):
        mod = True
        t = t.replace("neg(", "").replace("abs(", "").rstrip(")").strip("|-").strip("|")
    m = re.match(r"^([sva])(\d+)$", t)
    if m:
        return Op(m.group(1), int(m.group(2)), 1, mod=mod)
    m = re.match(r"^([sva])\[(\d+):(\d+)\]$", t)
    if m:
        a, b = int(m.group(2)), int(m.group(3))
        return Op(m.group(1), a, b - a + 1, mod=mod)
    if t in _SPECIAL:
        base, n = _SPECIAL[t]
        return Op("s", base, n, mod=mod)
    if t == "scc":
        return Op("scc")
    if re.match(r"^(-?0x[0-9a-fA-F]+|-?\d+)$", t):
        return Op("imm", val=int(t, 0) & 0xFFFFFFFFFFFFFFFF, mod=mod)
    if re.match(r"^-?\d+\.\d+$", t):
        return Op("imm", val=_f2u(float(t)), mod=mod)
    return Op("other", mod=mod)


def split_operands(text):
    ops, depth, cur = [], 0, ""
    for ch in text:
        if ch == "," and depth == 0:
            ops.append(cur.strip())
            cur = ""
            continue
        depth += ch in "[("
        depth -= ch in "])"
        cur += ch
    if cur.strip():
        ops.append(cur.strip())
    return ops


class Ins:
    __slots__ = ("text", "mn", "ops", "extra", "pops")

    def __init__(self, text):
        self.text = text
        parts = text.split(None, 1)
        self.mn = parts[0]
        ops, extra = [], []
        for tk in split_operands(parts[1] if len(parts) > 1 else ""):
            sub = tk.split()
            if len(sub) > 1 and not tk.startswith(("|", "-|")):
                ops.append(sub[0])
                extra += sub[1:]
            else:
                ops.append(tk)
        self.ops, self.extra = ops, extra
        self.pops = [parse_operand(o) for o in ops]


def kernel_functions(asm):
    return re.findall(r"^(_Z\w+):", asm, re.M)


def kernel_blocks(asm, name):
    """[(label or None, [Ins])] of one function, split at labels and after branches."""
    start = asm.index(name + ":")
    end = asm.index(".Lfunc_end", start)
    blocks, cur = [], [None, []]
    for line in asm[start:end].split("\n")[1:]:
        t = line.split(";")[0].strip()
        m = _LABEL.match(t)
        if m:
            if cur[0] is not None or cur[1]:
                blocks.append(cur)
            cur = [m.group(1), []]
            continue
        if not t or t.startswith("."):
            continue
        cur[1].append(Ins(t))
        if t.startswith(("s_branch", "s_cbranch", "s_endpgm", "s_setpc")):
            blocks.append(cur)
            cur = [None, []]
    if cur[0] is not None or cur[1]:
        blocks.append(cur)
    return blocks


def kernel_meta(asm, name):
    """(argument list [(offset, size)], workgroup size, index of the workgroup-id SGPR)."""
    i = asm.index(".name:           " + name + "\n")
    j = asm.rindex("- .agpr_count:", 0, i)
    args = [(int(o), int(s)) for o, s in
            re.findall(r"\.offset:\s+(\d+)\s*\n\s*\.size:\s+(\d+)", asm[j:i])]
    nxt = asm.find("- .agpr_count:", i)
    tail = asm[i:nxt if nxt > 0 else len(asm)]
    wg = int(re.search(r"\.max_flat_workgroup_size:\s+(\d+)", asm[j:i] + tail).group(1))
    k = asm.index(".amdhsa_kernel " + name + "\n")
    hdr = asm[k:asm.index(".end_amdhsa_kernel", k)]

    def flag(key):
        m = re.search(r"\.amdhsa_%s\s+(\d+)" % key, hdr)
        return int(m.group(1)) if m else 0
    if flag("user_sgpr_dispatch_ptr") or flag("user_sgpr_queue_ptr") or \
            flag("user_sgpr_kernarg_preload_length") or flag("user_sgpr_dispatch_id") or \
            flag("user_sgpr_private_segment_buffer"):
        raise Unsupported("user SGPR layout")
    if not flag("user_sgpr_kernarg_segment_ptr") or not flag("system_sgpr_workgroup_id_x"):
        raise Unsupported("no kernarg pointer or workgroup id")
    if flag("system_sgpr_workgroup_id_y") or flag("system_sgpr_workgroup_id_z") or \
            flag("system_vgpr_workitem_id") != 0:
        raise Unsupported("multi-dimensional ids")
    return args, wg, flag("user_sgpr_count")


# ----------------------------------------------------------------------------------- the CFG
def build_cfg(blocks):
    index = {lab: i for i, (lab, _) in enumerate(blocks) if lab}
    succ = []
    for i, (_, ins) in enumerate(blocks):
        last = ins[-1].text if ins else ""
        s = []
        m = re.match(r"^s_(c?branch)\w*\s+(\.LBB\w+)", last)
        if m:
            s.append(index[m.group(2)])
        if not last.startswith(("s_branch", "s_endpgm", "s_setpc")) and i + 1 < len(blocks):
            s.append(i + 1)
        succ.append(s)
    return index, succ


def post_dominators(succ):
    """Immediate post-dominator of each block; len(succ) stands for the exit."""
    n = len(succ)
    EXIT = n
    pdom = [set(range(n + 1)) for _ in range(n)] + [{EXIT}]
    changed = True
    while changed:
        changed = False
        for i in range(n - 1, -1, -1):
            ss = succ[i] if succ[i] else [EXIT]
            new = set.intersection(*(pdom[s] for s in ss)) | {i}
            if new != pdom[i]:
                pdom[i] = new
                changed = True
    ipdom = []
    for i in range(n):
        strict = pdom[i] - {i}
        ipdom.append(next(c for c in strict if pdom[c] == strict))
    return ipdom


# ----------------------------------------------------------------------------------- state
class State:
    """SGPRs: index -> 32-bit int (absent = UNKNOWN). VGPRs: index -> (values uint32[64],
    known bool[64]). SCC: 0, 1 or None. `valu`, `mfma`: vector ALU instructions other than MFMAs,
    and MFMAs, executed so far (along the cheaper side of every data-dependent branch)."""
    __slots__ = ("s", "v", "scc", "barriers", "valu", "mfma", "ebound", "marks")

    def __init__(self):
        self.s, self.v, self.scc, self.barriers, self.valu, self.mfma = {}, {}, None, 0, 0, 0
        self.ebound = FULL      # a known superset of EXEC (EXEC itself may be UNKNOWN)
        self.marks = []         # (valu, mfma) at each barrier

    def copy(self):
        c = State()
        c.s = dict(self.s)
        c.v = {k: (a.copy(), k_.copy()) for k, (a, k_) in self.v.items()}
        c.scc, c.barriers, c.valu, c.mfma = self.scc, self.barriers, self.valu, self.mfma
        c.ebound, c.marks = self.ebound, list(self.marks)
        return c

    def phases(self):
        """(VALU, MFMA) executed between consecutive barriers."""
        return [(b[0] - a[0], b[1] - a[1]) for a, b in zip(self.marks, self.marks[1:])]


def merge(a, b):
    """What holds after either of two paths: equal values kept, the rest UNKNOWN."""
    m = State()
    m.s = {k: x for k, x in a.s.items() if b.s.get(k) == x}
    for k, (va, ka) in a.v.items():
        if k in b.v:
            vb, kb = b.v[k]
            known = ka & kb & (va == vb)
            if known.any():
                m.v[k] = (va.copy(), known)
    m.scc = a.scc if a.scc == b.scc else None
    m.barriers = a.barriers
    m.valu, m.mfma = min(a.valu, b.valu), min(a.mfma, b.mfma)
    m.ebound = a.ebound | b.ebound
    m.marks = list(a.marks)
    return m


_NOKNOW = np.zeros(LANES, dtype=bool)


_BITS = {}


def _bits(mask):
    b = _BITS.get(mask)
    if b is None:
        b = np.array([(mask >> i) & 1 for i in range(LANES)], dtype=bool)
        if len(_BITS) < 4096:
            _BITS[mask] = b
    return b


def _mask(bits):
    return sum(1 << i for i in range(LANES) if bits[i])


# ----------------------------------------------------------------------------------- the machine
class Machine:
    def __init__(self, asm, name, max_steps=3_000_000):
        self.name = name
        self.blocks = kernel_blocks(asm, name)
        self.index, self.succ = build_cfg(self.blocks)
        self.ipdom = post_dominators(self.succ)
        self.args, self.wg, self.wgid_sgpr = kernel_meta(asm, name)
        self.max_steps = max_steps
        self.steps = 0
        self.kernarg = b""
        self.forks = 0

    # -- scalar operands
    def sget(self, st, op, width=None):
        n = width or op.n
        if op.kind == "imm":
            v = op.val
            if n == 1:
                return v & M32
            if v >> 32 == 0 and (v & 0x80000000):
                v |= 0xFFFFFFFF00000000     # 32-bit constants sign-extend for 64-bit operands
            return v & 0xFFFFFFFFFFFFFFFF
        if op.kind == "scc":
            return st.scc
        if op.kind != "s" or op.mod:
            return None
        out = 0
        for i in range(n):
            x = st.s.get(op.base + i)
            if x is None:
                return None
            out |= x << (32 * i)
        return out

    def sset(self, st, op, val, width=None):
        if op.kind != "s":
            return
        for i in range(width or op.n):
            if val is None:
                st.s.pop(op.base + i, None)
            else:
                st.s[op.base + i] = (val >> (32 * i)) & M32
        ex = self.exec_mask(st)
        if ex is not None:
            st.ebound = ex

    def exec_mask(self, st):
        lo, hi = st.s.get(126), st.s.get(127)
        return None if lo is None or hi is None else lo | (hi << 32)

    # -- vector operands: (values uint32[64], known bool[64])
    def vget(self, st, op, dword=0):
        if op.mod:
            return None
        if op.kind == "v":
            return st.v.get(op.base + dword)
        if op.kind == "s":
            x = st.s.get(op.base + dword)
            if x is None:
                return None
            return np.full(LANES, x, dtype=np.uint32), np.ones(LANES, dtype=bool)
        if op.kind == "imm":
            x = (op.val >> (32 * dword)) & M32 if dword else op.val & M32
            return np.full(LANES, x, dtype=np.uint32), np.ones(LANES, dtype=bool)
        return None

    def vset(self, st, op, vk, dword=0):
        """Write lanes active in EXEC (all lanes UNKNOWN when EXEC is)."""
        if op.kind != "v":
            return
        r = op.base + dword
        ex = self.exec_mask(st)
        if ex is None or (vk is None and ex == FULL):
            st.v.pop(r, None)
            return
        old = st.v.get(r)
        act = _bits(ex)
        if old is None:
            old = (np.zeros(LANES, dtype=np.uint32), _NOKNOW.copy())
        vals, known = old[0].copy(), old[1].copy()
        if vk is None:
            known[act] = False
        else:
            vals[act] = vk[0].astype(np.uint32)[act]
            known[act] = vk[1][act]
        if known.any():
            st.v[r] = (vals, known)
        else:
            st.v.pop(r, None)

    # -- run
    def run_wave(self, kernarg, wg_id, wave):
        self.kernarg = kernarg
        st = State()
        st.s[0], st.s[1] = KERNARG, 0
        st.s[self.wgid_sgpr] = wg_id & M32
        st.s[126], st.s[127] = M32, M32
        st.v[0] = (np.arange(LANES, dtype=np.uint32) + np.uint32(64 * wave),
                   np.ones(LANES, dtype=bool))
        self.steps = 0
        self.last = self.run(st, 0, None)
        return self.last.barriers

    def run(self, st, b, stop):
        """Run from the start of block b until block `stop` is reached (None: s_endpgm)."""
        while True:
            if b == stop:
                return st
            if b >= len(self.blocks):
                raise NoTermination("ran past the last block")
            nxt = self.step_block(st, b)
            if nxt == "end":
                if stop is not None:
                    raise DataDependentBarrier("a path ends inside a forked region")
                return st
            if isinstance(nxt, tuple):           # a branch on an UNKNOWN condition
                _, t, f = nxt
                join = self.ipdom[b]
                stop_j = None if join >= len(self.blocks) else join
                self.forks += 1
                sa = self.run(st.copy(), t, stop_j)
                sb = self.run(st.copy(), f, stop_j)
                if sa.barriers != sb.barriers:
                    raise DataDependentBarrier(
                        "%s: the branch `%s` (block %d) leads to %d or %d barriers"
                        % (self.name[:40], self.blocks[b][1][-1].text, b, sa.barriers,
                           sb.barriers))
                st = merge(sa, sb)
                if stop_j is None:
                    return st
                b = join
                continue
            b = nxt

    def step_block(self, st, b):
        for I in self.blocks[b][1]:
            self.steps += 1
            if self.steps > self.max_steps:
                raise NoTermination("%s: step budget exhausted" % self.name[:40])
            mn = I.mn
            if mn == "s_endpgm":
                return "end"
            if mn == "s_branch":
                return self.index[I.ops[0]]
            if mn.startswith("s_cbranch"):
                cond = self.branch_cond(st, mn)
                tgt = self.index[I.ops[0]]
                if cond is None:
                    return ("fork", tgt, b + 1)
                return tgt if cond else b + 1
            if mn.startswith(("s_setpc", "s_swappc", "s_call")):
                raise Unsupported(I.text)
            if mn == "s_barrier":
                st.barriers += 1
                st.marks.append((st.valu, st.mfma))
                continue
            if mn.startswith("s_"):
                self.salu(st, I)
            elif mn.startswith("v_"):
                if mn.startswith(("v_mfma", "v_smfmac")):
                    st.mfma += 1
                else:
                    st.valu += 1
                self.valu(st, I)
            elif mn.startswith(("global_load", "buffer_load", "flat_load", "ds_read", "ds_load",
                                "scratch_load", "global_atomic", "buffer_atomic", "flat_atomic",
                                "ds_bpermute", "ds_permute", "ds_swizzle", "ds_add_rtn",
                                "ds_max_rtn", "ds_min_rtn")):
                if "_lds" not in mn and I.pops:
                    for d in range(I.pops[0].n):
                        self.vset(st, I.pops[0], None, d)
            # stores, LDS writes and DMA to LDS have no register results
        return b + 1

    def branch_cond(self, st, mn):
        if mn in ("s_cbranch_scc0", "s_cbranch_scc1"):
            return None if st.scc is None else (st.scc == int(mn.endswith("1")))
        if mn in ("s_cbranch_vccz", "s_cbranch_vccnz"):
            lo, hi = st.s.get(106), st.s.get(107)
            if lo is None or hi is None:
                return None
            vcc = lo | (hi << 32)
            return (vcc == 0) if mn.endswith("vccz") else (vcc != 0)
        if mn in ("s_cbranch_execz", "s_cbranch_execnz"):
            ex = self.exec_mask(st)
            return None if ex is None else ((ex == 0) if mn.endswith("execz") else (ex != 0))
        raise Unsupported(mn)

    # -- scalar ALU
    def salu(self, st, I):
        mn, ops = I.mn, I.pops
        if mn.startswith(("s_waitcnt", "s_nop", "s_setprio", "s_sleep", "s_icache",
                          "s_sendmsg", "s_setreg", "s_ttrace", "s_set_gpr_idx")):
            return
        if mn.startswith(("s_load_dword", "s_buffer_load")):
            return self.s_load(st, ops)
        if mn in ("s_memtime", "s_memrealtime", "s_getreg_b32", "s_getpc_b64"):
            return self.sset(st, ops[0], None)
        m = re.match(r"s_(and|or|xor|andn2|orn2)_saveexec_b64$", mn)
        if m:
            src, ex = self.sget(st, ops[1], 2), self.exec_mask(st)
            self.sset(st, ops[0], ex, 2)
            if src is None or ex is None:
                # EXEC becomes UNKNOWN; for an and-form it stays within the EXEC it had
                if m.group(1) != "and":
                    st.ebound = FULL
                st.s.pop(126, None)
                st.s.pop(127, None)
                st.scc = None
                return
            new = {"and": src & ex, "or": src | ex, "xor": src ^ ex, "andn2": src & ~ex,
                   "orn2": src | (~ex & FULL)}[m.group(1)] & FULL
            st.s[126], st.s[127] = new & M32, new >> 32
            st.scc = int(new != 0)
            return
        w64 = mn.endswith(("_b64", "_u64", "_i64")) and not mn.startswith(("s_bcnt1_i32",
                                                                            "s_ff1_i32"))
        n, bits = (2, 64) if w64 else (1, 32)
        mask = (1 << bits) - 1

        def sx(x, b=bits):
            return x - (1 << b) if (x >> (b - 1)) & 1 else x

        if mn in ("s_mov_b32", "s_mov_b64", "s_movk_i32"):
            v = self.sget(st, ops[1], n)
            if mn == "s_movk_i32" and v is not None:
                v = sx(v & 0xFFFF, 16) & M32
            return self.sset(st, ops[0], v, n)
        if mn in ("s_cmov_b32", "s_cmov_b64"):
            if st.scc is None:
                v = self.sget(st, ops[1], n)
                if v != self.sget(st, ops[0], n):
                    self.sset(st, ops[0], None, n)
            elif st.scc:
                self.sset(st, ops[0], self.sget(st, ops[1], n), n)
            return
        if mn in ("s_cselect_b32", "s_cselect_b64"):
            a, b = self.sget(st, ops[1], n), self.sget(st, ops[2], n)
            if st.scc is None:
                return self.sset(st, ops[0], a if a == b else None, n)
            return self.sset(st, ops[0], a if st.scc else b, n)
        m = re.match(r"s_cmpk?_(eq|lg|gt|ge|lt|le)_(i32|u32|u64)$", mn)
        if m:
            wide = m.group(2) == "u64"
            a = self.sget(st, ops[0], 2 if wide else 1)
            if mn.startswith("s_cmpk"):
                b = ops[1].val & 0xFFFF
                if m.group(2) == "i32":
                    b = sx(b, 16)
            else:
                b = self.sget(st, ops[1], 2 if wide else 1)
            if a is None or b is None:
                st.scc = None
                return
            if m.group(2) == "i32":
                a = sx(a, 32)
                b = sx(b & M32, 32) if not mn.startswith("s_cmpk") else b
            st.scc = int({"eq": a == b, "lg": a != b, "gt": a > b, "ge": a >= b, "lt": a < b,
                          "le": a <= b}[m.group(1)])
            return
        if mn in ("s_bitcmp1_b32", "s_bitcmp0_b32"):
            a, b = self.sget(st, ops[0], 1), self.sget(st, ops[1], 1)
            st.scc = None if a is None or b is None else \
                int(((a >> (b & 31)) & 1) == (1 if mn == "s_bitcmp1_b32" else 0))
            return
        if mn in ("s_bitset0_b32", "s_bitset1_b32"):
            # D[S0 & 31] = 0 / 1, the rest of D kept (no SCC)
            a, b = self.sget(st, ops[0], 1), self.sget(st, ops[1], 1)
            if a is None or b is None:
                return self.sset(st, ops[0], None)
            bit = 1 << (b & 31)
            return self.sset(st, ops[0], (a | bit) if mn == "s_bitset1_b32" else (a & ~bit & M32))
        if mn in ("s_addk_i32", "s_mulk_i32"):
            a, k = self.sget(st, ops[0], 1), sx(ops[1].val & 0xFFFF, 16)
            if a is None:
                self.sset(st, ops[0], None)
                if mn == "s_addk_i32":
                    st.scc = None
                return
            r = sx(a, 32) + k if mn == "s_addk_i32" else sx(a, 32) * k
            if mn == "s_addk_i32":
                st.scc = int(r < -(1 << 31) or r >= (1 << 31))
            return self.sset(st, ops[0], r & M32)
        no_scc = ("s_mul_i32", "s_mul_hi_u32", "s_mul_hi_i32", "s_brev_b32", "s_sext_i32_i16",
                  "s_sext_i32_i8", "s_ff1_i32_b32", "s_ff1_i32_b64", "s_flbit_i32_b32",
                  "s_bitset0_b32", "s_bitset1_b32")
        if mn.startswith(("s_lshl_b64", "s_lshr_b64", "s_ashr_i64")):
            widths = [2, 1]
        elif mn in ("s_bcnt1_i32_b64", "s_ff1_i32_b64"):
            widths = [2]
        else:
            widths = [n] * (len(ops) - 1)
        srcs = [self.sget(st, ops[i], widths[i - 1]) for i in range(1, len(ops))]
        if mn == "s_or_b64" and ops[0].kind == ops[1].kind == "s" and ops[0].base == 126 \
                and ops[1].base == 126 and srcs[0] is None and srcs[1] is not None \
                and st.ebound & ~srcs[1] == 0:
            # the end of a divergent region: EXEC | saved EXEC, the saved value containing every
            # lane EXEC can hold
            srcs[0] = st.ebound & srcs[1]
        if any(x is None for x in srcs) or (mn in ("s_addc_u32", "s_subb_u32") and st.scc is None):
            self.sset(st, ops[0], None, n if not mn.startswith(("s_bcnt", "s_ff1")) else 1)
            if mn not in no_scc:
                st.scc = None
            return
        a = srcs[0]
        b = srcs[1] if len(srcs) > 1 else None
        scc = "keep"
        base = re.sub(r"_(b|i|u)(32|64)$", "", mn)
        if mn == "s_add_u32":
            t = a + b
            r, scc = t & M32, int(t >> 32)
        elif mn == "s_addc_u32":
            t = a + b + st.scc
            r, scc = t & M32, int(t >> 32)
        elif mn == "s_sub_u32":
            r, scc = (a - b) & M32, int(b > a)
        elif mn == "s_subb_u32":
            r, scc = (a - b - st.scc) & M32, int(b + st.scc > a)
        elif mn in ("s_add_i32", "s_sub_i32"):
            t = sx(a, 32) + sx(b, 32) if mn == "s_add_i32" else sx(a, 32) - sx(b, 32)
            r, scc = t & M32, int(t < -(1 << 31) or t >= (1 << 31))
        elif mn == "s_mul_i32":
            r = (sx(a, 32) * sx(b, 32)) & M32
        elif mn == "s_mul_hi_u32":
            r = ((a * b) >> 32) & M32
        elif mn == "s_mul_hi_i32":
            r = ((sx(a, 32) * sx(b, 32)) >> 32) & M32
        elif base in ("s_and", "s_or", "s_xor", "s_andn2", "s_orn2", "s_nand", "s_nor", "s_xnor"):
            r = {"s_and": a & b, "s_or": a | b, "s_xor": a ^ b, "s_andn2": a & ~b,
                 "s_orn2": a | (~b & mask), "s_nand": ~(a & b), "s_nor": ~(a | b),
                 "s_xnor": ~(a ^ b)}[base] & mask
            scc = int(r != 0)
        elif base == "s_not":
            r = ~a & mask
            scc = int(r != 0)
        elif base == "s_lshl":
            r = (a << (b & (bits - 1))) & mask
            scc = int(r != 0)
        elif base == "s_lshr":
            r = a >> (b & (bits - 1))
            scc = int(r != 0)
        elif base == "s_ashr":
            r = (sx(a) >> (b & (bits - 1))) & mask
            scc = int(r != 0)
        elif re.match(r"s_lshl[1-4]_add_u32$", mn):
            t = ((a << int(mn[6])) & M32) + b
            r, scc = t & M32, int(t >> 32)
        elif mn in ("s_min_i32", "s_max_i32"):
            x, y = sx(a, 32), sx(b, 32)
            r = (min(x, y) if mn == "s_min_i32" else max(x, y)) & M32
            scc = int((x < y) if mn == "s_min_i32" else (x > y))
        elif mn in ("s_min_u32", "s_max_u32"):
            r = min(a, b) if mn == "s_min_u32" else max(a, b)
            scc = int((a < b) if mn == "s_min_u32" else (a > b))
        elif mn == "s_abs_i32":
            r = abs(sx(a, 32)) & M32
            scc = int(r != 0)
        elif mn == "s_brev_b32":
            r = int("{:032b}".format(a)[::-1], 2)
        elif mn in ("s_bfe_u32", "s_bfe_i32"):
            off, width = b & 31, (b >> 16) & 0x7F
            v = (a >> off) & ((1 << width) - 1) if width else 0
            if mn == "s_bfe_i32" and width and (v >> (width - 1)) & 1:
                v -= 1 << width
            r = v & M32
            scc = int(r != 0)
        elif mn in ("s_sext_i32_i16", "s_sext_i32_i8"):
            w = 16 if mn.endswith("16") else 8
            r = sx(a & ((1 << w) - 1), w) & M32
        elif mn in ("s_bcnt1_i32_b32", "s_bcnt1_i32_b64"):
            r = bin(a).count("1")
            scc = int(r != 0)
            n = 1
        elif mn in ("s_ff1_i32_b32", "s_ff1_i32_b64"):
            r = ((a & -a).bit_length() - 1) & M32 if a else M32
            n = 1
        elif mn == "s_flbit_i32_b32":
            r = (32 - a.bit_length()) if a else M32
        else:
            raise Unsupported(I.text)
        self.sset(st, ops[0], r, n)
        if scc != "keep":
            st.scc = scc

    def s_load(self, st, ops):
        dst = ops[0]
        addr = self.sget(st, ops[1], 2)
        off = 0
        if len(ops) > 2:
            off = ops[2].val if ops[2].kind == "imm" else self.sget(st, ops[2], 1)
        for i in range(dst.n):
            p = None if addr != KERNARG or off is None else off + 4 * i
            if p is not None and p + 4 <= len(self.kernarg):
                st.s[dst.base + i] = struct.unpack_from("<I", self.kernarg, p)[0]
            else:
                st.s.pop(dst.base + i, None)

    # -- vector ALU
    def valu(self, st, I):
        mn, ops = I.mn, I.pops
        base = re.sub(r"_e(32|64)$", "", mn)
        if base.startswith(("v_cmp_", "v_cmpx_")):
            return self.vcmp(st, base, ops, I)
        if I.extra or base.startswith(("v_mfma", "v_smfmac")) or \
                any(o.mod for o in ops[1:]) or base.endswith(("_dpp", "_sdwa")):
            return self.unknown_dst(st, base, ops)
        if base in ("v_readfirstlane_b32", "v_readlane_b32"):
            src = self.vget(st, ops[1])
            if base == "v_readfirstlane_b32":
                ex = self.exec_mask(st)
                lane = None if ex is None else ((ex & -ex).bit_length() - 1 if ex else 0)
            else:
                ln = self.sget(st, ops[2], 1)
                lane = None if ln is None else ln & 63
            if src is None or lane is None or not src[1][lane]:
                return self.sset(st, ops[0], None)
            return self.sset(st, ops[0], int(src[0][lane]))
        if base == "v_writelane_b32":
            val, ln = self.sget(st, ops[1], 1), self.sget(st, ops[2], 1)
            old = st.v.get(ops[0].base, (np.zeros(LANES, dtype=np.uint32), _NOKNOW.copy()))
            vals, known = old[0].copy(), old[1].copy()
            if ln is None:
                st.v.pop(ops[0].base, None)
                return
            vals[ln & 63] = 0 if val is None else val
            known[ln & 63] = val is not None
            st.v[ops[0].base] = (vals, known)
            return
        fn = _VALU.get(base)
        if fn is None or fn(self, st, ops) is None:
            return self.unknown_dst(st, base, ops)

    def unknown_dst(self, st, base, ops):
        if not ops:
            return
        d = ops[0]
        if d.kind == "v":
            for i in range(d.n):
                self.vset(st, d, None, i)
        elif d.kind == "s":
            self.sset(st, d, None)
        if base.startswith(("v_add_co", "v_sub_co", "v_subrev_co", "v_addc", "v_subb",
                            "v_div_scale", "v_mad_u64", "v_mad_i64")) and len(ops) > 1:
            self.sset(st, ops[1], None)

    def vget64(self, st, op):
        """(values uint64[64], known) of a 64-bit source operand, or None."""
        if op.kind == "imm":
            v = op.val if op.val >> 32 == 0 and not (op.val & 0x80000000) else \
                op.val | 0xFFFFFFFF00000000
            return (np.full(LANES, v & 0xFFFFFFFFFFFFFFFF, dtype=np.uint64),
                    np.ones(LANES, dtype=bool))
        lo, hi = self.vget(st, op, 0), self.vget(st, op, 1)
        if lo is None or hi is None:
            return None
        return (lo[0].astype(np.uint64) | (hi[0].astype(np.uint64) << np.uint64(32)),
                lo[1] & hi[1])

    def vset64(self, st, op, vk):
        if vk is None:
            self.vset(st, op, None, 0)
            self.vset(st, op, None, 1)
            return
        v, k = vk
        self.vset(st, op, ((v & np.uint64(M32)).astype(np.uint32), k), 0)
        self.vset(st, op, ((v >> np.uint64(32)).astype(np.uint32), k), 1)

    def vcmp(self, st, base, ops, I):
        m = re.match(r"v_cmpx?_(\w+?)_(i32|u32|f32|i64|u64)$", base)
        if len(ops) == 2:
            dst, a_op, b_op = Op("s", 106, 2), ops[0], ops[1]
        else:
            dst, a_op, b_op = ops[0], ops[1], ops[2]
        if base.startswith("v_cmpx"):
            dst = Op("s", 126, 2)
        wide = bool(m) and m.group(2) in ("i64", "u64")
        a, b = ((self.vget64(st, a_op), self.vget64(st, b_op)) if wide
                else (self.vget(st, a_op), self.vget(st, b_op)))
        ex = self.exec_mask(st)
        if not m or I.extra or a is None or b is None or ex is None:
            return self.sset(st, dst, None, 2)
        op, ty = m.group(1), m.group(2)
        act = _bits(ex)
        if not (a[1] & b[1])[act].all():
            return self.sset(st, dst, None, 2)
        x, y = a[0], b[0]
        if ty == "i64":
            x, y = x.view(np.int64), y.view(np.int64)
        elif ty == "u64":
            x, y = x.astype(object), y.astype(object)
        elif ty == "i32":
            x, y = x.view(np.int32).astype(np.int64), y.view(np.int32).astype(np.int64)
        elif ty == "u32":
            x, y = x.astype(np.int64), y.astype(np.int64)
        else:
            x, y = x.view(np.float32).astype(np.float64), y.view(np.float32).astype(np.float64)
        with np.errstate(invalid="ignore"):
            table = {"eq": x == y, "ne": x != y, "lg": (x < y) | (x > y), "lt": x < y,
                     "le": x <= y, "gt": x > y, "ge": x >= y}
            table = {k: np.asarray(t, dtype=bool) for k, t in table.items()}
            if ty == "f32":
                nan = np.isnan(x) | np.isnan(y)
                table.update({"neq": ~table["eq"], "nlt": ~table["lt"], "nle": ~table["le"],
                              "ngt": ~table["gt"], "nge": ~table["ge"], "o": ~nan, "u": nan})
        if op not in table:
            return self.sset(st, dst, None, 2)
        self.sset(st, dst, _mask(table[op] & act), 2)


# ----------------------------------------------------------------------------------- VALU ops
def _lanes(m, st, ops, k):
    """The k source operands (values as uint64 arrays) and the lanes where all are known."""
    vs = [m.vget(st, o) for o in ops[1:1 + k]]
    if any(v is None for v in vs):
        return None, None
    known = np.ones(LANES, dtype=bool)
    for v in vs:
        known &= v[1]
    return [v[0].astype(np.uint64) for v in vs], known


def _int_op(k, fn):
    def op(m, st, ops):
        vs, known = _lanes(m, st, ops, k)
        if vs is None:
            return None
        m.vset(st, ops[0], ((fn(*vs) & M32).astype(np.uint32), known))
        return True
    return op


def _s32(x):
    return x.astype(np.uint32).view(np.int32).astype(np.int64)


def _f32(x):
    return x.astype(np.uint32).view(np.float32)


def _float_op(k, fn):
    def op(m, st, ops):
        vs, known = _lanes(m, st, ops, k)
        if vs is None:
            return None
        with np.errstate(all="ignore"):
            r = np.asarray(fn(*[_f32(v) for v in vs]), dtype=np.float32)
        m.vset(st, ops[0], (r.view(np.uint32), known))
        return True
    return op


def _cvt(fn):
    def op(m, st, ops):
        vs, known = _lanes(m, st, ops, 1)
        if vs is None:
            return None
        with np.errstate(all="ignore"):
            r = fn(vs[0])
        m.vset(st, ops[0], (r, known))
        return True
    return op


def _sat_int(x, lo, hi):
    x = np.where(np.isnan(x), 0, x)
    return np.clip(np.trunc(x), lo, hi)


def _v_mov64(m, st, ops):
    for d in range(2):
        m.vset(st, ops[0], m.vget(st, ops[1], d), d)
    return True


def _v_cndmask(m, st, ops):
    vs, known = _lanes(m, st, ops, 2)
    sel = m.sget(st, ops[3], 2) if len(ops) > 3 else m.sget(st, Op("s", 106, 2), 2)
    if vs is None or sel is None:
        return None
    m.vset(st, ops[0], (np.where(_bits(sel), vs[1], vs[0]).astype(np.uint32), known))
    return True


def _carry_op(kind):
    # v_add_co_u32 vdst, sdst(carry out), src0, src1; v_addc_co_u32 ..., src0, src1, carry in
    def op(m, st, ops):
        a, b = m.vget(st, ops[2]), m.vget(st, ops[3])
        cin = m.sget(st, ops[4], 2) if kind == "addc" and len(ops) > 4 else 0
        ex = m.exec_mask(st)
        if a is None or b is None or cin is None or ex is None:
            m.sset(st, ops[1], None, 2)
            return None
        x, y = a[0].astype(np.int64), b[0].astype(np.int64)
        known = a[1] & b[1]
        c = _bits(cin).astype(np.int64)
        t = {"add": x + y, "addc": x + y + c, "sub": x - y, "subrev": y - x}[kind]
        carry = (t > M32) if kind in ("add", "addc") else (t < 0)
        m.vset(st, ops[0], ((t & M32).astype(np.uint32), known))
        act = _bits(ex)
        m.sset(st, ops[1], _mask(carry & act) if known[act].all() else None, 2)
        return True
    return op


def _v_mad_u64_u32(m, st, ops):
    # v_mad_u64_u32 vdst[2], sdst, src0, src1, src2[64 bits]
    a, b = m.vget(st, ops[2]), m.vget(st, ops[3])
    lo, hi = m.vget(st, ops[4], 0), m.vget(st, ops[4], 1)
    m.sset(st, ops[1], None, 2)
    if a is None or b is None or lo is None or hi is None:
        m.vset(st, ops[0], None, 0)
        m.vset(st, ops[0], None, 1)
        return True
    known = a[1] & b[1] & lo[1] & hi[1]
    t = [int(a[0][i]) * int(b[0][i]) + (int(lo[0][i]) | (int(hi[0][i]) << 32))
         for i in range(LANES)]
    m.vset(st, ops[0], (np.array([x & M32 for x in t], dtype=np.uint32), known), 0)
    m.vset(st, ops[0], (np.array([(x >> 32) & M32 for x in t], dtype=np.uint32), known), 1)
    return True


def _bitop3(m, st, ops):
    # v_bitop3_b32 dst, a, b, c, lut: result bit = lut[(a << 2) | (b << 1) | c]
    if len(ops) < 5 or ops[4].kind != "imm":
        return None
    vs, known = _lanes(m, st, ops, 3)
    if vs is None:
        return None
    a, b, c = vs
    lut = ops[4].val & 0xFF
    out = np.zeros(LANES, dtype=np.uint64)
    for k in range(8):
        if (lut >> k) & 1:
            out |= (a if k & 4 else ~a) & (b if k & 2 else ~b) & (c if k & 1 else ~c)
    m.vset(st, ops[0], ((out & M32).astype(np.uint32), known))
    return True


def _v_lshl_add_u64(m, st, ops):
    a, c = m.vget64(st, ops[1]), m.vget64(st, ops[3])
    sh = m.vget(st, ops[2])
    if a is None or c is None or sh is None:
        return None
    with np.errstate(over="ignore"):
        r = (a[0] << (sh[0].astype(np.uint64) & np.uint64(63))) + c[0]
    m.vset64(st, ops[0], (r, a[1] & c[1] & sh[1]))
    return True


def _shift64(kind):
    def op(m, st, ops):
        sh, a = m.vget(st, ops[1]), m.vget64(st, ops[2])
        if a is None or sh is None:
            return None
        k = sh[0].astype(np.uint64) & np.uint64(63)
        if kind == "l":
            r = a[0] << k
        elif kind == "r":
            r = a[0] >> k
        else:
            r = (a[0].view(np.int64) >> k.astype(np.int64)).view(np.uint64)
        m.vset64(st, ops[0], (r, a[1] & sh[1]))
        return True
    return op


_SH = np.uint64(31)
_VALU = {
    "v_lshl_add_u64": _v_lshl_add_u64,
    "v_lshlrev_b64": _shift64("l"),
    "v_lshrrev_b64": _shift64("r"),
    "v_ashrrev_i64": _shift64("a"),
    "v_mov_b32": _int_op(1, lambda a: a),
    "v_mov_b64": _v_mov64,
    "v_cndmask_b32": _v_cndmask,
    "v_add_u32": _int_op(2, lambda a, b: a + b),
    "v_sub_u32": _int_op(2, lambda a, b: a - b),
    "v_subrev_u32": _int_op(2, lambda a, b: b - a),
    "v_add_co_u32": _carry_op("add"),
    "v_addc_co_u32": _carry_op("addc"),
    "v_sub_co_u32": _carry_op("sub"),
    "v_subrev_co_u32": _carry_op("subrev"),
    "v_mul_lo_u32": _int_op(2, lambda a, b: a * b),
    "v_mul_hi_u32": _int_op(2, lambda a, b: (a * b) >> np.uint64(32)),
    "v_mul_u32_u24": _int_op(2, lambda a, b: (a & 0xFFFFFF) * (b & 0xFFFFFF)),
    "v_mad_u32_u24": _int_op(3, lambda a, b, c: (a & 0xFFFFFF) * (b & 0xFFFFFF) + c),
    "v_mad_u64_u32": _v_mad_u64_u32,
    "v_lshlrev_b32": _int_op(2, lambda a, b: b << (a & _SH)),
    "v_lshrrev_b32": _int_op(2, lambda a, b: b >> (a & _SH)),
    "v_ashrrev_i32": _int_op(2, lambda a, b: (_s32(b) >> _s32(a & _SH)).astype(np.uint64)),
    "v_and_b32": _int_op(2, lambda a, b: a & b),
    "v_or_b32": _int_op(2, lambda a, b: a | b),
    "v_xor_b32": _int_op(2, lambda a, b: a ^ b),
    "v_not_b32": _int_op(1, lambda a: ~a),
    "v_bfe_u32": _int_op(3, lambda a, b, c: (a >> (b & _SH)) & ((np.uint64(1) << (c & _SH))
                                                                  - np.uint64(1))),
    "v_bfi_b32": _int_op(3, lambda a, b, c: (a & b) | (~a & c)),
    "v_lshl_add_u32": _int_op(3, lambda a, b, c: ((a << (b & _SH)) & M32) + c),
    "v_add_lshl_u32": _int_op(3, lambda a, b, c: ((a + b) & M32) << (c & _SH)),
    "v_lshl_or_b32": _int_op(3, lambda a, b, c: (a << (b & _SH)) | c),
    "v_and_or_b32": _int_op(3, lambda a, b, c: (a & b) | c),
    "v_or3_b32": _int_op(3, lambda a, b, c: a | b | c),
    "v_xad_u32": _int_op(3, lambda a, b, c: (a ^ b) + c),
    "v_add3_u32": _int_op(3, lambda a, b, c: a + b + c),
    "v_min_u32": _int_op(2, np.minimum),
    "v_max_u32": _int_op(2, np.maximum),
    "v_min_i32": _int_op(2, lambda a, b: np.minimum(_s32(a), _s32(b)).astype(np.uint64)),
    "v_max_i32": _int_op(2, lambda a, b: np.maximum(_s32(a), _s32(b)).astype(np.uint64)),
    "v_bitop3_b32": _bitop3,
    "v_cvt_f32_u32": _cvt(lambda a: a.astype(np.float64).astype(np.float32).view(np.uint32)),
    "v_cvt_f32_i32": _cvt(lambda a: _s32(a).astype(np.float64).astype(np.float32)
                          .view(np.uint32)),
    "v_cvt_u32_f32": _cvt(lambda a: _sat_int(_f32(a).astype(np.float64), 0, M32)
                          .astype(np.uint64).astype(np.uint32)),
    "v_cvt_i32_f32": _cvt(lambda a: _sat_int(_f32(a).astype(np.float64), -(1 << 31),
                                             (1 << 31) - 1).astype(np.int64).astype(np.uint32)),
    "v_rcp_iflag_f32": _float_op(1, lambda a: np.float32(1.0) / a),
    "v_rcp_f32": _float_op(1, lambda a: np.float32(1.0) / a),
    "v_mul_f32": _float_op(2, lambda a, b: a * b),
    "v_add_f32": _float_op(2, lambda a, b: a + b),
    "v_sub_f32": _float_op(2, lambda a, b: a - b),
    "v_subrev_f32": _float_op(2, lambda a, b: b - a),
}


def kernarg_bytes(args, values):
    """The kernel-argument segment for argument values in signature order: ints for integer and
    pointer arguments (8 or 4 bytes by the argument's size), floats for float arguments."""
    assert len(args) == len(values), (len(args), len(values))
    buf = bytearray(max(o + s for o, s in args))
    for (off, sz), v in zip(args, values):
        if isinstance(v, float):
            struct.pack_into("<f", buf, off, v)
        elif sz == 8:
            struct.pack_into("<Q", buf, off, v & 0xFFFFFFFFFFFFFFFF)
        else:
            struct.pack_into("<I", buf, off, v & M32)
    return bytes(buf)


_MACHINES = {}


def barrier_counts(asm, name, values, wg_id, max_steps=3_000_000, waves=None):
    """Barriers executed by each wave of workgroup `wg_id` of kernel `name`, for kernel arguments
    `values` (signature order), and the per-wave final states (their `valu` / `mfma` counts).
    Raises `DataDependentBarrier` or `NoTermination`."""
    key = (hash(asm), name)
    m = _MACHINES.get(key)
    if m is None:
        m = _MACHINES[key] = Machine(asm, name, max_steps)
    m.max_steps = max_steps
    kb = kernarg_bytes(m.args, values)
    counts, states = [], []
    for w in (range(m.wg // LANES) if waves is None else waves):
        counts.append(m.run_wave(kb, wg_id, w))
        states.append(m.last)
    return counts, states
