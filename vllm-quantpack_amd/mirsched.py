"""Post-register-allocation instruction scheduler for kernels that run one wave per SIMD on gfx950.

The build hands this module the LLVM machine IR (MIR) of a HIP source, stopped right after LLVM's post-RA machine
scheduler, and it reorders the instructions inside every basic block of the selected kernels that holds an MFMA.
LLVM then runs its remaining passes on the result: the memory legalizer, the wait-count insertion (s_waitcnt for
every register an instruction reads before its load has landed) and the hazard recognizer (s_nop where an operand
is not ready), so those stay LLVM's own, computed for the new order.

Why. With one wave per SIMD there is no other wave to fill the matrix pipe's shadow: a 16x16x32 bf16 MFMA occupies
the pipe for 16 cycles but the wave's issue for only about 9, so about 7 cycles of other instructions (one or two
VALU ops, an LDS read) come free behind each MFMA, and MFMAs issued back to back waste them. Measured on MI355X with
a fully unrolled loop of 32 MFMAs and N independent instructions after each: max(16.6, 9 + 4 N) cycles per MFMA for
v_fma_f32 (N = 0..8), 8 cycles per v_exp_f32, the same with VGPR or AGPR accumulators and operands. LLVM's scheduler
does not use that: its order leaves the kernel's MFMAs in back-to-back runs and its VALU work in clumps.

What it does. A list scheduler over each block's dependence graph, cycle by cycle on that issue model: an MFMA issues
as soon as its operands are ready and the matrix pipe is free, and in between the instruction on the longest
remaining path whose operands are ready fills the issue slots. Dependences:
  * registers: every read after the write it sees (with the writer's latency), every write after earlier reads and
    writes of the register; register tuples, subregisters and implicit operands (exec, vcc, scc, m0) are expanded to
    32-bit units;
  * memory and side effects: every instruction that is not a plain register-to-register ALU operation (loads,
    stores, LDS accesses, barriers, waits, fences, inline assembly that touches memory, wait counters or exec) keeps
    its order relative to all the others of that kind;
  * inline assembly reads EXEC (its vector instructions run under it, though the statement does not list it), so
    it never moves across an EXEC write such as a lane-masked region's s_and_saveexec;
  * a barrier (s_barrier) is a full fence: every instruction before it stays before it and every one after it stays
    after it, register-only ones included. A variant that let the scalar add forming an LDS-DMA copy's M0 value move
    from before a barrier to just after it gave results that differed from call to call (the cause was not found);
    with the fence the prefill kernels measure the same;
  * inline-assembly MFMAs (invisible to LLVM's hazard recognizer): one that carries trailing wait states stays after
    every earlier inline MFMA of its block, and no later one moves above it, so the wait states still follow the
    last of them;
  * a block's terminators stay at its end.
The build scans the final assembly for reads of inline-MFMA results within 18 wait states, VALU writes of MFMA
sources within 2, and spills in MFMA loops, as for every other source.
"""
import re
import sys
from collections import defaultdict

# issue model (cycles): what the wave's issue spends on an instruction, when its result can be read, and how long the
# matrix pipe stays busy
MFMA_ISSUE = 8
MFMA_PIPE = {16: 16, 32: 32}      # 16x16xK / 32x32xK bf16
MFMA_LATENCY = {16: 24, 32: 40}
VALU_ISSUE = 4
TRANS_ISSUE = 8                   # v_exp / v_log / v_rcp / ... (half rate)
LDS_ISSUE_WIDE = 8                # ds_read_b128 / ds_write_b128
LDS_ISSUE = 4
LDS_LATENCY = 120
SMEM_LATENCY = 200
VMEM_LATENCY = 600

_GPR = re.compile(r"^(vgpr|agpr|sgpr|ttmp)(\d+)$")
_PREFIX = {"vgpr": "v", "agpr": "a", "sgpr": "s", "ttmp": "t"}
_FLAGS = ("contract", "nofpexcept", "nsz", "arcp", "afn", "reassoc", "nnan", "ninf", "exact", "nuw", "nsw",
          "disjoint", "nneg", "samesign", "frame-setup", "frame-destroy")
_MODIFIERS = r"(?:dead|killed|undef|renamable|early-clobber|internal)\s+"
# plain register-to-register ALU operations; everything else is ordered as a memory / side-effect operation
_PURE = ("V_", "S_ADD", "S_SUB", "S_MUL", "S_MOV", "S_AND", "S_OR", "S_XOR", "S_LSH", "S_ASHR", "S_CSELECT", "S_CMP",
         "S_BFE", "S_NOT", "S_ANDN", "S_ORN", "S_NAND", "S_NOR", "S_XNOR", "S_MIN", "S_MAX", "S_ABS", "S_BREV", "S_FF",
         "S_FLBIT", "S_BCNT", "S_SEXT", "S_CMOV", "S_PACK", "S_BFM", "S_BITCMP", "S_CVT")
_TERMINATORS = ("S_BRANCH", "S_CBRANCH", "SI_RETURN", "S_ENDPGM", "SI_END_CF", "SI_LOOP", "SI_IF", "SI_ELSE",
                "S_SETPC", "SI_BRCOND")
# inline assembly that mentions any of these is ordered like a memory operation
_ASM_MEMORY = ("ds_", "global_", "buffer_", "flat_", "scratch_", "s_load", "s_store", "s_buffer", "s_waitcnt",
               "s_barrier", "s_dcache", "m0", "exec", "s_memtime", "s_sleep", "s_setprio", "s_sendmsg")
_TRANS = ("V_EXP", "V_LOG", "V_RCP", "V_RSQ", "V_SQRT", "V_SIN", "V_COS")
_VALU64 = ("V_LSHL_ADD_U64", "V_MAD_U64", "V_MOV_B64", "V_ADD_U64", "V_LSHLREV_B64", "V_LSHRREV_B64", "V_FMA_F64",
           "V_ADD_F64", "V_MUL_F64")  # two passes


def reg_units(name):
    """The 32-bit register units a MIR register names: '$vgpr4_vgpr5' -> {'v4', 'v5'}, '$vcc' -> {'vcc_lo',
    'vcc_hi'}, '$m0' -> {'m0'}; '$noreg', '$mode' and inline-asm operand numbers name none."""
    n = name.lstrip("$")
    if n.isdigit() or n in ("noreg", "sgpr_null", "mode", "private_rsrc_reg"):
        return set()
    if n in ("vcc", "exec", "flat_scr", "xnack_mask"):
        return {n + "_lo", n + "_hi"}
    parts = n.split("_")
    out = set()
    i = 0
    while i < len(parts):
        m = _GPR.match(parts[i])
        if m:
            out.add(_PREFIX[m.group(1)] + m.group(2))
            i += 1
        elif i + 1 < len(parts) and parts[i + 1] in ("lo", "hi", "lo16", "hi16"):
            out.add(parts[i] + "_" + parts[i + 1])
            i += 2
        else:
            out.add(parts[i])
            i += 1
    return out


class Inst:
    """One MIR instruction (a BUNDLE with its body counts as one): its register units read and written, whether it
    is ordered as a memory / side-effect operation, and its issue cost, latency and matrix-pipe time."""

    def __init__(self, text):
        self.text = text
        first = text.split("\n")[0].strip()
        head = first.split('"')[0]
        lhs, rhs = (first.split(" = ", 1) if " = " in head else ("", first))
        self.op = next((t for t in rhs.replace(",", " ").split() if t not in _FLAGS and not t.startswith("$")), "")
        self.defs, self.uses = set(), set()
        for r in re.findall(r"\$[A-Za-z0-9_]+", lhs):
            self.defs |= reg_units(r)
        self.asm = ""
        if self.op == "BUNDLE":
            self._implicit(text.split("{", 1)[0])
            for line in text.split("{", 1)[1].rsplit("}", 1)[0].split("\n"):
                if line.strip():
                    sub = Inst(line.strip())
                    self.defs |= sub.defs
                    self.uses |= sub.uses
            self.mem = True
        elif self.op == "INLINEASM":
            self.asm = text.split('"')[1] if '"' in text else ""
            operands = text.split('"', 2)[2] if text.count('"') >= 2 else text
            for m in re.finditer(r"(implicit-def|implicit|def)?\s*(?:" + _MODIFIERS + r")*(\$[A-Za-z0-9_]+)", operands):
                (self.defs if m.group(1) in ("def", "implicit-def") else self.uses).update(reg_units(m.group(2)))
            # vector instructions inside run under EXEC, which the statement does not list: never across its writes
            self.uses |= {"exec_lo", "exec_hi"}
            self.mem = any(k in self.asm for k in _ASM_MEMORY)
        else:
            self._implicit(rhs)
            for m in re.finditer(r"(implicit-def|implicit)?\s*(?:" + _MODIFIERS + r")*(\$[A-Za-z0-9_]+)", rhs):
                if not m.group(1):
                    self.uses |= reg_units(m.group(2))
            self.mem = not self.op.startswith(_PURE) or "::" in text
        self.term = self.op.startswith(_TERMINATORS)
        self.trailing_waits = "s_nop" in self.asm and "v_mfma" in self.asm
        self._cost()

    def _implicit(self, s):
        for m in re.finditer(r"(implicit-def|implicit)\s+(?:" + _MODIFIERS + r")*(\$[A-Za-z0-9_]+)", s):
            (self.defs if m.group(1) == "implicit-def" else self.uses).update(reg_units(m.group(2)))

    def _cost(self):
        op = self.op
        self.mfmas, self.pipe = 0, 0
        if "MFMA" in op:
            size = 32 if "32X32" in op else 16
            self.kind, self.mfmas = "mfma", 1
            self.cost, self.pipe, self.lat = MFMA_ISSUE, MFMA_PIPE[size], MFMA_LATENCY[size]
        elif op == "INLINEASM":
            n = self.asm.count("v_mfma")
            nops = sum(int(x) + 1 for x in re.findall(r"s_nop\s+(\d+)", self.asm))
            if n:
                size = 32 if "32x32" in self.asm else 16
                self.kind, self.mfmas = "mfma", n
                self.cost, self.pipe, self.lat = MFMA_ISSUE * n + nops, MFMA_PIPE[size] * n, MFMA_LATENCY[size]
            else:
                lds = self.asm.count("ds_read") + self.asm.count("ds_write")
                self.kind = "asm"
                self.cost = 4 + LDS_ISSUE_WIDE * (lds + self.asm.count("global_load")) + nops
                self.lat = LDS_LATENCY if lds else 8
        elif op.startswith("DS_") or op == "BUNDLE":
            n = max(1, self.text.count("DS_"))
            self.kind = "lds"
            self.cost = n * (LDS_ISSUE_WIDE if ("B128" in self.text or "B96" in self.text) else LDS_ISSUE)
            self.lat = LDS_LATENCY
        elif op.startswith(("S_LOAD", "S_BUFFER")):
            self.kind, self.cost, self.lat = "smem", 2, SMEM_LATENCY
        elif op.startswith(("GLOBAL_", "BUFFER_", "FLAT_", "SCRATCH_")):
            self.kind, self.cost, self.lat = "vmem", 8, VMEM_LATENCY
        elif op.startswith("V_"):
            self.kind = "valu"
            self.cost = self.lat = TRANS_ISSUE if op.startswith(_TRANS + _VALU64) else VALU_ISSUE
            if op.startswith(("V_READFIRSTLANE", "V_READLANE", "V_CMP")):
                self.lat = 8
        elif op.startswith("S_"):
            self.kind, self.cost, self.lat = "salu", 1, 2
        else:  # pseudo-instructions (IMPLICIT_DEF, KILL, ...)
            self.kind, self.cost, self.lat = "other", 1, 1


def dependences(insts):
    """preds[i] = {j: latency} for the instructions of one block, in their original order."""
    preds = [dict() for _ in insts]
    last_def, reads = {}, defaultdict(list)
    last_mem = last_nop_mfma = None
    inline_mfmas = []

    def edge(i, j, lat):
        if j is not None and j != i:
            preds[i][j] = max(preds[i].get(j, 0), lat)

    last_barrier = None
    for i, ins in enumerate(insts):
        if ins.op.startswith("S_BARRIER"):  # a full fence (module docstring)
            for j in range(i):
                edge(i, j, 1)
            last_barrier = i
        else:
            edge(i, last_barrier, 1)
        for u in ins.uses:
            if u in last_def:
                edge(i, last_def[u], insts[last_def[u]].lat)
        for d in ins.defs:
            edge(i, last_def.get(d), 1)
            for r in reads[d]:
                edge(i, r, 1)
        if ins.mem:
            edge(i, last_mem, 1)
            last_mem = i
        if ins.op == "INLINEASM" and ins.mfmas:
            if ins.trailing_waits:
                for j in inline_mfmas:
                    edge(i, j, 1)
                inline_mfmas = []
                last_nop_mfma = i
            else:
                edge(i, last_nop_mfma, 1)
                inline_mfmas.append(i)
        for u in ins.uses:
            reads[u].append(i)
        for d in ins.defs:
            last_def[d] = i
            reads[d] = []
    return preds


def schedule(insts):
    """The block's instructions in the list scheduler's order (terminators and whatever follows the first one stay
    at the end)."""
    first_term = next((k for k, x in enumerate(insts) if x.term), len(insts))
    body, tail = insts[:first_term], insts[first_term:]
    n = len(body)
    if n < 3:
        return list(insts)
    preds = dependences(body)
    succs = [dict() for _ in range(n)]
    for i in range(n):
        for p, lat in preds[i].items():
            succs[p][i] = lat
    height = [0] * n  # latency-weighted path to the block's end
    for i in reversed(range(n)):
        height[i] = body[i].cost + max((lat + height[s] for s, lat in succs[i].items()), default=0)
    waiting = [len(preds[i]) for i in range(n)]
    ready_at = [0] * n
    cand = {i for i in range(n) if not waiting[i]}
    order, t, pipe_free = [], 0, 0
    while cand:
        best_key, best = None, None
        for c in cand:
            ins = body[c]
            start = max(t, ready_at[c], pipe_free if ins.kind == "mfma" else 0)
            # what can start first; among those an MFMA (the pipe is the bottleneck), then the longest path
            key = (start, ins.kind != "mfma", -height[c], c)
            if best_key is None or key < best_key:
                best_key, best = key, c
        ins, start = body[best], best_key[0]
        if ins.kind == "mfma":
            pipe_free = start + ins.pipe
        t = start + ins.cost
        order.append(best)
        cand.remove(best)
        for s, lat in succs[best].items():
            waiting[s] -= 1
            ready_at[s] = max(ready_at[s], start + lat)
            if not waiting[s]:
                cand.add(s)
    assert len(order) == n, "dependence cycle"
    return [body[i] for i in order] + tail


def _function_ranges(lines, pattern):
    """(start, end) line ranges of the MIR functions whose name matches `pattern`."""
    out, start = [], None
    name_re = re.compile(pattern)
    for i, line in enumerate(lines):
        if line.startswith("name:"):
            start = i if name_re.search(line.split(":", 1)[1].strip()) else None
        elif start is not None and (line.startswith("---") or line.startswith("...")):
            out.append((start, i))
            start = None
    if start is not None:
        out.append((start, len(lines)))
    return out


def _blocks(lines, s, e):
    """(first instruction line, end line) of every basic block in lines[s:e]."""
    out, i = [], s
    while i < e:
        if re.match(r"^  bb\.\d+", lines[i]):
            h = i + 1
            while h < e and re.match(r"^    (successors|liveins|predecessors):", lines[h]):
                h += 1
            j = h
            while j < e and not re.match(r"^  bb\.\d+", lines[j]):
                j += 1
            out.append((h, j))
            i = j
        else:
            i += 1
    return out


def _instructions(lines, h, j):
    out, k = [], h
    while k < j:
        line = lines[k]
        if not line.strip() or line.strip().startswith(";"):
            k += 1
        elif line.rstrip().endswith("{"):
            m = k
            while lines[m].strip() != "}":
                m += 1
            out.append("\n".join(lines[k:m + 1]))
            k = m + 1
        else:
            out.append(line)
            k += 1
    return out


def schedule_mir(text, pattern):
    """The MIR text with every MFMA-holding block of the functions matching `pattern` rescheduled; returns (text,
    number of blocks rescheduled). Kill flags are dropped from moved blocks (the order they described changed)."""
    # The register scavenger's frame index is stale once prologue/epilogue insertion has lowered the frame (before
    # this point), and this LLVM's MIR parser rejects it when it names a stack object listed after it: drop it (the
    # round trip then reproduces LLVM's code exactly, spill code included).
    lines = [l for l in text.split("\n") if not re.match(r"^  scavengeFI:\s+'%stack\.\d+'\s*$", l)]
    repl = []
    for s, e in _function_ranges(lines, pattern):
        for h, j in _blocks(lines, s, e):
            insts = [Inst(t) for t in _instructions(lines, h, j)]
            if not any(x.mfmas for x in insts):
                continue
            repl.append((h, j, [re.sub(r"\bkilled ", "", x.text) for x in schedule(insts)]))
    for h, j, new in sorted(repl, reverse=True):
        lines[h:j] = new + [""]
    return "\n".join(lines), len(repl)


def main(argv=None):
    a = argv if argv is not None else sys.argv[1:]
    if len(a) != 3:
        raise SystemExit("usage: mirsched.py IN.mir OUT.mir FUNCTION_REGEX")
    text, n = schedule_mir(open(a[0]).read(), a[2])
    open(a[1], "w").write(text)
    print(f"{n} blocks rescheduled", file=sys.stderr)
    return 0


if __name__ == "__main__":
    sys.exit(main())
