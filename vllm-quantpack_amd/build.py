"""Build libquantpack_hip.so for gfx950 from csrc/*.hip with hipcc (objects in _build/, the library in-tree next to
the Python package so that it travels with the source tree).

    python vllm-quantpack_amd/build.py [--jobs N] [--verbose] [--only a.hip,b.hip]

The prefill source's device code goes through mirsched.py (an MFMA/VALU interleaving scheduler over LLVM's machine
IR); QP_NO_MIRSCHED=1 builds it in LLVM's own order instead, for comparison.
"""
import argparse
import concurrent.futures as cf
import os
import re
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
OBJ = os.path.join(HERE, "_build")
LIB = os.path.join(HERE, "vllm_quantpack", "libquantpack_hip.so")
ARCH = os.environ.get("QP_OFFLOAD_ARCH", "gfx950")

# -packed-fp32-ops: no v_pk_{add,mul,fma}_f32 in any generated code.
FLAGS = ["-O3", "-std=c++17", "-fPIC", f"--offload-arch={ARCH}", "-I", os.path.join(REPO, "include"), "-I", CSRC,
         "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops", "-Wall", "-Wno-unused-result",
         "-Wno-unused-variable"]


def hipcc():
    rocm = os.environ.get("ROCM_PATH", "/opt/rocm")
    path = os.path.join(rocm, "bin", "hipcc")
    return path if os.path.exists(path) else "hipcc"


# Per-source extra flags. The prefill kernel keeps its QK^T MFMA results in VGPRs (its PV accumulators own the AGPRs).
# The decode kernels take no NaN inputs (masked scores are -inf, never NaN), so their maxima need no quieting.
EXTRA = {"qp_prefill.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"],
         "qp_prefill_i8.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"],
         # the one atomic (a chunk claim by lane 0) needs no wave-level reduction around it
         "qp_decode.hip": ["-fno-honor-nans", "-mllvm", "-amdgpu-atomic-optimizer-strategy=None"]}


# Sources whose kernels (function names matching the pattern) go through the post-RA MFMA/VALU interleaving
# scheduler (mirsched.py): their device code is compiled to LLVM MIR, stopped after LLVM's post-RA scheduler,
# reordered, and finished by LLVM (wait counts, hazard wait states, emission). Measured on 1024-token prefill chunks
# over 131072 keys: the tile kernel 2.94-3.02 ms against 3.13 ms in LLVM's order, the wide kernel 6.28-6.30 against
# 6.50-6.52 ms (head 128, 64 / 8 heads) and 4.89-4.92 against 5.01-5.03 ms (head 512). The decode kernel measured
# slower scheduled (33.9-34.8 against 31.9-32.2 us) and the int8 alternative within 1 %, so they keep LLVM's order.
SCHEDULED = {"qp_prefill.hip": r"^_ZN2qp14prefill_kernel",
             "qp_prefill_wide.hip": r"^_ZN2qp19prefill_wide_kernel"}


def _flags(src):
    return FLAGS + EXTRA.get(os.path.basename(src), [])


def _run(cmd, what, verbose):
    if verbose:
        print(" ".join(cmd), flush=True)
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"{what} failed:\n{' '.join(cmd)}\n{r.stdout[-4000:]}\n{r.stderr[-4000:]}")


def _llvm_tool(name):
    return os.path.join(os.environ.get("ROCM_PATH", "/opt/rocm"), "llvm", "bin", name)


def _compile_scheduled(src, pattern, verbose):
    """Device code through LLVM MIR and mirsched, then the host object with that device binary embedded (what
    hipcc -c does in one step). Also writes the device assembly for the inline-MFMA checks."""
    if HERE not in sys.path:
        sys.path.insert(0, HERE)
    import mirsched
    stem = os.path.join(OBJ, os.path.basename(src).replace(".hip", ""))
    obj, asm = stem + ".o", stem + ".gfx.s"
    ll, mir, smir = stem + ".dev.ll", stem + ".dev.mir", stem + ".sched.mir"
    dobj, hsaco, fatbin = stem + ".dev.o", stem + ".hsaco", stem + ".hipfb"
    flags = _flags(src)
    cuid = ["-cuid=" + os.path.basename(src).replace(".", "_")]  # the same id for the device and the host half
    llvm_opts = [flags[i + 1] for i in range(len(flags) - 1) if flags[i] == "-mllvm"]
    llc = [_llvm_tool("llc"), "-O3", "-mtriple=amdgcn-amd-amdhsa", f"-mcpu={ARCH}", *llvm_opts]
    try:
        _run([hipcc(), *flags, *cuid, "--cuda-device-only", "-S", "-emit-llvm", src, "-o", ll], "device IR", verbose)
        _run([*llc, ll, "-stop-after=postmisched", "-o", mir], "llc (to MIR)", verbose)
        text, n = mirsched.schedule_mir(open(mir).read(), pattern)
        if n == 0:
            raise RuntimeError(f"mirsched: no MFMA block of {pattern} in {src}")
        with open(smir, "w") as f:
            f.write(text)
        _run([*llc, smir, "-start-after=postmisched", "-filetype=obj", "-o", dobj], "llc (from MIR)", verbose)
        _run([*llc, smir, "-start-after=postmisched", "-o", asm], "llc (assembly)", verbose)
        _run([_llvm_tool("lld"), "-flavor", "gnu", "-m", "elf64_amdgpu", "--no-undefined", "-shared", "-o", hsaco,
              dobj], "lld", verbose)
        _run([_llvm_tool("clang-offload-bundler"), "-type=o", "-bundle-align=4096",
              f"-targets=host-x86_64-unknown-linux-gnu,hipv4-amdgcn-amd-amdhsa--{ARCH}", "-input=/dev/null",
              f"-input={hsaco}", f"-output={fatbin}"], "offload bundler", verbose)
        _run([hipcc(), *flags, *cuid, "--cuda-host-only", "-Xclang", "-fcuda-include-gpubinary", "-Xclang", fatbin,
              "-c", src, "-o", obj], "host compile", verbose)
    finally:
        for f in (ll, mir, smir, dobj):  # tens of MB each
            if os.path.exists(f):
                os.remove(f)
    return obj


def _compile(src, verbose):
    """Compiles one source into _build/; returns whether its device code went through the scheduler."""
    obj = os.path.join(OBJ, os.path.basename(src).replace(".hip", ".o"))
    pattern = SCHEDULED.get(os.path.basename(src))
    if pattern and not os.environ.get("QP_NO_MIRSCHED"):
        try:
            _compile_scheduled(src, pattern, verbose)
            return True
        except (RuntimeError, OSError) as e:  # the plain compile below still builds a working library
            print(f"warning: {os.path.basename(src)}: scheduled build failed, compiling in LLVM's order ({e})",
                  file=sys.stderr, flush=True)
    _run([hipcc(), *_flags(src), "-c", src, "-o", obj], f"hipcc on {src}", verbose)
    return False


# Inline-assembly MFMAs are invisible to the compiler's hazard recognizer: it does not know that their results land
# some cycles after issue, and may read them (a copy of its own, for instance) too early. The kernels place the
# required wait states inside their assembly; this scan of the generated code checks that nothing reads or writes the
# destination of an inline-assembly MFMA within MFMA_WAIT wait states (each intervening instruction counted as one,
# s_nop N as N + 1), except a following MFMA that accumulates into exactly the same registers (srcC = vdst, which the
# hardware orders). The compiler's own MFMAs are covered by its hazard recognizer.
MFMA_WAIT = 18
_REG = re.compile(r"\b([va])\[(\d+):(\d+)\]|\b([va])(\d+)\b")


def _vregs(text):
    """VGPRs and AGPRs named in an operand list, as ('v', n) / ('a', n)."""
    out = set()
    for m in _REG.finditer(text):
        if m.group(4) is not None:
            out.add((m.group(4), int(m.group(5))))
        else:
            out.update((m.group(1), r) for r in range(int(m.group(2)), int(m.group(3)) + 1))
    return out


def mfma_hazards(asm):
    """[(line, mfma, reader)] of too-early accesses to the results of inline-assembly MFMAs (those between the
    compiler's ;;#ASMSTART / ;;#ASMEND markers) in one assembly listing."""
    ins = []
    inline = False
    for i, raw in enumerate(asm.splitlines()):
        l = raw.strip()
        if l.startswith(";;#ASMSTART"):
            inline = True
        elif l.startswith(";;#ASMEND"):
            inline = False
        elif l and not l.startswith((";", ".")) and not raw.startswith((".", "_")):
            ins.append((i, l.split(";")[0].strip(), inline))
    found = []
    for k, (i, line, inl) in enumerate(ins):
        if not (inl and line.startswith("v_mfma")):
            continue
        regs = _vregs(line.split(None, 1)[1].split(",")[0])
        waits = 0
        for _, nxt, _ in ins[k + 1:k + 1 + MFMA_WAIT]:
            if waits >= MFMA_WAIT:
                break
            op = nxt.split()[0]
            if op == "s_nop":
                waits += int(nxt.split()[1]) + 1
                continue
            args = nxt.split(None, 1)[1] if " " in nxt else ""
            if op.startswith("v_mfma"):
                ops = [a.strip() for a in args.split(",")]
                if _vregs(ops[0]) == regs and _vregs(ops[3]) == regs and not regs & _vregs(",".join(ops[1:3])):
                    waits += 1
                    continue
            if regs & _vregs(args):
                found.append((i, line, nxt))
                break
            waits += 1
    return found


VALU_WAIT = 2  # wait states between a VALU write of a VGPR and an MFMA reading it as a source


def valu_writes_before_mfma(asm):
    """[(line, mfma, writer)] of inline-assembly MFMAs that read a register (A, B or C) that a VALU instruction wrote
    fewer than VALU_WAIT wait states before. The compiler inserts these waits for its own MFMAs only; without them
    the MFMA reads the register's previous contents."""
    ins = []
    inline = False
    for i, raw in enumerate(asm.splitlines()):
        l = raw.strip()
        if l.startswith(";;#ASMSTART"):
            inline = True
        elif l.startswith(";;#ASMEND"):
            inline = False
        elif l and not l.startswith((";", ".")) and not raw.startswith((".", "_")):
            ins.append((i, l.split(";")[0].strip(), inline))
    found = []
    for k, (i, line, inl) in enumerate(ins):
        if not (inl and line.startswith("v_mfma")):
            continue
        srcs = _vregs(",".join(a.strip() for a in line.split(None, 1)[1].split(",")[1:4]))
        waits = 0
        for _, prev, _ in reversed(ins[max(0, k - VALU_WAIT):k]):
            op = prev.split()[0]
            if op == "s_nop":
                waits += int(prev.split()[1]) + 1
            else:
                if op.startswith("v_") and not op.startswith("v_mfma") and " " in prev:
                    if _vregs(prev.split(None, 1)[1].split(",")[0]) & srcs:
                        found.append((i, line, prev))
                        break
                waits += 1
            if waits >= VALU_WAIT:
                break
    return found


_FUNC = re.compile(r"^[A-Za-z_][\w.$]*:")
_BLOCK = re.compile(r"^\.LBB\d+_\d+:")


_LOOP_HEADER = re.compile(r"=>\s*This (?:Inner )?Loop Header: Depth=\d+")
_IN_LOOP = re.compile(r"in Loop: Header=(BB\d+_\d+) Depth=\d+")
_PARENT_LOOP = re.compile(r"Parent Loop (BB\d+_\d+) Depth=\d+")


def _loop_blocks(asm):
    """[(function, blocks, MFMA loops)] of an assembly listing: each block as a dict (name, innermost loop, scratch
    accesses), and the loops that issue MFMAs in their own blocks with no loop inside them that does (a tile loop,
    whatever small loops it holds). From the compiler's loop annotations: a block heading a loop is marked `=> This
    [Inner] Loop Header`, a nested one after `Parent Loop BBf_n` lines from the outermost loop in, and the other blocks
    of a loop `in Loop: Header=BBf_n` after the innermost loop holding them."""
    out = []

    def close(fn, blocks):
        parent = {b["name"][2:]: b["parent"] for b in blocks if b["head"]}
        mfma = {b["loop"] for b in blocks if b["mfma"] and b["loop"]}
        nested = set()
        for loop in mfma:  # a loop holding an MFMA loop is not one itself
            up = parent.get(loop)
            while up:
                nested.add(up)
                up = parent.get(up)
        out.append((fn, blocks, mfma - nested))

    def block(name):
        return {"name": name, "loop": None, "head": False, "parent": None, "mfma": False, "scratch": []}

    fn, blocks, cur = None, [], None
    for raw in asm.splitlines():
        l = raw.strip()
        if _FUNC.match(raw):
            if fn is not None:
                close(fn, blocks)
            fn = raw.split(":")[0]
            cur = block("entry")
            blocks = [cur]
            continue
        if cur is None:
            continue
        if _BLOCK.match(l) or l.startswith("; %bb."):
            cur = block(l.split(":")[0].lstrip("; "))
            blocks.append(cur)
        if _LOOP_HEADER.search(raw):  # heads a loop: its own, inside the last parent marked before (if any)
            cur["parent"], cur["loop"], cur["head"] = cur["parent"] or cur["loop"], cur["name"][2:], True
        elif _PARENT_LOOP.search(raw):
            cur["parent"] = _PARENT_LOOP.search(raw).group(1)
        else:
            m = _IN_LOOP.search(raw)
            if m and cur["loop"] is None:
                cur["loop"] = m.group(1)
        if l.startswith("v_mfma"):
            cur["mfma"] = True
        elif l.startswith("scratch_"):
            cur["scratch"].append(l.split(";")[0].strip())
    if fn is not None:
        close(fn, blocks)
    return out


def mfma_loops(asm):
    """{function: its MFMA loops (header block names)}."""
    return {fn: hot for fn, _, hot in _loop_blocks(asm)}


def spills_in_mfma_loops(asm):
    """[(function, block, instruction)] of scratch accesses in the MFMA loops. Kernels whose register state spills at
    all must keep the spill code off those loops: stored before them and reloaded after, or on an outer loop's path
    (a pass restarted) or in an epilogue, which run once per loop rather than per tile; this check holds them to it."""
    return [(fn, b["name"], x) for fn, blocks, hot in _loop_blocks(asm) for b in blocks if b["loop"] in hot
            for x in b["scratch"]]


def has_inline_mfma(text):
    """Whether a source holds an inline-assembly MFMA, wherever it stands in its assembly string."""
    return re.search(r'asm\s+volatile\s*\(\s*"[^;]*?v_mfma', text) is not None


def _check_inline_mfma(src, verbose, scheduled=False):
    text = open(src).read()
    if not has_inline_mfma(text):
        return
    out = os.path.join(OBJ, os.path.basename(src).replace(".hip", ".gfx.s"))
    if not scheduled:  # (a scheduled build wrote the assembly of the code it embedded)
        _run([hipcc(), *_flags(src), "--cuda-device-only", "-S", src, "-o", out], f"hipcc -S on {src}", verbose)
    asm = open(out).read()
    bad = mfma_hazards(asm)
    if bad:
        lines = "\n".join(f"  {a}: {b}  ->  {c}" for a, b, c in bad[:10])
        raise RuntimeError(f"{src}: MFMA results read within {MFMA_WAIT} wait states:\n{lines}")
    bad = valu_writes_before_mfma(asm)
    if bad:
        lines = "\n".join(f"  {a}: {c}  ->  {b}" for a, b, c in bad[:10])
        raise RuntimeError(f"{src}: MFMA sources written by the VALU within {VALU_WAIT} wait states:\n{lines}")
    spills = spills_in_mfma_loops(asm)
    if spills:
        lines = "\n".join(f"  {f} {b}: {i}" for f, b, i in spills[:10])
        raise RuntimeError(f"{src}: spill code in an MFMA loop:\n{lines}")


def build(jobs=None, verbose=False, only=None):
    """Compile every csrc/*.hip (or only the named ones, reusing the other objects of an earlier build), check the
    inline-MFMA wait states and link the shared library. Returns the library path."""
    os.makedirs(OBJ, exist_ok=True)
    srcs = sorted(os.path.join(CSRC, f) for f in os.listdir(CSRC) if f.endswith(".hip"))
    todo = [s for s in srcs if not only or os.path.basename(s) in only]
    jobs = jobs or min(8, os.cpu_count() or 1, len(srcs))
    with cf.ThreadPoolExecutor(jobs) as ex:
        scheduled = dict(zip(todo, ex.map(lambda s: _compile(s, verbose), todo)))
        list(ex.map(lambda s: _check_inline_mfma(s, verbose, scheduled[s]), todo))
    objs = [os.path.join(OBJ, os.path.basename(s).replace(".hip", ".o")) for s in srcs]
    tmp = LIB + ".tmp"
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs]
    if verbose:
        print(" ".join(cmd), flush=True)
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stdout}\n{r.stderr}")
    os.replace(tmp, LIB)
    return LIB


def main(argv=None):
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--jobs", type=int, default=None)
    ap.add_argument("--verbose", action="store_true")
    ap.add_argument("--only", default="", help="comma-separated sources to recompile (the rest from _build/)")
    a = ap.parse_args(argv)
    print(build(a.jobs, a.verbose, [x for x in a.only.split(",") if x]))


if __name__ == "__main__":
    sys.exit(main())
