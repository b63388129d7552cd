"""The post-RA MFMA/VALU scheduler the prefill build uses (vllm-quantpack_amd/mirsched.py): register parsing, the
dependence rules, that every order it emits respects them, and the build pipeline end to end on a small MFMA kernel
(LLVM MIR after the post-RA scheduler -> reordered -> LLVM's wait-count and hazard passes -> code object)."""
import importlib.util
import os
import random
import re
import shutil
import subprocess

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
PKG = os.path.join(os.path.dirname(HERE), "vllm-quantpack_amd")
_spec = importlib.util.spec_from_file_location("mirsched", os.path.join(PKG, "mirsched.py"))
ms = importlib.util.module_from_spec(_spec)
_spec.loader.exec_module(ms)

MFMA = ("renamable $vgpr{d}_vgpr{d1}_vgpr{d2}_vgpr{d3} = contract V_MFMA_F32_16X16X32_BF16_vgprcd_e64 "
        "$vgpr{a}_vgpr{a1}_vgpr{a2}_vgpr{a3}, $vgpr{b}_vgpr{b1}_vgpr{b2}_vgpr{b3}, "
        "$vgpr{d}_vgpr{d1}_vgpr{d2}_vgpr{d3}, 0, 0, 0, implicit $mode, implicit $exec")


def mfma(d, a, b):
    q = lambda r: {"": r, "1": r + 1, "2": r + 2, "3": r + 3}  # noqa: E731
    kw = {}
    for k, r in (("d", d), ("a", a), ("b", b)):
        kw.update({k + s: v for s, v in q(r).items()})
    return MFMA.format(**kw)


def fma(d, x, y, z):
    return (f"renamable $vgpr{d} = contract nofpexcept V_FMA_F32_e64 0, $vgpr{x}, 0, $vgpr{y}, 0, $vgpr{z}, 0, 0, "
            "implicit $mode, implicit $exec")


def ds_read(d, addr, off):
    return (f"renamable $vgpr{d}_vgpr{d + 1}_vgpr{d + 2}_vgpr{d + 3} = DS_READ_B128_gfx9 renamable $vgpr{addr}, "
            f"{off}, 0, implicit $exec :: (load (s128), addrspace 3)")


def ds_write(addr, v):
    return (f"DS_WRITE_B32_gfx9 renamable $vgpr{addr}, renamable $vgpr{v}, 0, 0, implicit $exec :: "
            "(store (s32), addrspace 3)")


def inline_mfma(acc, a, b, nops=False):
    tail = "\\0A\\09s_nop 7\\0A\\09s_nop 7\\0A\\09s_nop 1" if nops else ""
    return (f'INLINEASM &"v_mfma_f32_16x16x32_bf16 $0, $1, $2, $0{tail}", 33 /* sideeffect isconvergent attdialect */, '
            f"9240586 /* regdef:AReg_128_Align2 */, def renamable $agpr{acc}_agpr{acc + 1}_agpr{acc + 2}_agpr{acc + 3}, "
            f"7929865 /* reguse:VReg_128_Align2 */, renamable $vgpr{a}_vgpr{a + 1}_vgpr{a + 2}_vgpr{a + 3}, "
            f"7929865 /* reguse:VReg_128_Align2 */, renamable $vgpr{b}_vgpr{b + 1}_vgpr{b + 2}_vgpr{b + 3}, "
            f"2147483657 /* reguse tiedto:$0 */, renamable $agpr{acc}_agpr{acc + 1}_agpr{acc + 2}_agpr{acc + 3}"
            "(tied-def 3)")


def test_register_units():
    assert ms.reg_units("$vgpr4_vgpr5_vgpr6_vgpr7") == {"v4", "v5", "v6", "v7"}
    assert ms.reg_units("$agpr200_agpr201") == {"a200", "a201"}
    assert ms.reg_units("$sgpr62_sgpr63") == {"s62", "s63"}
    assert ms.reg_units("$vcc") == {"vcc_lo", "vcc_hi"}
    assert ms.reg_units("$exec_lo") == {"exec_lo"}
    assert ms.reg_units("$m0") == {"m0"} and ms.reg_units("$scc") == {"scc"}
    assert ms.reg_units("$noreg") == set() and ms.reg_units("$mode") == set() and ms.reg_units("$3") == set()


def test_instruction_operands():
    i = ms.Inst(fma(10, 11, 12, 13))
    assert i.defs == {"v10"} and i.uses == {"v11", "v12", "v13", "exec_lo", "exec_hi"}
    assert i.kind == "valu" and not i.mem and not i.term
    i = ms.Inst(mfma(20, 30, 40))
    assert i.kind == "mfma" and i.defs == {f"v{r}" for r in range(20, 24)}
    assert {f"v{r}" for r in range(20, 24)} <= i.uses and {f"v{r}" for r in range(30, 34)} <= i.uses
    i = ms.Inst(inline_mfma(200, 50, 60))
    assert i.kind == "mfma" and i.mfmas == 1 and not i.mem and not i.trailing_waits
    assert i.defs == {f"a{r}" for r in range(200, 204)}
    assert i.uses == ({f"a{r}" for r in range(200, 204)} | {f"v{r}" for r in range(50, 54)} |
                      {f"v{r}" for r in range(60, 64)} | {"exec_lo", "exec_hi"})
    assert ms.Inst(inline_mfma(200, 50, 60, nops=True)).trailing_waits
    i = ms.Inst('INLINEASM &"s_mov_b32 m0, $2\\0A\\09s_nop 0\\0A\\09global_load_lds_dwordx4 $0, $1", 57 /* sideeffect '
                'mayload maystore isconvergent attdialect */, 1835017 /* reguse:VGPR_32 */, killed renamable $vgpr0, '
                '5242889 /* reguse:SGPR_64 */, renamable $sgpr2_sgpr3, 2424841 /* reguse:SReg_32 */, killed renamable '
                '$sgpr7, 12 /* clobber */, implicit-def early-clobber $m0')
    assert i.mem and i.defs == {"m0"} and i.uses == {"v0", "s2", "s3", "s7", "exec_lo", "exec_hi"}
    i = ms.Inst("renamable $sgpr12 = S_ADD_U32 renamable $sgpr73, killed renamable $sgpr10, implicit-def $scc")
    assert i.kind == "salu" and i.defs == {"s12", "scc"} and i.uses == {"s73", "s10"} and not i.mem
    assert ms.Inst("S_BARRIER").mem and ms.Inst("ATOMIC_FENCE 5, 2").mem
    assert ms.Inst("S_CBRANCH_VCCZ %bb.204, implicit killed $vcc").term
    b = ms.Inst("BUNDLE implicit-def $vgpr110_vgpr111_vgpr112_vgpr113, implicit $vgpr241, implicit $exec {\n"
                "  " + ds_read(110, 241, 0) + "\n}")
    assert b.mem and b.kind == "lds" and {f"v{r}" for r in range(110, 114)} <= b.defs and "v241" in b.uses


def _respects(order, original):
    """Every dependence of the original order holds in `order`."""
    pos = {id(x): k for k, x in enumerate(order)}
    preds = ms.dependences([x for x in original if not x.term])
    body = [x for x in original if not x.term]
    for i, p in enumerate(preds):
        for j in p:
            if pos[id(body[j])] >= pos[id(body[i])]:
                return False
    # terminators last, in their order
    terms = [x for x in original if x.term]
    return [x for x in order[len(order) - len(terms):]] == terms


def test_dependences_are_kept():
    block = [ds_read(100, 1, 0), fma(10, 100, 11, 12), mfma(20, 30, 40), fma(11, 10, 12, 13), ds_write(2, 10),
             mfma(20, 31, 41), ds_read(104, 1, 16), fma(12, 104, 13, 14), "S_BARRIER",
             fma(10, 12, 13, 14), "S_CBRANCH_SCC1 %bb.3, implicit $scc"]
    insts = [ms.Inst(t) for t in block]
    order = ms.schedule(insts)
    assert _respects(order, insts)
    pos = {x.text: k for k, x in enumerate(order)}
    # memory order: read, write, read, barrier
    assert pos[block[0]] < pos[block[4]] < pos[block[6]] < pos[block[8]]
    # WAR: v10 is rewritten only after the write and the fma read it
    assert pos[block[9]] > pos[block[3]] and pos[block[9]] > pos[block[4]]


def test_inline_mfma_with_wait_states_stays_last():
    block = [inline_mfma(0, 50, 60), inline_mfma(4, 50, 64), inline_mfma(8, 50, 68, nops=True),
             fma(10, 11, 12, 13), fma(14, 15, 16, 17), inline_mfma(12, 54, 60)]
    insts = [ms.Inst(t) for t in block]
    order = [x.text for x in ms.schedule(insts)]
    last = order.index(block[2])
    assert order.index(block[0]) < last and order.index(block[1]) < last and order.index(block[5]) > last


def test_inline_assembly_stays_on_its_side_of_exec_writes():
    """A lane-masked copy region (s_and_saveexec ... branch): neither an LDS-DMA copy nor an inline MFMA written
    before the EXEC write may move below it (they would run on the narrowed mask)."""
    dma = ('INLINEASM &"s_mov_b32 m0, $2\\0A\\09s_nop 0\\0A\\09global_load_lds_dwordx4 $0, $1", 57 /* sideeffect '
           'mayload maystore isconvergent attdialect */, 1835017 /* reguse:VGPR_32 */, renamable $vgpr219, '
           '5242889 /* reguse:SGPR_64 */, renamable $sgpr52_sgpr53, 2424841 /* reguse:SReg_32 */, renamable $sgpr0, '
           '12 /* clobber */, implicit-def early-clobber $m0')
    save = "$sgpr64_sgpr65 = S_AND_SAVEEXEC_B64 $sgpr68_sgpr69, implicit-def $exec, implicit-def $scc, implicit $exec"
    block = [inline_mfma(0, 50, 60), inline_mfma(4, 50, 64), dma, save, "S_CBRANCH_EXECZ %bb.9, implicit $exec"]
    order = [x.text for x in ms.schedule([ms.Inst(t) for t in block])]
    assert order.index(save) > max(order.index(block[0]), order.index(block[1]), order.index(dma))
    assert "exec_lo" in ms.Inst(inline_mfma(0, 50, 60)).uses


def test_valu_fills_the_mfma_shadow():
    """Two independent MFMAs and two independent FMAs: LLVM-style order MFMA, MFMA, FMA, FMA becomes an interleave."""
    block = [mfma(20, 30, 40), mfma(24, 30, 44), fma(10, 11, 12, 13), fma(14, 15, 16, 17)]
    order = [x.text for x in ms.schedule([ms.Inst(t) for t in block])]
    assert order[0] == block[0] and order[1] in (block[2], block[3]) and block[1] in order[1:3] + order[2:4]
    assert order.index(block[1]) > order.index(block[2]) or order.index(block[1]) > order.index(block[3])


def test_random_blocks_respect_every_dependence():
    rng = random.Random(5)
    for _ in range(200):
        block = []
        for _ in range(rng.randint(3, 40)):
            r = rng.random()
            v = lambda: rng.randrange(8) * 4 + 100  # noqa: E731
            if r < 0.3:
                block.append(mfma(v(), v(), v()))
            elif r < 0.6:
                block.append(fma(rng.randrange(100, 132), rng.randrange(100, 132), rng.randrange(100, 132),
                                 rng.randrange(100, 132)))
            elif r < 0.75:
                block.append(ds_read(v(), rng.randrange(1, 4), 16 * rng.randrange(8)))
            elif r < 0.85:
                block.append(ds_write(rng.randrange(1, 4), rng.randrange(100, 132)))
            elif r < 0.95:
                block.append(inline_mfma(rng.randrange(4) * 4, v(), v(), nops=rng.random() < 0.2))
            else:
                block.append("S_BARRIER")
        block.append("S_BRANCH %bb.7")
        insts = [ms.Inst(t) for t in block]
        order = ms.schedule(insts)
        assert sorted(x.text for x in order) == sorted(block)
        assert _respects(order, insts)
        # every barrier keeps the same instructions on each side
        pos = {id(x): k for k, x in enumerate(order)}
        for b, x in enumerate(insts):
            if x.op == "S_BARRIER":
                assert all(pos[id(y)] < pos[id(x)] for y in insts[:b])
                assert all(pos[id(y)] > pos[id(x)] for y in insts[b + 1:-1])


def test_barrier_is_a_full_fence():
    """Register-only instructions (the scalar adds forming copy addresses, VALU work, MFMAs) stay on their side of a
    barrier in the middle of a block, although no register or memory dependence ties them to it."""
    before = ["renamable $sgpr13 = S_ADD_I32 renamable $sgpr18, killed renamable $sgpr13, implicit-def dead $scc",
              fma(10, 11, 12, 13), mfma(20, 30, 40)]
    after = [mfma(24, 30, 44), fma(14, 15, 16, 17),
             "renamable $sgpr12 = S_ADD_I32 renamable $sgpr18, killed renamable $sgpr12, implicit-def dead $scc"]
    block = before + ["S_BARRIER"] + after + ["S_BRANCH %bb.3"]
    order = [x.text for x in ms.schedule([ms.Inst(t) for t in block])]
    bar = order.index("S_BARRIER")
    assert all(order.index(t) < bar for t in before) and all(order.index(t) > bar for t in after)


MIR = """--- |
  define void @k() {{ ret void }}
...
---
name:            k
body:             |
  bb.0:
    successors: %bb.1

    {a}
    {b}
    {c}
    S_BRANCH %bb.1

  bb.1:
    S_ENDPGM 0
...
"""


def test_schedule_mir_touches_only_mfma_blocks_of_matching_functions():
    text = MIR.format(a=mfma(20, 30, 40), b=mfma(24, 30, 44), c=fma(10, 11, 12, 13))
    out, n = ms.schedule_mir(text, r"^k$")
    assert n == 1
    body = [l.strip() for l in out.splitlines() if l.startswith("    ") and not l.strip().startswith("successors")]
    assert body.index(fma(10, 11, 12, 13)) < body.index(mfma(24, 30, 44))
    assert ms.schedule_mir(text, r"^other$") == (text, 0)


def _tool(name):
    p = os.path.join(os.environ.get("ROCM_PATH", "/opt/rocm"), "llvm", "bin", name)
    return p if os.path.exists(p) else None


KERNEL = r"""
#include <hip/hip_runtime.h>
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
__global__ __launch_bounds__(256) void k(const bf16x8_t *a, const bf16x8_t *b, float *out, const float *x, int n) {
  f32x4_t acc0 = {}, acc1 = {};
  float s = 0.f;
  for (int i = 0; i < n; ++i) {
    acc0 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[i], b[i], acc0, 0, 0, 0);
    acc1 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[i + 1], b[i], acc1, 0, 0, 0);
    s += __builtin_amdgcn_exp2f(x[i * 64 + threadIdx.x]) * 0.5f;
  }
  out[threadIdx.x] = acc0[0] + acc1[1] + s;
}
"""


@pytest.mark.skipif(not (_tool("llc") and shutil.which(os.path.join(os.environ.get("ROCM_PATH", "/opt/rocm"), "bin", "hipcc"))),
                    reason="ROCm llc / hipcc not installed")
def test_pipeline_on_a_small_kernel(tmp_path):
    """hipcc -> LLVM IR -> llc up to the post-RA scheduler -> mirsched -> llc to gfx950 assembly and an object:
    the MIR round trip reproduces LLVM's code exactly when nothing is reordered, and the reordered code assembles
    with the same instructions."""
    src = tmp_path / "k.hip"
    src.write_text(KERNEL)
    hipcc = os.path.join(os.environ.get("ROCM_PATH", "/opt/rocm"), "bin", "hipcc")
    ll, mir = tmp_path / "k.ll", tmp_path / "k.mir"
    subprocess.run([hipcc, "-O3", "--offload-arch=gfx950", "--cuda-device-only", "-S", "-emit-llvm", str(src), "-o",
                    str(ll)], check=True, capture_output=True)
    llc = [_tool("llc"), "-O3", "-mtriple=amdgcn-amd-amdhsa", "-mcpu=gfx950"]
    subprocess.run([*llc, str(ll), "-o", str(tmp_path / "direct.s")], check=True, capture_output=True)
    subprocess.run([*llc, str(ll), "-stop-after=postmisched", "-o", str(mir)], check=True, capture_output=True)
    subprocess.run([*llc, str(mir), "-start-after=postmisched", "-o", str(tmp_path / "round.s")], check=True,
                   capture_output=True)

    def code(p):
        return [l.split(";")[0].strip() for l in open(p) if re.match(r"^\s+[sv]_", l)]

    assert code(tmp_path / "direct.s") == code(tmp_path / "round.s")
    text, n = ms.schedule_mir(mir.read_text(), r"k")
    assert n >= 1
    (tmp_path / "s.mir").write_text(text)
    subprocess.run([*llc, str(tmp_path / "s.mir"), "-start-after=postmisched", "-verify-machineinstrs", "-o",
                    str(tmp_path / "s.s")], check=True, capture_output=True)
    subprocess.run([*llc, str(tmp_path / "s.mir"), "-start-after=postmisched", "-filetype=obj", "-o",
                    str(tmp_path / "s.o")], check=True, capture_output=True)
    mfmas = lambda p: sum(1 for l in code(p) if l.startswith("v_mfma"))  # noqa: E731
    assert mfmas(tmp_path / "s.s") == mfmas(tmp_path / "direct.s") >= 2
