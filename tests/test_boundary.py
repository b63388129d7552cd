"""The drop-in boundary on the CPU: the C-ABI library exports what include/quantpack.h declares, the Python layer keeps
the reference's names, known answers and error behaviour (tests/test_int4_kv.py:13-87, tests/test_k8v4_kv.py:16-51).
No kernel runs here."""
import ctypes
import logging
import os
import re
import sys
import types

import pytest
import torch

from conftest import REPO

LOG = logging.getLogger("test")
HEADER = os.path.join(REPO, "include", "quantpack.h")


def _declared():
    src = open(HEADER).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    return sorted(set(re.findall(r"^\s*(?:const\s+)?\w+\s*\*?\s*(qp_\w+)\s*\(", src, flags=re.M)))


def test_header_declares_the_entry_points():
    assert _declared() == sorted(["qp_unpack_segment", "qp_decode_splitkv", "qp_merge_segments", "qp_prefill",
                                  "qp_prefill_workspace_size", "qp_prefill_i8", "qp_prefill_i8_workspace_size",
                                  "qp_attention", "qp_attention_workspace_size",
                                  "qp_attention_noalloc", "qp_store", "qp_rht", "qp_last_error", "qp_version"])


def test_library_loads_and_exports_every_declared_symbol():
    from vllm_quantpack import _hip
    if not os.path.exists(_hip.LIB_PATH):
        pytest.skip("library not built (python vllm-quantpack_amd/build.py)")
    lib = ctypes.CDLL(_hip.LIB_PATH)
    for name in _declared():
        assert hasattr(lib, name), name
    assert set(_declared()) == set(_hip.SIGNATURES)
    assert _hip.lib().qp_version().decode().startswith("quantpack-hip")


STRUCTS = {"CacheHalf": "qp_cache_half", "PagedCache": "qp_paged_cache", "DecodeArgs": "qp_decode_args",
           "MergeArgs": "qp_merge_args", "PrefillArgs": "qp_prefill_args", "AttentionArgs": "qp_attention_args",
           "StoreArgs": "qp_store_args"}


def test_ctypes_structs_have_the_header_layout(tmp_path):
    """Every ctypes Structure of the binding has the size and field offsets that gcc gives the header's struct."""
    import shutil
    import subprocess

    from vllm_quantpack import _hip
    if shutil.which("gcc") is None:
        pytest.skip("no gcc")
    lines = ['#include <stddef.h>', '#include <stdio.h>', '#include "quantpack.h"', "int main(void) {"]
    for py, c in STRUCTS.items():
        lines.append(f'  printf("{py} size %zu\\n", sizeof({c}));')
        for name, _ in getattr(_hip, py)._fields_:
            lines.append(f'  printf("{py} {name} %zu\\n", offsetof({c}, {name}));')
    lines += ["  return 0;", "}"]
    src = tmp_path / "layout.c"
    src.write_text("\n".join(lines) + "\n")
    exe = tmp_path / "layout"
    subprocess.run(["gcc", "-I", os.path.join(REPO, "include"), str(src), "-o", str(exe)], check=True)
    got = subprocess.run([str(exe)], check=True, capture_output=True, text=True).stdout.split("\n")
    want = []
    for py in STRUCTS:
        T = getattr(_hip, py)
        want.append(f"{py} size {ctypes.sizeof(T)}")
        want += [f"{py} {name} {getattr(T, name).offset}" for name, _ in T._fields_]
    assert got[:-1] == want


@pytest.mark.parametrize("name", list(STRUCTS))
def test_packer_writes_what_ctypes_writes(name):
    """Packer (one struct.pack_into) fills a Structure with the same bytes as setting its fields through ctypes."""
    import random

    from vllm_quantpack import _hip
    T = getattr(_hip, name)
    rnd = random.Random(len(name))
    codes = [c for _, c in _hip._scalars(T)]
    vals = [rnd.getrandbits(63) if c == "Q" else rnd.randrange(-2**62, 2**62) if c == "q"
            else rnd.randrange(-2**31, 2**31) if c == "i" else rnd.choice([0.5, -3.25, 1e-3, 7.0]) for c in codes]
    packed = T()
    _hip.Packer(T).pack(packed, *vals)

    def fill(obj, it):
        for field, ftype in type(obj)._fields_:
            if issubclass(ftype, ctypes.Structure):
                fill(getattr(obj, field), it)
            elif issubclass(ftype, ctypes.Array):
                arr = getattr(obj, field)
                for i in range(len(arr)):
                    arr[i] = next(it)
            else:
                setattr(obj, field, next(it))

    ref = T()
    ctypes.memset(ctypes.byref(ref), 0xAB, ctypes.sizeof(T))   # padding differs; fields must not
    fill(ref, iter(vals))
    for off, code in _hip._scalars(T):
        size = ctypes.sizeof({"Q": ctypes.c_void_p, "q": ctypes.c_int64, "i": ctypes.c_int32, "f": ctypes.c_float}[code])
        assert bytes(packed)[off:off + size] == bytes(ref)[off:off + size], (name, off)


def test_argument_errors_are_reported_without_a_gpu():
    """Validation runs on the host before any launch: a bad call returns QP_ERR_INVALID with a message."""
    from vllm_quantpack import _hip
    if not os.path.exists(_hip.LIB_PATH):
        pytest.skip("library not built")
    cache = _hip.PagedCache()
    args = _hip.DecodeArgs()
    st = _hip.lib().qp_decode_splitkv(cache, args, None)
    assert st == _hip.QP_ERR_INVALID
    assert "null" in _hip.lib().qp_last_error().decode()
    with pytest.raises(ValueError):
        _hip.check(st, "decode")


def test_missing_library_fails_loudly(monkeypatch):
    from vllm_quantpack import _hip
    monkeypatch.setattr(_hip, "_lib", None)
    monkeypatch.setattr(_hip, "LIB_PATH", "/nonexistent/libquantpack_hip.so")
    with pytest.raises(_hip.HipLibraryMissing):
        _hip.lib()


# --------------------------------------------------------------------------------- reference known answers
#
# Sizing and switches of the drop-in, held to the literal values the reference's own tests expect of its functions
# (tests/test_int4_kv.py:23-87). The vLLM hooks themselves (segment-buffer sizing in the metadata builder, the rebinding
# of the int4 module) run on the stand-in vLLM of tests/test_vllm_hooks.py.

# (VLLM_QUANTPACK_INT4_DECODE or None, CUs or SMs, expected decode_tiles): the default tile and warps with segments
# clamp(next_pow2(ceil(units / 4)), 16, 128), and the override's three or four comma-separated values, "auto"
# standing for the default segment count.
DECODE_TILES = [
    (None, 188, (64, 4, 64)), (None, 84, (64, 4, 32)), (None, 36, (64, 4, 16)), (None, 8, (64, 4, 16)),
    (None, 132, (64, 4, 64)), (None, 512, (64, 4, 128)), (None, 256, (64, 4, 64)),
    ("32,8,32", 188, (32, 8, 32)), ("64,4,auto", 84, (64, 4, 32)),
    ("64,4,auto,16", 188, (64, 4, 64, 16)), ("64,4,32,32", 84, (64, 4, 32, 32)),
]


@pytest.mark.parametrize("env,units,want", DECODE_TILES,
                         ids=[f"{e or 'default'}@{u}" for e, u, _ in DECODE_TILES])
def test_decode_tiles_known_answers(monkeypatch, env, units, want):
    from vllm_quantpack.attention import int4_kv
    if env is None:
        monkeypatch.delenv("VLLM_QUANTPACK_INT4_DECODE", raising=False)
    else:
        monkeypatch.setenv("VLLM_QUANTPACK_INT4_DECODE", env)
    assert int4_kv.decode_tiles(units) == want


def test_patch_is_a_no_op_when_switched_off_or_without_vllm(monkeypatch):
    """VLLM_QUANTPACK_INT4_KV=0 turns the patch off; a vLLM without the int4 ops module leaves it undone. Either way
    patch_int4_kv reports False and changes nothing."""
    from vllm_quantpack.attention import int4_kv
    monkeypatch.setenv("VLLM_QUANTPACK_INT4_KV", "0")
    assert int4_kv.patch_int4_kv(LOG) is False
    monkeypatch.delenv("VLLM_QUANTPACK_INT4_KV")
    monkeypatch.setattr(int4_kv, "MODULE", "vllm_quantpack_no_such_module")
    assert int4_kv.patch_int4_kv(LOG) is False


@pytest.mark.parametrize("requested,seqs,heads,sms,want", [(64, 1, 4, 256, 64), (64, 32, 4, 256, 16),
                                                         (64, 256, 8, 256, 1), (16, 1, 4, 256, 16), (64, 12, 4, 256, 43)])
def test_decode_segments_follow_the_batch(requested, seqs, heads, sms, want):
    """The router keeps the caller's segment count for one sequence and lowers it for batches (about 8 workgroups
    per CU), never above the caller's count (the capacity of its segment buffers)."""
    from vllm_quantpack.attention import int4_kv
    assert int4_kv.decode_segments(requested, seqs, heads, sms) == want


def test_cell_is_key_bytes_plus_packed_value_plus_two_scales():
    from vllm_quantpack.attention import k8v4_kv
    assert k8v4_kv.cell_bytes(256, 256) == 392
    assert k8v4_kv.cell_bytes(128, 64) == 168


@pytest.mark.parametrize("layout", ["hnd", "nhd"])
def test_views_cover_the_cell_without_overlap(layout):
    from vllm_quantpack.attention import k8v4_kv
    nb, nkv, bs, hs = 3, 2, 4, 16
    cell = k8v4_kv.cell_bytes(hs, hs)
    if layout == "hnd":
        kv = torch.zeros((nb, nkv, bs, cell), dtype=torch.int8)
    else:
        kv = torch.zeros((nb, bs, nkv, cell), dtype=torch.int8).transpose(1, 2)
    key, value, ks, vs = k8v4_kv.views(kv, hs)
    assert key.shape == (nb, bs, nkv, hs) and key.dtype == torch.int8
    assert value.shape == (nb, bs, nkv, hs // 2) and value.dtype == torch.uint8
    assert ks.shape == vs.shape == (nb, bs, nkv) and ks.dtype == torch.float32
    key.fill_(1)
    ks.view(torch.int32).fill_(0x02020202)
    value.fill_(3)
    vs.view(torch.int32).fill_(0x04040404)
    want = torch.tensor([1] * hs + [2] * 4 + [3] * (hs // 2) + [4] * 4, dtype=torch.int8)
    assert (kv == want).all()
    ks[1, 2, 1] = 7.0
    assert kv[1, 1, 2, hs:hs + 4].view(torch.float32).item() == 7.0


def test_views_reject_another_cell_size():
    from vllm_quantpack.attention import k8v4_kv
    with pytest.raises(ValueError, match="expected 392"):
        k8v4_kv.views(torch.zeros((1, 4, 16, 264), dtype=torch.int8), 256)


def test_int4_cache_views_are_not_taken_for_k8v4():
    from vllm_quantpack.attention import k8v4_kv
    assert not k8v4_kv.is_k8v4(torch.zeros(1, dtype=torch.uint8))
    assert k8v4_kv.is_k8v4(torch.zeros(1, dtype=torch.int8))


def test_int4_views_match_the_reference_test_layout():
    """tests/test_int4_kv.py:95-103: kc/vc (blocks, bs, nkv, hs/2 + 4) uint8 slices, fp32 scales at hs/2 and at
    hs + 4 + hs/2 within each cell."""
    from vllm_quantpack.attention import k8v4_kv
    nb, nkv, bs, hs = 2, 4, 16, 256
    kv = torch.zeros((nb, nkv, bs, hs + 8), dtype=torch.uint8)
    kc, vc, ks, vs = k8v4_kv.int4_views(kv, hs)
    assert kc.shape == vc.shape == (nb, bs, nkv, hs // 2 + 4)
    assert kc.stride() == (nkv * bs * (hs + 8), hs + 8, bs * (hs + 8), 1)
    ks[1, 3, 2] = 5.0
    vs[1, 3, 2] = 6.0
    assert kv[1, 2, 3, hs // 2:hs // 2 + 4].view(torch.float32).item() == 5.0
    assert kv[1, 2, 3, hs + 4:hs + 8].view(torch.float32).item() == 6.0
    assert vc.storage_offset() == hs // 2 + 4


def test_unsupported_features_raise():
    from vllm_quantpack.attention import int4_kv
    q = torch.zeros((1, 24, 256), dtype=torch.bfloat16)
    with pytest.raises(NotImplementedError, match="sliding window"):
        int4_kv._plain(q, (128, 0), 0.0, None, None, None, None, None)
    with pytest.raises(NotImplementedError, match="softcap"):
        int4_kv._plain(q, (-1, -1), 30.0, None, None, None, None, None)


def _build_module():
    import importlib.util
    spec = importlib.util.spec_from_file_location("qp_build", os.path.join(REPO, "vllm-quantpack_amd", "build.py"))
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def test_inline_mfma_sources_are_scanned():
    """Every source with an inline-assembly MFMA goes through the scan, also when the MFMA is not the first
    instruction of its assembly string (the decode's PV tiles open with the wait states their operands need)."""
    build = _build_module()
    assert build.has_inline_mfma('asm volatile("v_mfma_f32_16x16x32_bf16 %0, %1, %2, %0" : "+a"(x));')
    assert build.has_inline_mfma('asm volatile("s_nop 1\\n\\tv_mfma_f32_16x16x32_bf16 %0, %1, %2, %0" : "+a"(x));')
    assert not build.has_inline_mfma('asm volatile("s_mov_b32 m0, %1\\n\\ts_nop 0" ::"s"(x));\n// v_mfma in a comment')
    csrc = os.path.join(os.path.dirname(build.__file__), "csrc")
    for name in ("qp_decode.hip", "qp_prefill.hip", "qp_prefill_wide.hip"):
        assert build.has_inline_mfma(open(os.path.join(csrc, name)).read()), name


def test_inline_mfma_wait_scan():
    """The build's scan flags a read of an inline-assembly MFMA result inside the wait window and nothing else."""
    scan = _build_module().mfma_hazards
    mfma = "v_mfma_f32_16x16x32_bf16 a[0:3], v[4:7], v[8:11], a[0:3]"
    early = f";;#ASMSTART\n\t{mfma}\n;;#ASMEND\n\tv_accvgpr_read_b32 v1, a2\n"
    assert len(scan(early)) == 1
    waited = f";;#ASMSTART\n\t{mfma}\n\ts_nop 7\n\ts_nop 7\n\ts_nop 1\n;;#ASMEND\n\tv_accvgpr_read_b32 v1, a2\n"
    assert scan(waited) == []
    # an accumulating MFMA on the same registers is ordered by the hardware; one reading them as srcA is not
    chained = f";;#ASMSTART\n\t{mfma}\n\t{mfma}\n\ts_nop 7\n\ts_nop 7\n\ts_nop 1\n;;#ASMEND\n"
    assert scan(chained) == []
    srca = f";;#ASMSTART\n\t{mfma}\n;;#ASMEND\n\tv_mfma_f32_16x16x32_bf16 v[0:3], a[0:3], v[8:11], 0\n"
    assert len(scan(srca)) == 1
    # the compiler's own MFMAs are left to its hazard recognizer
    assert scan("\tv_mfma_f32_16x16x32_bf16 v[0:3], v[4:7], v[8:11], 0\n\tv_mov_b32 v9, v1\n") == []
    # a VGPR destination too
    vdst = ";;#ASMSTART\n\tv_mfma_f32_16x16x32_bf16 v[20:23], v[4:7], v[8:11], v[20:23]\n;;#ASMEND\n\tv_mov_b32 v0, v21\n"
    assert len(scan(vdst)) == 1


def test_valu_write_before_inline_mfma_scan():
    """The build's scan flags an inline-assembly MFMA that reads (as A, B or C) a register a VALU instruction wrote
    fewer than 2 wait states before: the hardware then reads the register's previous contents. Two wait states (an
    s_nop 1, or two other instructions) in between, a load's result, or the compiler's own MFMAs pass."""
    build = _build_module()
    scan = build.valu_writes_before_mfma
    mfma = "v_mfma_f32_32x32x16_bf16 v[0:15], v[148:151], v[140:143], v[0:15]"
    fresh = f"\tv_bitop3_b32 v150, v2, s53, v232 bitop3:0xea\n;;#ASMSTART\n\t{mfma}\n;;#ASMEND\n"
    assert scan(fresh) == [(2, mfma, "v_bitop3_b32 v150, v2, s53, v232 bitop3:0xea")]
    one = f"\tv_cvt_pk_bf16_f32 v143, v1, v2\n\ts_mov_b32 s0, 1\n;;#ASMSTART\n\t{mfma}\n;;#ASMEND\n"
    assert len(scan(one)) == 1
    acc = f"\tv_mov_b32 v3, 0\n;;#ASMSTART\n\t{mfma}\n;;#ASMEND\n"
    assert len(scan(acc)) == 1  # the C operand counts too
    waited = f"\tv_bitop3_b32 v150, v2, s53, v232 bitop3:0xea\n;;#ASMSTART\n\ts_nop 1\n\t{mfma}\n;;#ASMEND\n"
    assert scan(waited) == []
    apart = (f"\tv_bitop3_b32 v150, v2, s53, v232 bitop3:0xea\n\tv_add_u32 v200, v8, v7\n\ts_mov_b32 s0, 1\n"
             f";;#ASMSTART\n\t{mfma}\n;;#ASMEND\n")
    assert scan(apart) == []
    other = f"\tv_bitop3_b32 v152, v2, s53, v232 bitop3:0xea\n;;#ASMSTART\n\t{mfma}\n;;#ASMEND\n"
    assert scan(other) == []
    load = f"\tds_read_b128 v[148:151], v1\n\ts_waitcnt lgkmcnt(0)\n;;#ASMSTART\n\t{mfma}\n;;#ASMEND\n"
    assert scan(load) == []
    assert scan(f"\tv_bitop3_b32 v150, v2, s53, v232 bitop3:0xea\n\t{mfma}\n") == []


def test_spill_scan_flags_scratch_in_mfma_loops():
    """The build fails when spill code runs in a loop that issues MFMAs with no MFMA loop inside it (the tile loop);
    spills stored before it and reloaded after, in an outer loop around it (a pass restarted) or in an epilogue that
    issues MFMAs pass. The listings follow the compiler's loop annotations."""
    build = _build_module()
    scan = build.spills_in_mfma_loops
    mfma = "\tv_mfma_f32_16x16x32_bf16 v[0:3], v[4:7], v[8:11], 0\n"
    spill = "\tscratch_load_dword v5, off, off ; Reload\n"
    hot = (f"kern:\n.LBB0_1:                                ; =>This Inner Loop Header: Depth=1\n{mfma}"
           f"\ts_cbranch_scc1 .LBB0_2\n; %bb.2:                                ; in Loop: Header=BB0_1 Depth=1\n{spill}"
           "\ts_branch .LBB0_1\n")
    assert scan(hot) == [("kern", "%bb.2", "scratch_load_dword v5, off, off")]
    cold = (f"kern:\n\tscratch_store_dword off, v5, off\n.LBB0_1:                                ; =>This Inner Loop "
            f"Header: Depth=1\n{mfma}\ts_cbranch_scc1 .LBB0_1\n.LBB0_2:\n{mfma}{spill}")
    assert scan(cold) == []
    # a pass loop (depth 1) around the tile loop (depth 2): its own MFMAs and spills are once per pass
    nested = (f"kern:\n.LBB0_1:                                ; =>This Loop Header: Depth=1\n{mfma}{spill}"
              f".LBB0_2:                                ;   Parent Loop BB0_1 Depth=1\n"
              f"                                        ; =>  This Inner Loop Header: Depth=2\n{mfma}"
              "\ts_cbranch_scc1 .LBB0_2\n; %bb.3:                                ; in Loop: Header=BB0_1 Depth=1\n"
              f"{spill}\ts_branch .LBB0_1\n")
    assert scan(nested) == []
    assert build.mfma_loops(nested) == {"kern": {"BB0_2"}}
    # a tile loop holding a small loop without MFMAs (a gather) is still the MFMA loop
    gather = (f"kern:\n.LBB0_1:                                ; =>This Loop Header: Depth=1\n{mfma}{spill}"
              ".LBB0_2:                                ;   Parent Loop BB0_1 Depth=1\n"
              "                                        ; =>  This Inner Loop Header: Depth=2\n"
              "\ts_cbranch_scc1 .LBB0_2\n")
    assert scan(gather) == [("kern", ".LBB0_1", "scratch_load_dword v5, off, off")]
    # a new function resets the block state
    two = f"k1:\n.LBB0_1:                                ; =>This Inner Loop Header: Depth=1\n{mfma}k2:\n{spill}"
    assert scan(two) == []


def test_built_kernels_keep_spills_off_the_mfma_loops():
    """Every kernel source with MFMAs, compiled as the build does, has an MFMA loop in each of its MFMA kernels, no
    spill code in one, and the wait states its inline MFMAs need."""
    import shutil
    build = _build_module()
    if shutil.which(build.hipcc()) is None and not os.path.exists(build.hipcc()):
        pytest.skip("no hipcc")
    asm = os.path.join(build.OBJ, "qp_prefill_wide.gfx.s")
    if not os.path.exists(asm):
        pytest.skip("not built")
    for name in ("qp_decode", "qp_prefill", "qp_prefill_wide"):
        text = open(os.path.join(build.OBJ, f"{name}.gfx.s")).read()
        assert "v_mfma" in text
        assert build.spills_in_mfma_loops(text) == [], name
        assert build.mfma_hazards(text) == [], name
        assert build.valu_writes_before_mfma(text) == [], name
        loops = build.mfma_loops(text)
        kernels = [fn for fn in loops if "decode_" in fn or "prefill_" in fn]
        assert kernels, name
        assert all(loops[fn] for fn in kernels), [fn for fn in kernels if not loops[fn]]
