"""The vLLM integration hooks against a stand-in of the vLLM objects they attach to (vLLM is not installed here).

The stand-in has the attributes the reference plugin and this package both rely on (k8v4_kv.py:89-166,
int4_kv.py:190-257): the int4 ops module's globals, the Triton backend's customize_spec / supported dtypes, the
implementation's scale and view methods, the metadata builder's segment constant and the KV-cache dtype registry.
The checks follow the reference's registration test (tests/test_k8v4_kv.py:73-93): k8v4 registered with int8 storage
and the int4 quantisation mode, cells of 264 (int4, unchanged), 392 (k8v4) and 520 (fp8, unchanged) bytes.
"""
import dataclasses
import enum
import logging
import os
import sys
import types

import numpy as np
import pytest
import torch

LOG = logging.getLogger("test")
NKV, HS = 4, 256


def _lib_built():
    from vllm_quantpack import _hip
    return os.path.exists(_hip.LIB_PATH)


@pytest.fixture
def fake_vllm(monkeypatch):
    """Stand-in vLLM modules in sys.modules; every hook installed during the test is undone afterwards."""
    from vllm_quantpack.attention.vllm_hooks import HOOKS

    class KVQuantMode(enum.Enum):
        NONE = 0
        INT4_PER_TOKEN_HEAD = 1
        FP8_PER_TOKEN_HEAD = 2

    @dataclasses.dataclass(frozen=True)
    class FullAttentionSpec:
        block_size: int
        num_kv_heads: int
        head_size: int
        dtype: torch.dtype
        kv_quant_mode: KVQuantMode = KVQuantMode.NONE
        head_size_v: int = None
        state_content_bytes: int = None

        def __post_init__(self):
            if self.head_size_v is None:
                object.__setattr__(self, "head_size_v", self.head_size)

        @property
        def state_content_size_bytes(self):
            return self.state_content_bytes

    handlers = {}

    def register_kv_cache_dtype(name):
        def deco(cls):
            handlers[name] = cls()
            return cls
        return deco

    cache = types.ModuleType("vllm.config.cache")
    cache.register_kv_cache_dtype = register_kv_cache_dtype
    cache.get_kv_cache_dtype_handler = handlers.get
    cache.is_known_kv_cache_dtype = lambda name: name in handlers or name in ("auto", "int4_per_token_head")
    iface = types.ModuleType("vllm.v1.kv_cache_interface")
    iface.KVQuantMode = KVQuantMode
    iface.FullAttentionSpec = FullAttentionSpec

    triton_attn = types.ModuleType("vllm.v1.attention.backends.triton_attn")
    triton_attn.NUM_PAR_SOFTMAX_SEGMENTS = 16

    class TritonAttentionBackend:
        supported_kv_cache_dtypes = ["auto", "int4_per_token_head", "fp8_per_token_head"]

        @classmethod
        def customize_spec(cls, spec):                   # vLLM's own sizes: int4 hs + 8, fp8 2 hs + 8
            per = {KVQuantMode.INT4_PER_TOKEN_HEAD: spec.head_size + 8,
                   KVQuantMode.FP8_PER_TOKEN_HEAD: 2 * spec.head_size + 8}.get(spec.kv_quant_mode)
            return dataclasses.replace(spec, state_content_bytes=per)

        @classmethod
        def supports_kv_cache_dtype(cls, name):
            return name in cls.supported_kv_cache_dtypes

    class TritonAttentionImpl:
        def __init__(self, dtype, head_size=HS):
            self.kv_cache_dtype, self.head_size = dtype, head_size
            self._k_scale_cache = self._v_scale_cache = None

        def _ensure_scale_caches(self, kv_cache):
            self._k_scale_cache = "stock"

        def _pth_key_value_caches(self, kv_cache):
            return "stock", "stock"

    class TritonAttentionMetadataBuilder:
        def __init__(self, kv_cache_spec, layer_names, vllm_config, device):
            self.num_par_softmax_segments = triton_attn.NUM_PAR_SOFTMAX_SEGMENTS

    triton_attn.TritonAttentionBackend = TritonAttentionBackend
    triton_attn.TritonAttentionImpl = TritonAttentionImpl
    triton_attn.TritonAttentionMetadataBuilder = TritonAttentionMetadataBuilder
    ops = types.ModuleType("vllm.v1.attention.ops.int4_per_token_head")
    ops.unified_attention_int4 = lambda *a, **k: "stock attention"
    ops.reshape_and_cache_int4 = lambda *a, **k: "stock store"

    mods = {m.__name__: m for m in (cache, iface, triton_attn, ops)}
    for name in ("vllm", "vllm.config", "vllm.v1", "vllm.v1.attention", "vllm.v1.attention.backends",
                 "vllm.v1.attention.ops"):
        mods[name] = types.ModuleType(name)
    for name, mod in mods.items():
        monkeypatch.setitem(sys.modules, name, mod)
    for name, mod in mods.items():
        parent, _, leaf = name.rpartition(".")
        if parent:
            setattr(mods[parent], leaf, mod)
    yield types.SimpleNamespace(ops=ops, triton_attn=triton_attn, handlers=handlers, Spec=FullAttentionSpec,
                                Mode=KVQuantMode, cache=cache)
    HOOKS.restore()


def test_patch_registers_and_sizes_k8v4(fake_vllm):
    """tests/test_k8v4_kv.py:73-93 on the stand-in: registered, int8 storage, int4 mode, cells 264 / 392 / 520."""
    from vllm_quantpack.attention import int4_kv, k8v4_kv
    if not _lib_built():
        pytest.skip("library not built")
    assert int4_kv.patch_int4_kv(LOG)
    assert fake_vllm.cache.is_known_kv_cache_dtype(k8v4_kv.NAME)
    handler = fake_vllm.handlers[k8v4_kv.NAME]
    assert handler.name == k8v4_kv.NAME and handler.torch_dtype() == torch.int8
    assert handler.quant_mode() == fake_vllm.Mode.INT4_PER_TOKEN_HEAD
    backend = fake_vllm.triton_attn.TritonAttentionBackend
    assert backend.supports_kv_cache_dtype(k8v4_kv.NAME)
    int4 = fake_vllm.Spec(block_size=16, num_kv_heads=NKV, head_size=HS, dtype=torch.uint8,
                          kv_quant_mode=fake_vllm.Mode.INT4_PER_TOKEN_HEAD)
    assert backend.customize_spec(int4).state_content_size_bytes == 264
    k8v4 = dataclasses.replace(int4, dtype=torch.int8)
    assert backend.customize_spec(k8v4).state_content_size_bytes == 392
    fp8 = dataclasses.replace(int4, kv_quant_mode=fake_vllm.Mode.FP8_PER_TOKEN_HEAD)
    assert backend.customize_spec(fp8).state_content_size_bytes == 520
    assert backend.customize_spec(dataclasses.replace(k8v4, head_size_v=128)).state_content_size_bytes == 328


def test_patch_rebinds_the_int4_module_once(fake_vllm):
    from vllm_quantpack.attention import int4_kv
    from vllm_quantpack.attention.vllm_hooks import HOOKS, marked
    if not _lib_built():
        pytest.skip("library not built")
    assert int4_kv.patch_int4_kv(LOG)
    assert fake_vllm.ops.unified_attention_int4 is int4_kv.unified_attention_int4
    assert fake_vllm.ops.reshape_and_cache_int4 is int4_kv.reshape_and_cache_int4
    assert marked(fake_vllm.ops.unified_attention_int4)
    n = len(HOOKS.applied)
    assert int4_kv.patch_int4_kv(LOG)                      # idempotent: nothing is wrapped twice
    assert len(HOOKS.applied) == n
    builder = fake_vllm.triton_attn.TritonAttentionMetadataBuilder
    cfg = lambda d: types.SimpleNamespace(cache_config=types.SimpleNamespace(cache_dtype=d))  # noqa: E731
    want = int4_kv.decode_tiles(0)[2]
    assert builder(None, [], cfg("k8v4_per_token_head"), None).num_par_softmax_segments == want
    assert builder(None, [], cfg("auto"), None).num_par_softmax_segments == 16
    HOOKS.restore()                                        # vLLM exactly as it was
    assert fake_vllm.ops.unified_attention_int4() == "stock attention"
    assert fake_vllm.ops.reshape_and_cache_int4() == "stock store"
    assert builder(None, [], cfg("k8v4_per_token_head"), None).num_par_softmax_segments == 16
    assert "k8v4_per_token_head" not in fake_vllm.triton_attn.TritonAttentionBackend.supported_kv_cache_dtypes


@pytest.mark.parametrize("count,installed", [(64, 64), (128, 128), (48, 0), (96, 0)])
def test_segment_buffers_sized_for_int4_and_k8v4_layers_only(fake_vllm, count, installed):
    """_patch_decode_segments (int4_kv.py:229-257): a power-of-two count becomes the segment count of the metadata
    builder for int4 and k8v4 layers, other dtypes keep vLLM's module constant; any other count is refused (0) and
    the builder stays stock. The module constant itself never changes."""
    from vllm_quantpack.attention import int4_kv
    builder = fake_vllm.triton_attn.TritonAttentionMetadataBuilder
    cfg = lambda d: types.SimpleNamespace(cache_config=types.SimpleNamespace(cache_dtype=d))  # noqa: E731
    assert int4_kv._patch_decode_segments(count, LOG) == installed
    for dtype in ("int4_per_token_head", "k8v4_per_token_head", "auto", "fp8_per_token_head"):
        quantised = dtype in ("int4_per_token_head", "k8v4_per_token_head")
        want = installed if installed and quantised else 16
        assert builder(None, [], cfg(dtype), None).num_par_softmax_segments == want, dtype
    assert fake_vllm.triton_attn.NUM_PAR_SOFTMAX_SEGMENTS == 16


@pytest.mark.parametrize("layout", ["hnd", "nhd"])
def test_backend_hands_out_k8v4_views_and_unit_scales(fake_vllm, layout):
    """A k8v4 layer gets the int8 key / uint8 value views of its byte cache and both scale views at 1.0; a layer of
    another dtype still goes to vLLM's own methods."""
    from vllm_quantpack.attention import k8v4_kv
    assert k8v4_kv.patch_backend(None, LOG)
    impl_cls = fake_vllm.triton_attn.TritonAttentionImpl
    nb, bs = 3, 16
    cell = k8v4_kv.cell_bytes(HS, HS)
    if layout == "hnd":
        kv = torch.zeros((nb, NKV, bs, cell), dtype=torch.int8)
    else:
        kv = torch.zeros((nb, bs, NKV, cell), dtype=torch.int8).transpose(1, 2)
    impl = impl_cls(k8v4_kv.NAME)
    key, value = impl._pth_key_value_caches(kv)
    assert key.dtype == torch.int8 and tuple(key.shape) == (nb, bs, NKV, HS)
    assert value.dtype == torch.uint8 and tuple(value.shape) == (nb, bs, NKV, HS // 2)
    assert (impl._k_scale_cache == 1.0).all() and (impl._v_scale_cache == 1.0).all()
    key[1, 2, 3, 5] = -7                                   # the views alias the cache: cell (1, head 3, slot 2)
    assert int(kv[1, 3, 2, 5]) == -7
    impl._k_scale_cache[1, 2, 3] = 0.5
    assert kv[1, 3, 2, HS:HS + 4].view(torch.float32).item() == 0.5
    first = impl._k_scale_cache
    impl._ensure_scale_caches(kv)
    assert impl._k_scale_cache is first                    # made once
    other = impl_cls("int4_per_token_head")
    assert other._pth_key_value_caches(kv) == ("stock", "stock")
    other._ensure_scale_caches(kv)
    assert other._k_scale_cache == "stock"


def test_registry_absent_leaves_the_dtype_unregistered(monkeypatch):
    from vllm_quantpack.attention import k8v4_kv
    monkeypatch.setitem(sys.modules, "vllm.config.cache", types.ModuleType("vllm.config.cache"))
    assert k8v4_kv.register_dtype(LOG) is False


def test_header_structs_match_the_ctypes_layout(tmp_path):
    """Every struct of include/quantpack.h as the C compiler lays it out (sizeof / offsetof from gcc) against the
    ctypes declarations the Python side passes through the boundary."""
    import re
    import shutil
    import subprocess

    from conftest import REPO
    from vllm_quantpack import _hip
    if shutil.which("gcc") is None:
        pytest.skip("no gcc")
    header = open(os.path.join(REPO, "include", "quantpack.h")).read()
    structs = {"qp_cache_half": _hip.CacheHalf, "qp_paged_cache": _hip.PagedCache, "qp_decode_args": _hip.DecodeArgs,
               "qp_merge_args": _hip.MergeArgs, "qp_prefill_args": _hip.PrefillArgs,
               "qp_attention_args": _hip.AttentionArgs, "qp_store_args": _hip.StoreArgs}
    assert set(re.findall(r"typedef struct (qp_\w+) \{", header)) == set(structs)
    lines = ['#include <stdio.h>', '#include <stddef.h>', '#include "quantpack.h"', "int main(void) {"]
    for cname, py in structs.items():
        lines.append(f'printf("{cname} size %zu\\n", sizeof({cname}));')
        for field, _ in py._fields_:
            lines.append(f'printf("{cname} {field} %zu\\n", offsetof({cname}, {field}));')
    lines.append("return 0; }")
    src = tmp_path / "layout.c"
    src.write_text("\n".join(lines))
    exe = tmp_path / "layout"
    subprocess.run(["gcc", "-I", os.path.join(REPO, "include"), str(src), "-o", str(exe)], check=True)
    got = {}
    for line in subprocess.run([str(exe)], capture_output=True, text=True, check=True).stdout.splitlines():
        cname, field, val = line.split()
        got[(cname, field)] = int(val)
    for cname, py in structs.items():
        assert got[(cname, "size")] == __import__("ctypes").sizeof(py), cname
        for field, _ in py._fields_:
            assert got[(cname, field)] == getattr(py, field).offset, (cname, field)


def test_rht_signs_made_on_the_device_equal_the_hash():
    """The sign vector is built with tensor kernels (no host copy): the same +/-1 vector as the numpy hash."""
    from vllm_quantpack.attention import rht
    for hs in (64, 256, 1024):
        for seed in (0, 7):
            got = rht._signs_on(hs, torch.device("cpu"), seed).numpy()
            assert (got == rht.signs_np(hs, seed)).all()
    assert np.abs(rht.signs(256, "cpu").numpy()).min() == 1.0
