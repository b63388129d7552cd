"""The committed golden fixture tests/golden/int4_small.npz (written by tests/golden/make_fixtures.py from the oracle):
the oracle must still reproduce it exactly (CPU), and the HIP kernels must meet it (GPU) without recomputing anything:
bit-exact unpack and store, decode and prefill within 1e-2 of the emulation and 5e-3 of fp64."""
import os

import numpy as np
import pytest

from conftest import REPO
from qp_testlib import assert_emulation

PATH = os.path.join(REPO, "tests", "golden", "int4_small.npz")
NQ, NKV, HS, BS = 24, 4, 256, 16


def _load():
    return dict(np.load(PATH))


def test_oracle_reproduces_the_fixture():
    import importlib.util
    spec = importlib.util.spec_from_file_location("make_fixtures", os.path.join(REPO, "tests", "golden",
                                                                                "make_fixtures.py"))
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    now, saved = mod.build(), _load()
    assert sorted(now) == sorted(saved)
    for k in saved:
        assert np.array_equal(np.asarray(now[k]), saved[k]), k


def _device_case(device):
    from oracle import qp_oracle as O
    from qp_testlib import i32, torch_cache
    f = _load()
    kv = f["cache"]
    _, views = torch_cache(kv, HS, "int4", device)
    table = i32(f["table"][None], device)
    return f, views, table, O


@pytest.mark.gpu
def test_golden_decode(device):
    from qp_testlib import bf16_tensor, i32, run_decode
    f, views, table, O = _device_case(device)
    q = bf16_tensor(f["q_decode"], device)
    T, n = q.shape[0], int(f["n"])
    out, _ = run_decode(views, q, i32([0, T], device), i32([n], device), table, T, float(f["scale"]),
                        int(f["decode_segments"]), device)
    assert_emulation(out, f["decode_emu"].astype(np.float32))
    assert O.relerr(out, f["decode_ref"].astype(np.float32)) < 5e-3


@pytest.mark.gpu
def test_golden_prefill(device):
    import torch

    from qp_testlib import bf16_tensor, i32, to_f32
    from vllm_quantpack.attention import int4_prefill
    f, (kc, vc, ks, vs), table, O = _device_case(device)
    q = bf16_tensor(f["q_prefill"], device)
    T, n = q.shape[0], int(f["n"])
    out = torch.full_like(q, float("nan"))
    int4_prefill.prefill_attention(q, kc, vc, ks, vs, out, cu_seqlens_q=i32([0, T], device),
                                   seqused_k=i32([n], device), block_table=table, max_seqlen_q=T,
                                   softmax_scale=float(f["scale"]))
    torch.cuda.synchronize()
    got = to_f32(out)
    assert_emulation(got, f["prefill_emu"].astype(np.float32))
    assert O.relerr(got, f["prefill_ref"].astype(np.float32)) < 5e-3


@pytest.mark.gpu
def test_golden_unpack(device):
    import torch

    from vllm_quantpack.attention import int4_prefill
    f, (kc, vc, ks, vs), table, O = _device_case(device)
    start = int(f["unpack_start"])
    for cache, scales, key in ((kc, ks, "unpack_key"), (vc, vs, "unpack_value")):
        out = torch.empty((16, NKV, HS), dtype=torch.bfloat16, device=device)
        int4_prefill.unpack_segment(cache, scales, table[0], start, 16, out)
        torch.cuda.synchronize()
        assert np.array_equal(out.view(torch.int16).cpu().numpy().view(np.uint16), f[key]), key


@pytest.mark.gpu
def test_golden_store(device):
    import torch

    from oracle import qp_oracle as O
    from qp_testlib import bf16_tensor, torch_cache
    from vllm_quantpack.attention import k8v4_kv
    f = _load()
    fresh = O.new_cache(2, NKV, BS, O.int4_cell_bytes(HS))
    t, (kc, vc, ks, vs) = torch_cache(fresh, HS, "int4", device)
    slots = torch.as_tensor(f["store_slots"], device=device)
    k8v4_kv.store(None, bf16_tensor(f["store_key"], device), bf16_tensor(f["store_value"], device), kc, vc, slots,
                  k_scale_cache=ks, v_scale_cache=vs, rotate=False)
    torch.cuda.synchronize()
    assert np.array_equal(t.cpu().numpy(), f["store_cells"])
