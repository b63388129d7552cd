"""The per-layer timing tool `vllm_quantpack.tools.int4_kv_bench` (the reference's tools/int4_kv_bench.py, tested at
tests/test_int4_kv.py:342-347): its command line on the CPU, its fp64 dequantisation against the oracle's on the CPU,
and one short run on the MI355X whose every line stays within the 1e-2 bar."""
import numpy as np
import pytest

from oracle import qp_oracle as O
from qp_testlib import torch_cache


def test_bench_tool_help(capsys):
    from vllm_quantpack.tools import int4_kv_bench
    with pytest.raises(SystemExit) as e:
        int4_kv_bench.main(["--help"])
    assert e.value.code == 0
    assert "VLLM_QUANTPACK_INT4_DECODE" in capsys.readouterr().out


def test_decode_configs_parse():
    from vllm_quantpack.tools.int4_kv_bench import parse_configs
    assert parse_configs("64,4,16:64,4,auto,16") == [(64, 4, 16), (64, 4, "auto", 16)]
    with pytest.raises(ValueError):
        parse_configs("64,4")


@pytest.mark.parametrize("fmt", ["int4", "int8"])
def test_tool_dequant_matches_the_oracle(fmt):
    from vllm_quantpack.tools import int4_kv_bench, synth
    rng = np.random.default_rng(40)
    nb, nkv, bs, hs, n = 5, 2, 16, 32, 70
    kv = (synth.fill_k8v4_cache if fmt == "int8" else synth.fill_int4_cache)(rng, nb, nkv, bs, hs)
    views = O.k8v4_views(kv, hs) if fmt == "int8" else O.int4_views(kv, hs)
    want_k, want_v = O.dequant_f64(views, np.arange(nb, dtype=np.int32), n)
    _, tviews = torch_cache(kv, hs, fmt, "cpu")
    got_k, got_v = int4_kv_bench._dequant(tviews, n, hs)
    assert np.array_equal(got_k.numpy(), want_k)
    assert np.array_equal(got_v.numpy(), want_v)


def test_max_row_relerr_matches_the_oracle():
    import torch

    from vllm_quantpack.tools.int4_kv_bench import max_row_relerr
    rng = np.random.default_rng(41)
    ref = rng.standard_normal((3, 4, 16))
    o = ref + rng.standard_normal(ref.shape) * 1e-3
    assert abs(max_row_relerr(torch.from_numpy(o), torch.from_numpy(ref)) - O.max_row_relerr(o, ref)) < 1e-12


@pytest.mark.gpu
@pytest.mark.parametrize("fmt", ["int4", "int8"])
def test_bench_tool_short_run(device, fmt):
    from vllm_quantpack.tools import int4_kv_bench
    print(f"int4_kv_bench short run, {fmt} keys", flush=True)
    res = int4_kv_bench.main(["--contexts", "3000,9000", "--decode", "64,4,16:64,4,auto,16", "--head-size", "128",
                              "--block-size", "48", "--key-format", fmt, "--reps", "3"])
    assert [r["kind"] for r in res] == ["decode", "decode", "prefill"] * 2
    for r in res:
        assert r["ms"] > 0
        assert r["relerr"] < 1e-2, r
