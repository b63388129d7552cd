"""The split-KV merge (qp_merge_segments) on synthetic partials, against the oracle's merge (merge_partials,
merge_lse) and rotation (rht).

The library merges at most 16 segments with one wave per row and more with a workgroup per row, and rotates the
merged row back in registers up to head 256 and in LDS above; the cases cover every head size of both kernels, with
and without the rotation, with empty segments (m = -inf, partial rows never written: NaN here) and segments past the
context (garbage statistics that must be ignored), and output rows that are not 4-byte aligned.
"""
import numpy as np
import pytest

from oracle import qp_oracle as O
from qp_testlib import i32, to_f32

pytestmark = pytest.mark.gpu

TILE = 32          # keys per decode chunk: the segment rule's granularity


def _partials(rng, lens, nq, S, hs):
    """Random (acc, m, l) of every segment-buffer row, with empty and past-context segments, and the oracle's merged
    rows and LSE."""
    rows = sum(T for T, _ in lens)
    acc = rng.standard_normal((rows, nq, S, hs)).astype(np.float32)
    m = (rng.standard_normal((rows, nq, S)) * 6).astype(np.float32)
    l_ = rng.uniform(0.5, 40.0, (rows, nq, S)).astype(np.float32)
    want = np.empty((rows, nq, hs), np.float32)
    want_lse = np.empty((rows, nq), np.float32)
    r = 0
    for T, n in lens:
        seg = O.segment_length(n, S, TILE)
        active = min(S, -(-n // seg))
        for _ in range(T):
            empty = rng.random((nq, S)) < 0.25
            for h in range(nq):                            # every row keeps at least one active segment
                if empty[h, :active].all():
                    empty[h, rng.integers(active)] = False
            m[r][empty] = -np.inf
            l_[r][empty] = 0.0
            acc[r][empty] = np.nan                         # never written by the decode
            mm = m[r].copy()
            mm[:, active:] = -np.inf                        # past the context: read, then ignored
            aa = np.where(np.isneginf(mm)[..., None], np.float32(0), acc[r])
            ll = np.where(np.isneginf(mm), np.float32(0), l_[r])
            want[r] = O.merge_partials(aa, mm, ll)
            want_lse[r] = O.merge_lse(mm, ll)
            m[r][:, active:] = rng.uniform(50, 90, (nq, S - active))   # larger than any real maximum
            r += 1
    return acc, m, l_, want, want_lse


@pytest.mark.parametrize("hs", [32, 64, 128, 256, 512, 1024])
@pytest.mark.parametrize("S", [1, 7, 16, 17, 64])
@pytest.mark.parametrize("rotate", [False, True], ids=["plain", "rotated"])
def test_merge_matches_the_oracle(device, hs, S, rotate):
    import torch

    from vllm_quantpack import _hip
    from vllm_quantpack.attention import rht
    print(f"merge hs={hs} segments={S} rotate={rotate}", flush=True)
    rng = np.random.default_rng(hs * 131 + S * 7 + rotate)
    nq = 3
    lens = [(1, 40), (3, 5000), (2, 1 + S * TILE * 3)]
    acc, m, l_, want, want_lse = _partials(rng, lens, nq, S, hs)
    rows = acc.shape[0]
    so, sm, ss = (torch.from_numpy(x).to(device) for x in (acc, m, l_))
    cu = np.concatenate(([0], np.cumsum([T for T, _ in lens]))).astype(np.int32)
    cu_t, used_t = i32(cu, device), i32([n for _, n in lens], device)
    wide = torch.full((rows, nq, hs + 3), float("nan"), dtype=torch.bfloat16, device=device)
    out = wide[:, :, 1:hs + 1]                       # rows start 2 bytes off a 4-byte boundary
    lse = torch.full((rows, nq), float("nan"), dtype=torch.float32, device=device)
    signs = rht.signs(hs, device) if rotate else None
    args = _hip.MergeArgs(so.data_ptr(), _hip.I64x3(*so.stride()[:3]), sm.data_ptr(), ss.data_ptr(),
                          _hip.I64x2(sm.stride(0), sm.stride(1)), cu_t.data_ptr(), used_t.data_ptr(), len(lens), rows,
                          nq, hs, S, out.data_ptr(), _hip.I64x2(out.stride(0), out.stride(1)), lse.data_ptr(),
                          _hip.I64x2(lse.stride(0), lse.stride(1)), _hip.ptr(signs), 1.0 / hs)
    _hip.check(_hip.lib().qp_merge_segments(args, _hip.stream_of(out)), "merge")
    torch.cuda.synchronize()
    got = to_f32(out)
    if rotate:
        want = (O.rht(want, inverse=True) / hs).astype(np.float32)
    assert np.isfinite(got).all()
    assert O.max_row_relerr(got, want) < 4e-3
    assert (np.abs(got - want) <= np.abs(want) * 2.0 ** -7 + 1e-3 * np.abs(want).max()).all()
    assert np.isnan(to_f32(wide[:, :, 0])).all() and np.isnan(to_f32(wide[:, :, hs + 1:])).all()
    assert np.abs(to_f32(lse) - want_lse).max() < 1e-4


def test_merge_rotation_agrees_with_rotating_afterwards(device):
    """The merge's fused inverse rotation, in registers (head 256, one wave per row at 8 segments, a workgroup per row
    at 64) and in LDS (head 512), equals merging plainly and then rotating with single_rht, to bf16 rounding."""
    import torch

    from vllm_quantpack import _hip
    from vllm_quantpack.attention import rht
    for hs, S in ((256, 8), (256, 64), (512, 8), (512, 64)):
        rng = np.random.default_rng(hs + S)
        nq, lens = 2, [(2, 3000), (1, 700)]
        acc, m, l_, _, _ = _partials(rng, lens, nq, S, hs)
        rows = acc.shape[0]
        so, sm, ss = (torch.from_numpy(x).to(device) for x in (acc, m, l_))
        cu_t = i32(np.concatenate(([0], np.cumsum([T for T, _ in lens]))), device)
        used_t = i32([n for _, n in lens], device)
        outs = []
        for signs in (None, rht.signs(hs, device)):
            out = torch.empty((rows, nq, hs), dtype=torch.bfloat16, device=device)
            args = _hip.MergeArgs(so.data_ptr(), _hip.I64x3(*so.stride()[:3]), sm.data_ptr(), ss.data_ptr(),
                                  _hip.I64x2(sm.stride(0), sm.stride(1)), cu_t.data_ptr(), used_t.data_ptr(),
                                  len(lens), rows, nq, hs, S, out.data_ptr(), _hip.I64x2(out.stride(0), out.stride(1)),
                                  None, _hip.I64x2(0, 0), _hip.ptr(signs), 1.0 / hs)
            _hip.check(_hip.lib().qp_merge_segments(args, _hip.stream_of(out)), "merge")
            outs.append(out)
        after = rht.single_rht(outs[0].float(), inverse=True, out_scale=1.0 / hs)
        torch.cuda.synchronize()
        assert O.max_row_relerr(to_f32(outs[1]), to_f32(after)) < 8e-3, (hs, S)
