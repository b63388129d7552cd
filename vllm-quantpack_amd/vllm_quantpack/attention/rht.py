"""Randomized Hadamard rotation of the int4 / k8v4 cache domain, on the HIP library.

R = H D with H the Sylvester Hadamard matrix of the head size and D a fixed +/-1 diagonal, unnormalised:
R R^T = head_size * I. Keys and values are stored rotated (k8v4_kv.py:71-72), queries are rotated before attention and
outputs rotated back with R^T / head_size (int4_kv.py:326-329), so <R q, R k> = head_size * <q, k> and the kernels
take softmax_scale / head_size.

The sign of channel c is bit 0 of the `lowbias32` integer hash (C. Wellons) of c + seed * 0x9E3779B9 (mod 2^32).
vLLM's own sign vector is not part of the reference; a cache written by this package's store is read by this
package's attention, which is the pairing that matters.
"""
from __future__ import annotations

import numpy as np
import torch

from .. import _hip

_SIGNS: dict = {}


def signs_np(head_size: int, seed: int = 0) -> np.ndarray:
    x = (np.arange(head_size, dtype=np.uint64) + np.uint64(seed) * np.uint64(0x9E3779B9)) & np.uint64(0xFFFFFFFF)
    x ^= x >> np.uint64(16)
    x = (x * np.uint64(0x7FEB352D)) & np.uint64(0xFFFFFFFF)
    x ^= x >> np.uint64(15)
    x = (x * np.uint64(0x846CA68B)) & np.uint64(0xFFFFFFFF)
    x ^= x >> np.uint64(16)
    return np.where(x & np.uint64(1), -1.0, 1.0).astype(np.float32)


def _signs_on(head_size: int, device: torch.device, seed: int) -> torch.Tensor:
    """signs_np computed by kernels on `device` (an arange and integer arithmetic), so that no host buffer is copied
    and the host never waits: the int64 products keep their low 32 bits exact, which is all the hash uses."""
    x = (torch.arange(head_size, dtype=torch.int64, device=device) + seed * 0x9E3779B9) & 0xFFFFFFFF
    x = x ^ (x >> 16)
    x = (x * 0x7FEB352D) & 0xFFFFFFFF
    x = x ^ (x >> 15)
    x = (x * 0x846CA68B) & 0xFFFFFFFF
    x = x ^ (x >> 16)
    return 1.0 - 2.0 * (x & 1).to(torch.float32)


def signs(head_size: int, device, seed: int = 0) -> torch.Tensor:
    """The diagonal D as an fp32 device tensor, cached per device, head size and seed. Made on the device without a
    host copy; inside a HIP-graph capture only a cached tensor can be returned (kernels recorded there would not run
    before the capture ends), so callers that capture create it first (patch_int4_kv does, for the usual head
    sizes)."""
    device = torch.device(device)
    if device.type == "cuda" and device.index is None:
        device = torch.device("cuda", torch.cuda.current_device())
    key = (device, head_size, seed)
    t = _SIGNS.get(key)
    if t is None:
        if device.type == "cuda" and torch.cuda.is_current_stream_capturing():
            raise RuntimeError(f"rht.signs({head_size}) first requested during a HIP-graph capture: create it before "
                               "capturing (vllm_quantpack.attention.rht.signs or patch_int4_kv)")
        t = _signs_on(head_size, device, seed)
        _SIGNS[key] = t
    return t


def single_rht(x: torch.Tensor, inverse: bool = False, *, out_dtype=None, out_scale: float = 1.0,
               seed: int = 0) -> torch.Tensor:
    """Rows of x (last dim = head size) rotated: x D H (forward) or x H D (inverse, unnormalised), times out_scale.
    bf16 or fp32 in; the result has x's dtype unless out_dtype says otherwise. Stands in for vLLM's `single_rht`
    (called at int4_kv.py:326,329 and k8v4_kv.py:71-72)."""
    if x.dtype not in (torch.bfloat16, torch.float32):
        raise ValueError(f"single_rht: bf16 or fp32 input, got {x.dtype}")
    out_dtype = x.dtype if out_dtype is None else out_dtype
    hs = x.shape[-1]
    rows = x.reshape(-1, hs)
    if rows.stride(-1) != 1:
        rows = rows.contiguous()
    out = torch.empty(rows.shape, dtype=out_dtype, device=x.device)
    dt = {torch.bfloat16: _hip.DTYPE_BF16, torch.float32: _hip.DTYPE_F32}
    _hip.check(_hip.lib().qp_rht(_hip.ptr(rows), dt[x.dtype], rows.stride(0), _hip.ptr(out), dt[out_dtype],
                                 out.stride(0), rows.shape[0], hs, _hip.ptr(signs(hs, x.device, seed)),
                                 int(inverse), float(out_scale), _hip.stream_of(x)), "single_rht")
    return out.reshape(x.shape)
