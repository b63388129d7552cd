"""CPU oracle for the int4 / k8v4 KV-cache attention path (test infrastructure only).

Only `tests/`, `__graft_entry__.smoke()` and the `cpu_baseline` leg of `bench.py` may import this package, and only
as the reference results the HIP kernels are compared with or as the CPU baseline: nothing in `vllm-quantpack_amd/`
imports it, and the product path fails loudly when its HIP library is missing instead of falling back to anything
here.
"""
