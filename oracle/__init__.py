"""CPU oracle for the quantized-matvec hot path — TEST INFRASTRUCTURE ONLY.

Nothing in the product (`gdsllm_amd/`) imports this package.  Only `tests/`,
`__graft_entry__.smoke()` and the `cpu_baseline` leg of `bench.py` use it, and
only as the checker / the reported CPU baseline, never as the thing measured.
"""
