"""CPU oracle for the HEX fused-MoE path. TEST INFRASTRUCTURE ONLY.

Only `tests/`, `__graft_entry__.smoke()` and the `cpu_baseline` leg of `bench.py` import this
package, and only as the checker (or as the timed CPU baseline). The product package under
`blackhole-harness_amd/` never imports it and has no CPU fallback through it.

`oracle.hex_oracle` restates, in numpy, the reference's algorithms for this path; every function
cites the reference file:line it follows (paths relative to the reference checkout). See the module
docstring there for what pins each function.
"""
