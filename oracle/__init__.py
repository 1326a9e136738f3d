"""CPU oracle of the INT8 DenseNet encoder -- TEST INFRASTRUCTURE ONLY.

Only `tests/`, `__graft_entry__.smoke()` and the `cpu_baseline` leg of `bench.py` may import this
package, and only as the checker (or the timed CPU baseline), never as the thing measured or shipped.
The product (`rsna-knee-efficiency_amd/`) never imports it and has no CPU fallback.

- `lib`       ctypes binding of `d8s_oracle.c` (bit-exact per-pixel restatement of every kernel);
- `fp32`      the float32 DenseNet forward from a state_dict (parity reference and CPU baseline),
              restated from `src/knee/models/densenet.py:27-104`;
- `emulate`   the float64 integer emulation of the whole INT8 pipeline, restated from
              `src/knee/dense8s.py:549-643` (the reference's own CPU path);
- `checks`    comparisons of the HIP kernels with the above, shared by the tests and smoke().

How each function is pinned (closed forms, invariants, brute force, library routines) is tested in
`tests/test_oracle.py`; see the header of each module for the reference lines it follows.
"""
