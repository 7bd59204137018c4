"""CPU oracle for the dynamic short-convolution hot path.

TEST INFRASTRUCTURE ONLY.  Nothing in the product path (the `dynconv`
package, the HIP library) may import this package.  It is imported by
`tests/`, by `__graft_entry__.smoke()` and by the `cpu_baseline` leg of
`bench.py`, and there only as the checker / the CPU baseline.

Modules:
  reference_cpu  fp32 torch restatement of the reference algorithm
                 (reference.py:5-39), differentiable through autograd.
  brute          float64 numpy index loops: an independent formulation
                 used to pin `reference_cpu` on tiny shapes, with
                 hand-derived gradient formulas.

Parity status of each oracle function (what pins it) is listed in the
module docstrings; no function is "parity unpinned".
"""

from .reference_cpu import (  # noqa: F401
    headwise_dynamic_convolution_ref,
    lowrank_dynamic_convolution_ref,
    lowrank_weights_ref,
)
