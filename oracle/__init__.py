"""CPU oracle for the ParaRNN fused Newton + scan path — TEST INFRASTRUCTURE ONLY.

This package restates, in plain PyTorch on the CPU, the reference's *eager*
algorithm for the two Jacobian classes of the hot path:

* ParaSLSTM ``mix='diag'`` (per-channel 4x4 ``block4`` Jacobian): cell step,
  analytic Jacobian, frozen-gate / Picard warm start, eager Newton loop with a
  Blelloch scan on the affine monoid.
* ParaGRU ``mix='head'`` (block-diagonal 64x64 Jacobian): cell step, dense
  per-head Jacobian, App. A initial guess, eager Newton with the dense
  Blelloch scan.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s CPU-baseline
leg may import this package, and only as the checker.  The shipped package
(``pararnn-torch_amd/pararnn_amd``) never imports it: its Newton path runs the
HIP kernels and fails loudly when they are missing.

Every function cites the reference file:line it restates (paths relative to
the reference's ``src/pararnn``).  Op order follows the reference wherever it
changes rounding (bf16 tensors round after every torch op on the CPU), so the
oracle reproduces the reference's eager outputs bit-for-bit on the committed
golden vectors.

Pinning (see tests/test_oracle.py):
* golden vectors written from the reference (tests/golden/make_golden.py);
* Jacobians against float64 autograd of the oracle's own step;
* scans against a brute-force sequential recurrence;
* Newton against the sequential unroll (its fixed point);
* the R = 0 special case, where the frozen-gate scan is exact.
"""

from oracle.scan import (  # noqa: F401
    blelloch_inclusive,
    scan_block4,
    scan_dense,
    scan_diag,
    sequential_affine,
)
from oracle.slstm import (  # noqa: F401
    SLSTMParams,
    auto_picard,
    frozen_gate_scan,
    picard_init,
    slstm_jacobian,
    slstm_newton,
    slstm_sequential,
    slstm_step,
)
from oracle.gru_head import (  # noqa: F401
    GRUHeadParams,
    gru_head_jacobian,
    gru_head_newton,
    gru_head_sequential,
    gru_head_step,
)
