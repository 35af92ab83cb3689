"""CPU oracle for the FlashUMA ZeroAllocBackbone hot path — TEST INFRASTRUCTURE ONLY.

This package restates the reference algorithm (ArcelliEmanuele/flash-uma: model.py,
wrapper.py, ops/*.py) on the CPU so that the HIP kernels can be checked against it:
  - graph.py   : Morton reorder, receiver/sender CSR, brute-force neighbour list (numpy,
                 integer/bit-exact work);
  - ops_ref.py : the per-edge / per-node float kernels (torch CPU, float64 or float32);
                 backward passes come from torch autograd of these restatements;
  - model_ref.py: the whole backbone + energy/force/stress head on the CPU.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import this
package, and only as the checker (or the timed CPU baseline).  The product path
(flash-uma_amd/) never imports it: it runs the HIP library or raises.

Parity pins (what each function is checked against besides the HIP path) are listed in
each module's docstring.  The FAIRChem node modules in model_ref.py, whose code is absent
from the reference tree, are pinned by tests/test_oracle_node_pins.py (library routines
they reduce to, known answers, equivariance).
"""
