"""CPU oracle for the MI355X hot path — TEST INFRASTRUCTURE ONLY.

A restatement, in numpy (and, for the model-level CPU baseline, PyTorch CPU
eager, which is the reference's own ground truth and benchmark baseline), of
what the reference computes on its hot path.  Every function cites the
reference file:line it follows.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
import this package, and only as the checker or the timed CPU baseline.  The
product (applegpu-runtime_amd/) never imports it: with the HIP library
missing, the product raises instead of falling back to the CPU.

Pinning: each function is checked in tests/test_oracle.py against the
reference's own known answers (committed in tests/golden/), against PyTorch
CPU (the reference's parity oracle, torch 2.10 as pinned in its uv.lock) and
against closed forms / brute force.  See tests/test_oracle.py for which check
pins which function.
"""
