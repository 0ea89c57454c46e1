"""CPU oracle for the paged-KV attention hot path — test infrastructure only.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
import this package.  The reference is Python + Triton: there is no C or C++
source on this path to compile into oracle/_ref, so the oracle is a numpy /
fp32-torch restatement pinned by the checks in tests/test_oracle.py.
"""
