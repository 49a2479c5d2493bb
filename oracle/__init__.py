"""CPU ORACLE -- test infrastructure only.

A restatement of the reference's mixed-batch forward on the CPU (oracle.cpp)
and a pin library built from the reference's own quant-core sources
(ref_shim.cpp -> _ref/).  Only tests/, __graft_entry__.smoke() and bench.py's
cpu_baseline leg may load anything here, and only as the checker or the timed
CPU baseline; the product (intfer_amd/) never does.

Functions with no check beyond their own restatement are called "parity
unpinned" in tests/test_oracle.py's header; every other function is pinned
there against the reference library, closed forms or brute force.
"""
