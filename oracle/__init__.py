"""CPU oracle for the MoE forward path. TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
import this package, and only as the checker (or, for bench.py, as the timed
CPU baseline): the product path (sparsebench_amd) never imports it and has no
CPU fallback.

    topology_ref  the block-sparse layout (integer work, numpy), restating
                  sparsebench/topology.py:53-118 and the worst-case/past-the-end
                  conventions of csrc/routing.cu:44-51, 125-132, 157-158, 162-193, 248-249; pinned by a
                  brute-force loop version, invariants and known answers.
    moe_ref       fp32/fp64 torch references of the layer and its stages,
                  restating sparsebench/reference.py:49-114 and
                  sparsebench/moe.py:51-54; pinned by a per-token oracle,
                  the loop-vs-block-sparse identity and closed forms.

Every function is pinned by a test in tests/test_oracle_*.py.
"""
