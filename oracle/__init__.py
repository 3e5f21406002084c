"""CPU oracle for the causal GQA attention hot path.

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and the
CPU-baseline leg of bench.py, always as the checker.  The product package
(tinytrain_amd) never imports it.
"""
