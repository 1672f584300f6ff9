"""CPU oracle for the qwen36 kernel nodes.

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and bench.py's
cpu_baseline leg as the checker.  The product package (bundles_amd) never imports it.
"""
