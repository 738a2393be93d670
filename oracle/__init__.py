"""Test infrastructure only: the CPU oracle for the reduction + topk path.

Importable only from tests/, __graft_entry__.smoke() and bench.py's
cpu_baseline leg.  The product package (tensorplay_amd) never imports it.
"""
