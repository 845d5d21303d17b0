"""CPU oracle for the Cortex-S inference forward (test infrastructure only).

Imported only by tests/, __graft_entry__.smoke() and the cpu_baseline leg of
bench.py.  The product package never imports it.
"""
