"""Test infrastructure: the CPU oracle for the PSGD-Kron hot path. Imported only by tests/, __graft_entry__.smoke()
and bench.py's cpu_baseline leg."""
