"""CPU oracle for the tensor-op path.  TEST INFRASTRUCTURE: only tests/, __graft_entry__.smoke()
and bench.py's cpu_baseline leg may import it."""
