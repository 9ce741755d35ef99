"""CPU oracle for the Ornith G256 hot path.  Test infrastructure only: used
by tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg as the
checker, never by the product path."""
