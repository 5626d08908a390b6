"""CPU oracle of the PI0 / PI0.5 path -- test infrastructure only (see
pi0_oracle.py).  Only tests/, __graft_entry__.smoke() and bench.py's
cpu_baseline leg import it."""
