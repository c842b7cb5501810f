"""CPU oracle (test infrastructure only): the checker for the HIP path.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg import this.
"""
