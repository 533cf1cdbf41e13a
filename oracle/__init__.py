"""TEST INFRASTRUCTURE, NOT PRODUCT CODE: the CPU oracle (C restatement + numpy) of the reference's hot path.
Imported only by tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg."""
