"""ORACLE: CPU restatements of the reference's integer semantics, used only as a checker
by tests/, __graft_entry__.smoke() and bench.py's CPU-baseline leg."""
