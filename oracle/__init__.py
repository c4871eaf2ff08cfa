"""CPU oracle for the SimpleMoE hot path — test infrastructure only.

Imported by tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg,
never by the smoe package.  Parity status of each function is listed in
smoe_oracle's module docstring."""
