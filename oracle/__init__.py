"""CPU oracle for the EXL3 decode path -- test infrastructure only.

Importable only from tests/, __graft_entry__.smoke() and bench.py's cpu_baseline
leg, and only as the checker; the product package never imports it."""
