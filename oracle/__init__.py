"""CPU oracle for flash-Born attention -- test infrastructure only.

Importable only by tests/, __graft_entry__.smoke() and bench.py's cpu_baseline
leg, as the checker.  The product package never imports it.
"""
