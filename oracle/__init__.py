"""CPU oracle for the K-Means hot path — test infrastructure only.

Importable by tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg,
never by the product package.
"""
