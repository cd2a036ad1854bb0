"""TEST INFRASTRUCTURE ONLY: the CPU oracle for the selective-scan path.

Importable only from tests/, __graft_entry__.smoke() and bench.py's
cpu_baseline leg, as the checker. See oracle.py and torch_ref.py.
"""
