"""CPU oracle of the MLA decode path -- test infrastructure only.

Importable by tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg; never
by the product package (flagattention_amd), which has no CPU fallback.
"""
