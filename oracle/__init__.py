"""CPU oracle of the multi-pathway attention op -- test infrastructure only.

Importable only from tests/, __graft_entry__.smoke() and bench.py's
cpu_baseline leg; the product path (mint_plus_amd) never uses it.
"""
