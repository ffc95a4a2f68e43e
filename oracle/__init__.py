"""CPU oracle of the attention path — test infrastructure only.

Importable only from tests/, __graft_entry__.smoke() and bench.py's CPU-baseline
leg. See attn_oracle.py.
"""
