"""Test-only CPU checker for the SGSA hot path (see sgsa_oracle.py's header).

Importable only from tests/, __graft_entry__.smoke() and bench.py's
cpu_baseline leg.  The product package never imports it.
"""
