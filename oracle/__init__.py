"""CPU restatement of the reference arithmetic -- test infrastructure only.

Importable by tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg.
The product (polykernel_amd) never imports it.
"""
