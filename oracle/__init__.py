"""CPU oracle of the Q4_0 x Q8_1 path — TEST INFRASTRUCTURE ONLY.

Importable only from tests/, __graft_entry__.smoke() and bench.py's
cpu_baseline leg.  The product package (jjjetson_ops_amd) never imports it.
"""
