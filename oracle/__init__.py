"""CPU oracle of the group-quantized linear path — test infrastructure only.

Importable by tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg;
never by the product package.
"""
