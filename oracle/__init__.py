"""TEST INFRASTRUCTURE ONLY: the CPU oracle of the hot path.

Importable only from tests/, __graft_entry__.smoke() and bench.py's
cpu_baseline leg, and only as the checker.  The product package
(rwkv-quant_amd/) never imports it.
"""
