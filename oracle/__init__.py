"""Test infrastructure: CPU oracle of the packed 4-bit affine quantized matmul.

Importable only from tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg, where it is
the reference results are checked against (or the timed CPU baseline), never the thing measured
or shipped.
"""
