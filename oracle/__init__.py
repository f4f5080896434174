"""ORACLE — test infrastructure, not part of the product.

Python access to the CPU restatement of the StrasGPT reference forward pass
(oracle/oracle.c). Only tests/, __graft_entry__.smoke() and bench.py's
cpu_baseline leg import this package: the reference the GPU results are
compared against, and the CPU baseline.
"""
from .oracle import OracleModel, load_lib, oracle_available  # noqa: F401
