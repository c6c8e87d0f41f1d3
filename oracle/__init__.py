"""ORACLE -- test infrastructure only.

CPU restatements of rocm_qlora's quantized-linear path, used solely as the
parity checker by tests/, by __graft_entry__.smoke(), and as the timed CPU
baseline in bench.py.  Nothing in the product package imports this.
"""
