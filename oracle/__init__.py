"""ORACLE -- test infrastructure only (the checker, never the product).

quants.py  numpy restatement of the reference quantizers (ggml-quants.c)
ref.py     ctypes binding of the reference's own C build in oracle/_ref (see oracle/Makefile)

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import this package.
"""
