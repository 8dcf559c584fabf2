"""CPU checker for the HIP kernels (test infrastructure only).

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import
this package. The product path under levo2.cpp_amd/ never imports it.
"""
