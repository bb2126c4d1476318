"""CPU oracles of the sparse-prefill path -- test infrastructure only.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg import
this package, as the checker of the HIP kernels; nothing shipped uses it.
"""
