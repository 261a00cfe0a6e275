"""CPU oracle for the GOAP quantized-linear path (test infrastructure only).

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg import
this package. The product package tensorshrink_amd never does.
"""
