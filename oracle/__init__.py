"""CPU checker of the W8g128 quantized-MLP path (test infrastructure only).

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import this package, and only as the checker.
The product path (the HIP library under sepal-runner_amd/) never calls it.
"""
