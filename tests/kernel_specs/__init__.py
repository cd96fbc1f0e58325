"""NumPy kernels with their input specifications (``kernel_specs`` lists),
the workloads of the conformance suite: each module states one workload of
the reference's tests/kernels/ in this package's own NumPy code."""
