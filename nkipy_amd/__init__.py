"""NKIPy MI355X backend.

NumPy kernel functions run unchanged in two modes: called directly they are
plain NumPy on the CPU; through ``trace`` / ``baremetal_jit`` /
``DeviceKernel`` they are traced into a graph that is pattern-matched onto
hand-written gfx950 (CDNA4) HIP kernels and run through a thin C-ABI runtime.
"""

__version__ = "0.1.0"
