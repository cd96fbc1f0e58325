"""Device presence probe.

``is_neuron_compatible`` keeps the reference's name
(nkipy/src/nkipy/runtime/utils.py:3-19), so tests gate device runs on it the
same way; here it reports whether a GPU is visible to the HIP runtime.
"""


def is_gpu_available() -> bool:
    try:
        from nkipy_amd.runtime.hip import device_count

        return device_count() > 0
    except Exception:
        return False


is_neuron_compatible = is_gpu_available
