"""Tracer front end: tensor refs, op registry, IR and NKIPyKernel."""
