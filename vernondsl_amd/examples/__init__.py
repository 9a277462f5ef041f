"""Taichi-style programs that run unchanged under `python -m vernondsl_amd.run`."""
