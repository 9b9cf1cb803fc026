"""Routing sweeps for this build's devices (see sweep.py)."""
