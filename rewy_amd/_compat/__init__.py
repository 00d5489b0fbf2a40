"""Autograd contracts of the four operator families (optimized backend)."""
