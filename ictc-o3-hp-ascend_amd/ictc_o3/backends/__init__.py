"""Backends of the ictc_o3 operators (HIP only)."""
