"""Operator modules (symmetric contraction)."""
