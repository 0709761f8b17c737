"""Autograd helpers."""
