"""MACE radial embedding: Bessel basis times the polynomial cutoff envelope.

Follows reference ``mace_ictc/models/radial_basis.py:11-39`` (``mace_polynomial_cutoff``)
and ``:42-92`` (``mace_radial_embedding``, ``function_type="bessel"``):

    e_n(r) = sqrt(2 / r_max) * sin(n pi r / r_max) / r,          n = 1..num_basis
    u(r)   = 1 - (p+1)(p+2)/2 (r/r_max)^p + p(p+2) (r/r_max)^(p+1) - p(p+1)/2 (r/r_max)^(p+2)
             for r < r_max, 0 beyond;
    emb    = e(r) * u(r)        (times sqrt(num_basis) only when sqrt_num_basis_norm).
"""
from __future__ import annotations

import math

import torch


def polynomial_cutoff(r: torch.Tensor, r_max: float, p: int = 5) -> torch.Tensor:
    x = r / float(r_max)
    pf = float(p)
    env = (1.0 - ((pf + 1.0) * (pf + 2.0) / 2.0) * torch.pow(x, p) + pf * (pf + 2.0) * torch.pow(x, p + 1)
           - (pf * (pf + 1.0) / 2.0) * torch.pow(x, p + 2))
    return env * (r < float(r_max)).to(r.dtype)


def bessel_embedding(r: torch.Tensor, *, r_max: float, num_basis: int = 8, cutoff_p: int | None = 5,
                     sqrt_num_basis_norm: bool = False) -> torch.Tensor:
    """[E] edge lengths -> [E, num_basis]."""
    freq = (math.pi / float(r_max)) * torch.arange(1, num_basis + 1, dtype=r.dtype, device=r.device)
    emb = math.sqrt(2.0 / float(r_max)) * torch.sin(r.unsqueeze(-1) * freq) / r.clamp_min(1e-12).unsqueeze(-1)
    if cutoff_p is not None:
        emb = emb * polynomial_cutoff(r, r_max, cutoff_p).unsqueeze(-1)
    if sqrt_num_basis_norm:
        emb = emb * math.sqrt(num_basis)
    return emb
