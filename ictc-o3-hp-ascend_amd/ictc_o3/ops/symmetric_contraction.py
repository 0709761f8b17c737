"""Species-conditioned symmetric contraction module (correlation <= 3) on HIP kernels.

Mirrors the reference's pure-ICTC contraction
(``ICTDPureUSymmetricContractionSO3`` / ``_ICTDPureUContraction``,
``mace_ictc/models/pure_cartesian_ictd_fix.py:1202-1389``) and its public factory
(``ictc_o3/operators.py:189-218``): one contraction per target degree l, each with
``weights_max [S, K_corr, C]`` and ``weights[i] [S, K, C]`` for the lower orders
(init ``randn / K``), U tensors from the ICTC coupling chains
(``ictd_irreps.py:1387-1517``, kept as buffers ``U_matrix_{nu}`` for inspection),
and the flat layouts of the reference module (input ``[N, C*(L+1)^2]`` with degree
blocks ``[C, 2l+1]``; output concatenated over target degrees).  The contraction
itself runs in ``libictc_hip.so``.
"""
from __future__ import annotations

from typing import Optional

import torch
import torch.nn as nn

from ictc_o3.backends.hip.runtime import require_gpu_fp32
from ictc_o3.backends.hip.species import validate_species


class _Contraction(nn.Module):
    """Weights of one target degree (same parameter names/shapes as the reference)."""

    def __init__(self, lmax: int, output_l: int, correlation: int, num_elements: int, channels: int,
                 with_u_buffers: bool = False):
        super().__init__()
        from ictc_o3.basis.symmetric_u import chains, u_matrix
        self.output_l, self.correlation = int(output_l), int(correlation)
        self.num_elements, self.num_features = int(num_elements), int(channels)
        self.num_params = {nu: len(chains(lmax, output_l, nu)) for nu in range(1, correlation + 1)}
        if with_u_buffers:
            for nu in range(1, correlation + 1):
                self.register_buffer(f"U_matrix_{nu}", torch.from_numpy(u_matrix(lmax, output_l, nu)).float(),
                                     persistent=False)
        k = self.num_params[correlation]
        self.weights_max = nn.Parameter(torch.randn(num_elements, k, channels) / max(k, 1))
        self.weights = nn.ParameterList(
            [nn.Parameter(torch.randn(num_elements, self.num_params[nu], channels) / max(self.num_params[nu], 1))
             for nu in range(correlation - 1, 0, -1)])

    def columns(self):
        """Weight blocks in kernel column order: orders correlation, correlation-1, ..., 1."""
        return [self.weights_max, *self.weights]


class ICTDPureUSymmetricContractionSO3(nn.Module):
    def __init__(self, *, num_elements: int, channels: int, lmax: int, target_lmax: int,
                 correlation: int = 3, with_u_buffers: bool = False):
        super().__init__()
        if correlation not in (1, 2, 3):
            raise ValueError("symmetric contraction supports correlation 1, 2 and 3")
        self.channels, self.lmax, self.target_lmax = int(channels), int(lmax), int(target_lmax)
        self.num_elements, self.correlation = int(num_elements), int(correlation)
        self.contractions = nn.ModuleList(
            [_Contraction(self.lmax, l, self.correlation, self.num_elements, self.channels, with_u_buffers)
             for l in range(self.target_lmax + 1)])
        self._plan = None

    @property
    def plan(self):
        if self._plan is None:
            from ictc_o3.backends.hip.symmetric_contraction import ContractionPlan
            self._plan = ContractionPlan(self.lmax, self.target_lmax, self.correlation, self.channels,
                                         self.num_elements)
        return self._plan

    def weight_table(self) -> torch.Tensor:
        """[S, KTOT, C]: all weight columns in kernel order (differentiable)."""
        return torch.cat([w for c in self.contractions for w in c.columns()], 1)

    def _species(self, node_attrs, node_type_idx, nodes):
        species = node_attrs.argmax(-1) if node_type_idx is None else node_type_idx
        species = species.to(torch.int64).contiguous()
        if species.shape != (nodes,):
            raise ValueError("species indices must have shape [N]")
        validate_species(species, self.num_elements)
        return species

    def forward(self, node_feats: torch.Tensor, node_attrs: Optional[torch.Tensor] = None,
                node_type_idx: Optional[torch.Tensor] = None) -> torch.Tensor:
        from ictc_o3.backends.hip.symmetric_contraction import symmetric_contraction
        require_gpu_fp32(node_feats)
        plan = self.plan
        if node_feats.ndim != 2 or node_feats.shape[1] != plan.in_width:
            raise ValueError("node features must have shape [N, C*(lmax+1)^2]")
        if node_attrs is None and node_type_idx is None:
            raise ValueError("either node_attrs or node_type_idx is required")
        species = self._species(node_attrs, node_type_idx, node_feats.shape[0])
        return symmetric_contraction(plan, node_feats, species, self.weight_table())
