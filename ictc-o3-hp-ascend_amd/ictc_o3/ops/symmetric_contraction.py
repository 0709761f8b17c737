"""Species-conditioned symmetric contraction modules (correlation <= 3) on HIP kernels.

``ICTDBridgeUSymmetricContractionSO3`` is the module the reference's factory returns
(``ictc_o3/ops/symmetric_contraction.py:92-206``, ``operators.py:204-218``): a MACE
contraction (``ops/_mace_symmetric_contraction.py:30-378``) whose U tensors are the e3nn
generalized couplings (``basis/_mace_cg.py:39-190``) with the per-degree basis bridge to the
ICTC basis (``SO3ToE3NNBasisBridge``, ``:24-89``) folded into them, so that it consumes and
returns ICTC-basis features.  Same submodule, parameter and buffer names as the reference
(``basis_bridge.q_l``, ``symmetric_contractions.contractions.<i>.U_matrix_<nu>``,
``weights_max``, ``weights.<i>``, ``weights_<i>_zeroed``, ``weights_max_zeroed``), so a
reference state dict loads unchanged.  Its U buffers are whatever the module holds (built here
from the restated e3nn conventions of ``ictc_o3/basis/e3nn_convention.py``, or loaded from a
checkpoint): the forward projects them onto the coupling chains the HIP kernels evaluate
(``ictc_o3/ops/factorized_contraction.py``) behind the reference's 4e-6 reconstruction gate and
runs the kernels on the mapped weights.

``ICTDPureUSymmetricContractionSO3`` is the reference's pure-ICTC variant
(``mace_ictc/models/pure_cartesian_ictd_fix.py:1202-1389``), whose weights already address the
chain columns.

Layouts (both modules): input ``[N, C*(L+1)^2]`` with degree blocks ``[C, 2l+1]``; output the
concatenation over target degrees of ``[C, 2l+1]`` blocks.
"""
from __future__ import annotations

from typing import Dict, List, Optional

import numpy as np
import torch
import torch.nn as nn

from ictc_o3.backends.hip.runtime import require_gpu_fp32
from ictc_o3.backends.hip.species import validate_species


def _split_irreps(x: torch.Tensor, channels: int, lmax: int) -> Dict[int, torch.Tensor]:
    """Flat [N, C*(L+1)^2] -> {l: [N, C, 2l+1]} (reference ``basis/layout.py:4-18``)."""
    out, offset = {}, 0
    for l in range(lmax + 1):
        width = channels * (2 * l + 1)
        out[l] = x[..., offset:offset + width].reshape(*x.shape[:-1], channels, 2 * l + 1)
        offset += width
    return out


def _merge_blocks(blocks: Dict[int, torch.Tensor], channels: int, lmax: int) -> torch.Tensor:
    return torch.cat([blocks[l].reshape(*blocks[l].shape[:-2], channels * (2 * l + 1)) for l in range(lmax + 1)],
                     dim=-1)


def _so3_flat_to_mace_features(x: torch.Tensor, channels: int, lmax: int) -> torch.Tensor:
    """Flat [N, C*(L+1)^2] -> [N, C, (L+1)^2] (reference ``ops/symmetric_contraction.py:14-16``)."""
    blocks = _split_irreps(x, channels, lmax)
    return torch.cat([blocks[l] for l in range(lmax + 1)], dim=-1)


def _mace_features_to_flat(x: torch.Tensor, lmax: int) -> torch.Tensor:
    """[N, C, (L+1)^2] -> flat [N, C*(L+1)^2] (inverse of the above)."""
    n, c = x.shape[0], x.shape[1]
    return torch.cat([x[:, :, l * l:(l + 1) ** 2].reshape(n, c * (2 * l + 1)) for l in range(lmax + 1)], -1)


class SO3ToE3NNBasisBridge(nn.Module):
    """Per-degree orthogonal maps Q_l with Y_ictc_l Q_l = Y_e3nn_l (buffers ``q_l``; reference
    ``ops/symmetric_contraction.py:24-89``: Procrustes fit on 8192 seeded directions)."""

    def __init__(self, channels: int, lmax: int, num_samples: int = 8192):
        super().__init__()
        from ictc_o3.basis.e3nn_convention import basis_bridge
        self.channels, self.lmax = int(channels), int(lmax)
        for l, q in enumerate(basis_bridge(self.lmax, num_samples)):
            self.register_buffer(f"q_{l}", torch.from_numpy(q).to(torch.get_default_dtype()), persistent=True)

    def _q(self, l: int, *, dtype: torch.dtype, device: torch.device) -> torch.Tensor:
        return getattr(self, f"q_{int(l)}").to(dtype=dtype, device=device)

    def ictd_flat_to_e3nn_blocks(self, x: torch.Tensor, lmax: int) -> Dict[int, torch.Tensor]:
        return {l: torch.einsum("ncm,mp->ncp", b, self._q(l, dtype=x.dtype, device=x.device))
                for l, b in _split_irreps(x, self.channels, lmax).items()}

    def e3nn_flat_to_ictd_blocks(self, x: torch.Tensor, lmax: int) -> Dict[int, torch.Tensor]:
        return {l: torch.einsum("ncm,pm->ncp", b, self._q(l, dtype=x.dtype, device=x.device))
                for l, b in _split_irreps(x, self.channels, lmax).items()}

    def ictd_flat_to_e3nn_flat(self, x: torch.Tensor, lmax: int) -> torch.Tensor:
        return _merge_blocks(self.ictd_flat_to_e3nn_blocks(x, lmax), self.channels, lmax)

    def e3nn_flat_to_ictd_flat(self, x: torch.Tensor, lmax: int) -> torch.Tensor:
        return _merge_blocks(self.e3nn_flat_to_ictd_blocks(x, lmax), self.channels, lmax)


class _Contraction(nn.Module):
    """One target irrep of the MACE contraction: U buffers ``U_matrix_<nu>`` and the weights
    ``weights_max [S, K_corr, C]`` / ``weights[i] [S, K_{corr-1-i}, C]`` (init randn / K), with
    the reference's names (``_mace_symmetric_contraction.py:86-237``)."""

    def __init__(self, u_tensors: List[torch.Tensor], output_lmax: int, correlation: int, num_elements: int,
                 num_features: int):
        super().__init__()
        self.correlation, self.output_lmax = int(correlation), int(output_lmax)
        self.num_features, self.num_elements = int(num_features), int(num_elements)
        keep = []
        for nu, u in enumerate(u_tensors, start=1):
            keep.append(bool(torch.any(u != 0)))
            self.register_buffer(f"U_matrix_{nu}", u)
        k = self.U_tensors(self.correlation).shape[-1]
        self.weights_max = nn.Parameter(torch.randn(num_elements, k, num_features) / k)
        self.weights = nn.ParameterList()
        for nu in range(self.correlation - 1, 0, -1):
            k = self.U_tensors(nu).shape[-1]
            self.weights.append(nn.Parameter(torch.randn(num_elements, k, num_features) / k))
        for idx, flag in enumerate(keep):
            name = f"weights_{idx}_zeroed" if idx < self.correlation - 1 else "weights_max_zeroed"
            self.register_buffer(name, torch.tensor(not flag, dtype=torch.bool))

    def U_tensors(self, nu: int) -> torch.Tensor:
        return getattr(self, f"U_matrix_{int(nu)}")

    def columns(self):
        """Weight blocks in kernel column order: orders correlation, correlation-1, ..., 1."""
        return [self.weights_max, *self.weights]


class MaceSymmetricContraction(nn.Module):
    """Container of the per-target-irrep contractions (reference ``:30-83``)."""

    def __init__(self, contractions: List[_Contraction]):
        super().__init__()
        self.contractions = nn.ModuleList(contractions)


def _species(node_attrs, node_type_idx, nodes, num_elements):
    if node_attrs is None and node_type_idx is None:
        raise ValueError("either node_attrs or node_type_idx is required")
    species = node_attrs.argmax(-1) if node_type_idx is None else node_type_idx
    species = species.to(torch.int64).contiguous()
    if species.shape != (nodes,):
        raise ValueError("species indices must have shape [N]")
    validate_species(species, num_elements)
    return species


class ICTDBridgeUSymmetricContractionSO3(nn.Module):
    """Bridge-U symmetric contraction in the ICTC basis (reference
    ``ops/symmetric_contraction.py:92-206``)."""

    def __init__(self, *, num_elements: int, channels: int, lmax: int, target_lmax: int, correlation: int = 3,
                 use_reduced_cg: bool = False):
        super().__init__()
        from ictc_o3.basis.e3nn_convention import fold_u, u_matrix_real
        if correlation not in (1, 2, 3):
            raise ValueError("symmetric contraction supports correlation 1, 2 and 3")
        self.channels, self.lmax, self.target_lmax = int(channels), int(lmax), int(target_lmax)
        self.num_elements, self.correlation = int(num_elements), int(correlation)
        self.use_reduced_cg = bool(use_reduced_cg)
        self.basis_bridge = SO3ToE3NNBasisBridge(self.channels, max(self.lmax, self.target_lmax))
        qs = [getattr(self.basis_bridge, f"q_{l}").double().numpy() for l in range(max(self.lmax, self.target_lmax) + 1)]
        dtype = torch.get_default_dtype()
        contractions = []
        for l_out in range(self.target_lmax + 1):
            us = [torch.from_numpy(np.ascontiguousarray(fold_u(u_matrix_real(self.lmax, l_out, nu), qs, self.lmax,
                                                               l_out, nu))).to(dtype)
                  for nu in range(1, self.correlation + 1)]
            contractions.append(_Contraction(us, l_out, self.correlation, self.num_elements, self.channels))
        self.symmetric_contractions = MaceSymmetricContraction(contractions)
        self._kernel_plan = None

    @property
    def plan(self):
        """Kernel configuration (compiled degree combination)."""
        if self._kernel_plan is None:
            from ictc_o3.backends.hip.symmetric_contraction import ContractionPlan
            self._kernel_plan = ContractionPlan(self.lmax, self.target_lmax, self.correlation, self.channels,
                                                self.num_elements)
        return self._kernel_plan

    def weight_table(self, x: torch.Tensor) -> torch.Tensor:
        """[S, KTOT, C] kernel weights: the live module weights mapped onto the chain columns
        (differentiable); raises when the U buffers fail the reconstruction gate."""
        from ictc_o3.ops.factorized_contraction import _plan
        plan = _plan(self, x)
        if plan is None:
            raise ValueError("Symmetric-contraction constants do not reconstruct within the FP32 budget")
        return plan.weight_table(self.symmetric_contractions.contractions)

    def forward(self, node_feats: torch.Tensor, node_attrs: Optional[torch.Tensor] = None,
                node_type_idx: Optional[torch.Tensor] = None) -> torch.Tensor:
        from ictc_o3.backends.hip.symmetric_contraction import symmetric_contraction
        require_gpu_fp32(node_feats)
        plan = self.plan
        if node_feats.ndim != 2 or node_feats.shape[1] != plan.in_width:
            raise ValueError("node features must have shape [N, C*(lmax+1)^2]")
        species = _species(node_attrs, node_type_idx, node_feats.shape[0], self.num_elements)
        return symmetric_contraction(plan, node_feats, species, self.weight_table(node_feats))


class _PureContraction(nn.Module):
    """Weights of one target degree of the pure-ICTC module (the reference's parameter names)."""

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
        return [self.weights_max, *self.weights]


class ICTDPureUSymmetricContractionSO3(nn.Module):
    """Pure-ICTC contraction (reference ``pure_cartesian_ictd_fix.py:1202-1389``): weights address
    the coupling chains of ``ictc_o3/basis/symmetric_u.py`` directly."""

    def __init__(self, *, num_elements: int, channels: int, lmax: int, target_lmax: int,
                 correlation: int = 3, with_u_buffers: bool = False):
        super().__init__()
        if correlation not in (1, 2, 3):
            raise ValueError("symmetric contraction supports correlation 1, 2 and 3")
        self.channels, self.lmax, self.target_lmax = int(channels), int(lmax), int(target_lmax)
        self.num_elements, self.correlation = int(num_elements), int(correlation)
        self.contractions = nn.ModuleList(
            [_PureContraction(self.lmax, l, self.correlation, self.num_elements, self.channels, with_u_buffers)
             for l in range(self.target_lmax + 1)])
        self._kernel_plan = None

    @property
    def plan(self):
        if self._kernel_plan is None:
            from ictc_o3.backends.hip.symmetric_contraction import ContractionPlan
            self._kernel_plan = ContractionPlan(self.lmax, self.target_lmax, self.correlation, self.channels,
                                                self.num_elements)
        return self._kernel_plan

    def weight_table(self, x: Optional[torch.Tensor] = None) -> torch.Tensor:
        """[S, KTOT, C]: all weight columns in kernel order (differentiable)."""
        return torch.cat([w for c in self.contractions for w in c.columns()], 1)

    def forward(self, node_feats: torch.Tensor, node_attrs: Optional[torch.Tensor] = None,
                node_type_idx: Optional[torch.Tensor] = None) -> torch.Tensor:
        from ictc_o3.backends.hip.symmetric_contraction import symmetric_contraction
        require_gpu_fp32(node_feats)
        plan = self.plan
        if node_feats.ndim != 2 or node_feats.shape[1] != plan.in_width:
            raise ValueError("node features must have shape [N, C*(lmax+1)^2]")
        species = _species(node_attrs, node_type_idx, node_feats.shape[0], self.num_elements)
        return symmetric_contraction(plan, node_feats, species, self.weight_table())
