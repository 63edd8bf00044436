"""Path-preserving edge TP module (coefficient holder for the HIP kernels).

Mirrors the public surface of the reference's
``EdgeWeightedPathPreservingTensorProduct`` (ictc_o3/basis/ictd_irreps.py:2681-2971,
constructor of HarmonicPathWeightedTensorProduct :2316-2387): path enumeration
(l1 outer, l2, l3 ascending, natural parity, ``allowed_paths`` filter), the
``weight [P, C]`` parameter, ``path_l3`` / ``path_offset`` /
``path_counts_by_l`` placement tables.  Only component irrep normalisation and
element path normalisation are compiled into the kernels (the reference
defaults, ictd_irreps.py:100-113); other choices raise.

Its forward takes the reference's dictionary form ({l: [E, C, 2l+1]},
{l: [E, 1, 2l+1]} or {l: [E, 2l+1]}, gates [E, P*C]) and runs on the HIP
kernels; there is no CPU implementation in the product.
"""
from __future__ import annotations

from typing import Dict, List, Tuple

import torch
import torch.nn as nn

from ictc_o3.basis import tables


class EdgeWeightedPathPreservingTensorProduct(nn.Module):
    def __init__(self, channels: int, lmax: int, *, allowed_paths: List[Tuple[int, int, int]] | None = None,
                 path_policy: str = "full", max_rank_other: int | None = None, normalization: str = "component",
                 irrep_normalization: str | None = None, path_normalization: str = "element",
                 internal_compute_dtype: torch.dtype | None = None):
        super().__init__()
        self.channels, self.lmax = int(channels), int(lmax)
        norm = irrep_normalization if irrep_normalization is not None else normalization
        if norm != "component" or path_normalization != "element":
            raise ValueError("MI355X kernels implement component irrep and element path normalisation only")
        self.internal_compute_dtype = internal_compute_dtype or torch.get_default_dtype()
        all_paths = [(l1, l2, l3) for l1 in range(self.lmax + 1) for l2 in range(self.lmax + 1)
                     for l3 in range(abs(l1 - l2), min(l1 + l2, self.lmax) + 1) if (l1 + l2 + l3) % 2 == 0]
        if allowed_paths is not None:
            allowed = {tuple(p) for p in allowed_paths}
            self.paths = [p for p in all_paths if p in allowed]
        elif path_policy == "full":
            self.paths = all_paths
        elif path_policy == "max_rank_other":
            if max_rank_other is None:
                raise ValueError("path_policy='max_rank_other' requires max_rank_other")
            self.paths = [p for p in all_paths if min(p[0], p[1]) <= int(max_rank_other)]
        else:
            raise ValueError(f"Unknown path_policy={path_policy!r}")
        self.num_paths = len(self.paths)
        self.weight = nn.Parameter(torch.randn(self.num_paths, self.channels) * 0.02)
        counts: Dict[int, int] = {l: 0 for l in range(self.lmax + 1)}
        self.path_l3, self.path_offset = [], []
        for (_, _, l3) in self.paths:
            self.path_l3.append(l3)
            self.path_offset.append(counts[l3])
            counts[l3] += 1
        self.path_counts_by_l = counts

    def kernel_degrees(self):
        """(LI, LE, LO) when the paths are the natural-parity set of those degrees, else None."""
        if not self.paths:
            return None
        li = max(p[0] for p in self.paths)
        le = max(p[1] for p in self.paths)
        lo = max(p[2] for p in self.paths)
        if [tuple(p) for p in self.paths] != tables.natural_paths(li, le, lo):
            return None
        return li, le, lo

    def forward(self, x1: Dict[int, torch.Tensor], x2: Dict[int, torch.Tensor], gates: torch.Tensor | None = None):
        from ictc_o3.operators import EdgeTensorProduct
        degrees = self.kernel_degrees()
        if degrees is None:
            raise ValueError("path set is not a natural-parity triangle set; unsupported by the MI355X kernels")
        li, le, _ = degrees
        op = EdgeTensorProduct(self, input_lmax=li, edge_lmax=le) if not self.weight.requires_grad else None
        if op is None:
            raise ValueError("TP base coefficients must already be fixed; HP does not freeze learned weights")
        sample = next(iter(x1.values()))
        E = sample.shape[0]
        blocks = {l: x1[l] if l in x1 else sample.new_zeros(E, self.channels, 2 * l + 1) for l in range(li + 1)}
        feats = op.pack_input(blocks)
        sh = torch.cat([x2[l].reshape(E, 2 * l + 1) for l in range(le + 1)], -1)
        if gates is None:
            gates = feats.new_ones(E, self.num_paths * self.channels)
        return op.unpack_output(op(feats, sh, gates.reshape(E, -1)))
