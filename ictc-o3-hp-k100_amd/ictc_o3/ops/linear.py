"""Channel-mixing linears on the packed component-major layout.

These are the only GEMM-shaped maps of the model (north-star: the MFMA
site).  Shapes (C channels, N nodes):
  degree_linear  out[n, l*l+m, :] = scale * W_l @ x[n, l*l+m, :]            (linear_up, product linear)
  path_linear    out[n, l*l+m, :] = scale * W_l @ concat_k msg[n, l, k, m, :] (message_linear / avg_num_neighbors)
  species_linear out[n, :] = W[s_n] @ x[n, :]                               (element-conditioned self-connection)
Here they are dense FP32 GEMMs through the ROCm BLAS library (TF32 off).
"""
from __future__ import annotations

from typing import Dict, List

import torch


def degree_linear(x: torch.Tensor, weights: List[torch.Tensor], C: int, lmax: int, scale: float = 1.0):
    N = x.shape[0]
    parts = []
    for l in range(lmax + 1):
        blk = x[:, l * l * C:(l + 1) ** 2 * C].reshape(N * (2 * l + 1), C)
        w = weights[l] if scale == 1.0 else weights[l] * scale
        parts.append(torch.matmul(blk, w.t()).reshape(N, (2 * l + 1) * C))
    return torch.cat(parts, 1)


def path_linear(m: torch.Tensor, weights: List[torch.Tensor], counts: Dict[int, int], C: int, lmax: int,
                scale: float = 1.0):
    N = m.shape[0]
    parts, off = [], 0
    for l in range(lmax + 1):
        k, w = counts.get(l, 0), 2 * l + 1
        blk = m[:, off:off + k * w * C].reshape(N, k, w, C).transpose(1, 2).reshape(N * w, k * C)
        off += k * w * C
        parts.append(torch.matmul(blk, (weights[l] * scale).t()).reshape(N, w * C))
    return torch.cat(parts, 1)


def species_linear(x: torch.Tensor, weight: torch.Tensor, species: torch.Tensor):
    """weight [S, Cout, Cin]: all species products in one GEMM, then select per node."""
    S, Co, Ci = weight.shape
    allp = torch.matmul(x, weight.reshape(S * Co, Ci).t()).reshape(x.shape[0], S, Co)
    return allp.gather(1, species.view(-1, 1, 1).expand(-1, 1, Co)).squeeze(1)


def channel_linear(features: torch.Tensor, weight: torch.Tensor, bias=None):
    """[*, Cin, m] x [Cout, Cin] -> [*, Cout, m] (operators.py:609-628)."""
    angular = features.movedim(-2, -1).contiguous()
    out = torch.nn.functional.linear(angular.reshape(-1, weight.shape[1]), weight, bias)
    return out.reshape(*angular.shape[:-1], weight.shape[0]).movedim(-1, -2)
