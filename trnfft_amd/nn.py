"""ComplexLinear on the HIP complex GEMM (trnfft/nn.py:18-49).

Same parameters, initialisation and state_dict keys as the reference (``W_re.weight``,
``W_im.weight``, ``bias_re``, ``bias_im``), so checkpoints move between the two unchanged.  The
forward pass is one fused kernel: the four real products share their A/B tiles and the bias is
added in the epilogue.
"""

from __future__ import annotations

import math

import torch
import torch.nn as nn

from .complex import ComplexTensor
from .dispatch import complex_linear


class ComplexLinear(nn.Module):
    """Complex-valued linear layer: y = W x + b (complex arithmetic)."""

    def __init__(self, in_features: int, out_features: int, bias: bool = True):
        super().__init__()
        self.W_re = nn.Linear(in_features, out_features, bias=False)
        self.W_im = nn.Linear(in_features, out_features, bias=False)
        self.bias_re = nn.Parameter(torch.zeros(out_features)) if bias else None
        self.bias_im = nn.Parameter(torch.zeros(out_features)) if bias else None
        self._reset_parameters()

    def _reset_parameters(self):
        # trnfft/nn.py:29-31
        nn.init.kaiming_uniform_(self.W_re.weight, a=math.sqrt(5))
        nn.init.kaiming_uniform_(self.W_im.weight, a=math.sqrt(5))

    def forward(self, x: ComplexTensor) -> ComplexTensor:
        # differentiable in x, both weights and the bias (adjoint GEMMs on the same kernel)
        return complex_linear(x, self.W_re.weight, self.W_im.weight, self.bias_re, self.bias_im)
