"""nn.Linear whose few-row calls run the weight-streaming skinny kernel.

The decoder's projections (the reference's QKVParallelLinear, RowParallelLinear,
MergedColumnParallelLinear and ParallelLMHead, layers/linear.py, layers/embed_head.py,
on one GPU) are plain linear layers; in a decode step they see one row per
sequence, and streaming the weights is the whole cost.  Calls with at most 16
rows that vlc_linear_skinny takes run there; every other call is torch's
F.linear (hipBLASLt).
"""
from __future__ import annotations

import torch.nn.functional as F
from torch import nn

from .. import kernels


class Linear(nn.Linear):

    def forward(self, x):
        x2 = x if x.dim() == 2 else x.reshape(-1, x.shape[-1])
        if x2.shape[0] <= kernels.SKINNY_MAX_ROWS and kernels.linear_skinny_supported(x2, self.weight, self.bias):
            y = kernels.linear_skinny(x2, self.weight, self.bias)
            return y if x.dim() == 2 else y.view(*x.shape[:-1], y.shape[-1])
        return F.linear(x, self.weight, self.bias)
