"""OptimizedConvSequence (hydra/attention/backends/ccgqa/kernels/fused_conv.py:10-62).

Holds the two Conv1d parameters under the reference's names (conv1, conv2)
so state_dicts load unchanged.  Its forward runs the same two causal convs
through the generic path of the fused CCGQA prep kernel; inside
CCGQAAttention the convs are fused with the rest of the q/k preparation and
this forward is not used.
"""
from __future__ import annotations

import torch
import torch.nn as nn


class OptimizedConvSequence(nn.Module):
    def __init__(self, channels, groups1, groups2, kernel_size=3):
        super().__init__()
        self.channels = channels
        self.kernel_size = kernel_size
        self.conv1 = nn.Conv1d(channels, channels, kernel_size=kernel_size, padding=0,
                               groups=groups1, bias=False)
        self.conv2 = nn.Conv1d(channels, channels, kernel_size=kernel_size, padding=0,
                               groups=groups2, bias=False)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        """[B, N, C] -> [B, N, C]: conv1(pad_left(k-1)) then conv2(pad_left(k-1))."""
        from ..ops import conv_sequence

        return conv_sequence(x, self.conv1.weight, self.conv2.weight, self.conv1.groups,
                             self.conv2.groups)


def replace_conv_sequence(conv1, conv2):
    """fused_conv.py:65-82."""
    opt = OptimizedConvSequence(conv1.out_channels, conv1.groups, conv2.groups, conv1.kernel_size[0])
    opt.conv1.weight.data.copy_(conv1.weight.data)
    opt.conv2.weight.data.copy_(conv2.weight.data)
    return opt
