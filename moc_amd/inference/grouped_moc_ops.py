"""MoC 2:8 operators moc::fused_grouped_top2_up_silu and moc::selected_grouped_down
(moc/inference/triton_grouped_moc_ops.py:26-143), registered by importing this
module."""
from __future__ import annotations

import torch

from .. import ops

ops.register()

fused_grouped_top2_up_silu = torch.ops.moc.fused_grouped_top2_up_silu
selected_grouped_down = torch.ops.moc.selected_grouped_down
