"""Inference MoC FFN (InferenceMoCSwiGLUFFN of moc/inference/inference_ffn.py:17-315).

Modes (same names as the reference):
  dense_baseline      dense SwiGLU, stock torch modules (the comparison row)
  masked_reference    dense MoC masking with torch ops, the reference's own
                      correctness oracle (:169-180)
  moc_inference_optimized_global_after_gate_native
                      gfx950 path: gate GEMV (MFMA) -> Top-K -> selected
                      Up*SiLU -> selected Down
  moc_inference_grouped_top2of8
                      gfx950 path: fused gate/up + top-2-of-8 -> selected Down
make_moc2_8_graph_runner() captures the 2:8 path in a HIP graph writing
into persistent buffers (:205-279).
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import Optional

import torch
import torch.nn as nn
import torch.nn.functional as F

from .. import kernels as K
from . import optimized_global_moc_ops  # noqa: F401  (registers the operators)
from .fused_ffn_kernels import (
    fused_gate_top2of8_selected_up_silu_into,
    selected_down_from_sparse_z_into,
)
from .optimized_global_moc_ops import ensure_native_ops_ready


@dataclass(frozen=True)
class InferenceMoCConfig:
    hidden_size: int
    intermediate_size: int
    k: int
    grouped_a: Optional[int] = None
    grouped_b: Optional[int] = None

    @property
    def grouped(self) -> bool:
        return self.grouped_a is not None and self.grouped_b is not None


class InferenceMoCSwiGLUFFN(nn.Module):
    """Inference-only MoC FFN with dense, masked-reference and gfx950 modes."""

    GUSILU_BLOCK_B_DEFAULT = 16
    GUSILU_BLOCK_G_DEFAULT = 16
    GUSILU_BLOCK_H_DEFAULT = 64
    GROUPED_DOWN_BLOCK_K_DEFAULT = 128
    GROUPED_DOWN_BLOCK_H_DEFAULT = 16

    def __init__(self, hidden_size: int, intermediate_size: int, k: int,
                 grouped_a: Optional[int] = None, grouped_b: Optional[int] = None):
        super().__init__()
        if k < 1 or k > intermediate_size:
            raise ValueError(f"k={k} must be in [1, {intermediate_size}]")
        if (grouped_a is None) != (grouped_b is None):
            raise ValueError("grouped_a and grouped_b must be set together")
        if grouped_a is not None:
            if intermediate_size % grouped_b != 0:
                raise ValueError(
                    f"intermediate_size={intermediate_size} must be divisible by grouped_b={grouped_b}")
            expected_k = intermediate_size * grouped_a // grouped_b
            if k != expected_k:
                raise ValueError(f"grouped MoC requires k=intermediate_size*a/b={expected_k}, got {k}")
        self.config = InferenceMoCConfig(hidden_size, intermediate_size, k, grouped_a, grouped_b)
        self.gate_proj = nn.Linear(hidden_size, intermediate_size, bias=False)
        self.up_proj = nn.Linear(hidden_size, intermediate_size, bias=False)
        self.down_proj = nn.Linear(intermediate_size, hidden_size, bias=False)
        # Derived state, rebuilt when the weights change and frozen by
        # freeze_for_compile(): the [inter, hidden] copy of W_down that the
        # selected Down kernels stream row by row (with the weight version it
        # was made from), flat channel offsets of the 2:8 groups for the
        # masked reference, the decode kernels' workspaces (one per batch
        # size of at most 16 tokens, owned by this module so that a HIP graph
        # captured with one never sees it freed or shared with another
        # module), and the 2:8 prefill buffers (one grow-only set per device).
        self._down_weight_t: torch.Tensor | None = None
        self._down_weight_t_key: tuple | None = None
        self._group_offsets: dict = {}
        self._after_gate_ws: dict = {}
        self._decode_ws: dict = {}
        self._packed28: dict = {}
        self._packed28_captured: list = []
        self._compile_frozen: bool = False

    # -- derived state (the caches of inference_ffn.py:78-129)
    def _ensure_down_weight_t(self) -> None:
        """(Re)build the cached W_down^T unless frozen; the key includes the
        weight's in-place version counter, so optimizer steps and
        load_state_dict() on the same storage also refresh it."""
        if self._compile_frozen:
            return
        w = self.down_proj.weight
        key = (w.data_ptr(), w._version, w.device, w.dtype)
        if self._down_weight_t_key != key:
            # [inter, hidden] at a row pitch of hidden + 64 (128 bytes): the
            # decode kernels read one column block of it per workgroup down
            # the selected rows, and a 4 KB pitch puts every row's block on
            # the same memory channels
            self._down_weight_t = K.down_weight_t_for_decode(w)
            self._down_weight_t_key = key

    def _group_offset(self, device: torch.device) -> torch.Tensor:
        """[1, groups, 1] first channel of every group of grouped_b."""
        off = self._group_offsets.get(device)
        if off is None:
            b = self.config.grouped_b
            groups = self.config.intermediate_size // b
            off = torch.arange(0, groups * b, b, device=device, dtype=torch.int64)[None, :, None]
            if not self._compile_frozen:
                self._group_offsets[device] = off
        return off

    def _workspace(self, nb: int, device: torch.device) -> torch.Tensor:
        """This module's zeroed after-gate workspace for nb tokens."""
        ws = self._after_gate_ws.get((device, nb))
        if ws is None:
            c = self.config
            ws = K.global_after_gate_workspace(nb, c.intermediate_size, c.k, c.hidden_size, device)
            self._after_gate_ws[(device, nb)] = ws
        return ws

    def _global_decode_workspace(self, nb: int, device: torch.device) -> torch.Tensor:
        """This module's zeroed gate GEMV + after-gate workspace for nb <= 16
        tokens."""
        ws = self._decode_ws.get((device, nb))
        if ws is None:
            c = self.config
            ws = K.global_decode_workspace(nb, c.intermediate_size, c.k, c.hidden_size, device)
            self._decode_ws[(device, nb)] = ws
        return ws

    def _moc28_decode_workspace(self, nb: int, device: torch.device) -> torch.Tensor:
        """This module's workspace of the 2:8 decode layer entry for nb <= 16
        tokens (G and U rows, the normalised tokens; no zeroing needed)."""
        ws = self._decode_ws.get(("2:8", device, nb))
        if ws is None:
            c = self.config
            nbytes = K.moc28_decode_workspace_bytes(nb, c.intermediate_size, c.hidden_size)
            ws = torch.empty(max(nbytes, 256), dtype=torch.uint8, device=device)
            self._decode_ws[("2:8", device, nb)] = ws
        return ws

    def _packed28_state(self, nb: int, device: torch.device):
        """Row views for nb tokens of this module's 2:4-packed operand
        buffers and zeroed sparse-Down workspace (MoC 2:8 prefill).  One set
        per device, sized for the largest batch seen so far (rounded up to
        256 rows, the positions' row block) and replaced only when a larger
        batch comes; a set used while a HIP graph was being captured is kept
        alive when it is replaced (the graph still uses it)."""
        st = self._packed28.get(device)
        c = self.config
        if st is None or st["rows"] < nb:
            if st is not None and st["captured"]:
                self._packed28_captured.append(st)
            rows = K.round_up(max(nb, 1), 256)
            ap, meta = K.packed28_buffers(rows, c.intermediate_size, device)
            ws = K.sparse28_down_workspace(rows, c.intermediate_size, c.hidden_size, device)
            st = {"rows": rows, "ap": ap, "meta": meta, "ws": ws, "captured": False}
            self._packed28[device] = st
        need = K.sparse28_down_workspace_bytes(nb, c.intermediate_size, c.hidden_size)
        if st["ws"].numel() < need:
            if st["captured"]:
                self._packed28_captured.append(dict(st))
            st["ws"] = K.sparse28_down_workspace(nb, c.intermediate_size, c.hidden_size, device)
        if torch.cuda.is_current_stream_capturing():
            st["captured"] = True
        return st["ap"][:nb], st["meta"], st["ws"]

    def freeze_for_compile(self, device: torch.device | None = None) -> None:
        """Build the derived state now and stop updating it inside forward."""
        self._compile_frozen = False
        self._ensure_down_weight_t()
        dev = device if device is not None else self.down_proj.weight.device
        if self.config.grouped:
            self._group_offset(torch.device(dev))
        self._compile_frozen = True

    # -- shapes (inference_ffn.py:131-143)
    def _flatten_decode_input(self, x: torch.Tensor):
        if x.dim() == 2:
            return x, tuple(x.shape)
        if x.dim() == 3 and x.shape[1] == 1:
            return x[:, 0, :], tuple(x.shape)
        raise ValueError(
            f"expected decode shape [batch, hidden] or [batch, 1, hidden], got {tuple(x.shape)}")

    def _restore_output_shape(self, y_2d: torch.Tensor, original_shape) -> torch.Tensor:
        return y_2d if len(original_shape) == 2 else y_2d[:, None, :]

    def _select_channels(self, gate_values: torch.Tensor):
        """(values, channel indices) of the reference's torch selection: Top-K
        over all channels, or top-a inside every group of b (:145-162)."""
        c = self.config
        if not c.grouped:
            return gate_values.topk(c.k, dim=-1, largest=True, sorted=False)
        rows = gate_values.shape[0]
        per_group = gate_values.unflatten(-1, (c.intermediate_size // c.grouped_b, c.grouped_b))
        vals, within = per_group.topk(c.grouped_a, dim=-1)
        chans = within + self._group_offset(gate_values.device)
        return vals.reshape(rows, c.k), chans.reshape(rows, c.k)

    # -- modes
    def dense_baseline(self, x: torch.Tensor) -> torch.Tensor:
        x_2d, shp = self._flatten_decode_input(x)
        y = self.down_proj(F.silu(self.gate_proj(x_2d)) * self.up_proj(x_2d))
        return self._restore_output_shape(y, shp)

    def masked_reference(self, x: torch.Tensor) -> torch.Tensor:
        x_2d, shp = self._flatten_decode_input(x)
        gate_full = self.gate_proj(x_2d)
        up_full = self.up_proj(x_2d)
        topk_vals, topk_idx = self._select_channels(gate_full)
        sparse_up = torch.gather(up_full, -1, topk_idx)
        sparse_z = F.silu(topk_vals) * sparse_up
        z_full = torch.zeros_like(gate_full)
        z_full.scatter_(-1, topk_idx, sparse_z)
        return self._restore_output_shape(self.down_proj(z_full), shp)

    def moc_inference_optimized_global_after_gate_native(self, x: torch.Tensor) -> torch.Tensor:
        """Global MoC: gfx950 gate projection, then moc_native::optimized_global_after_gate_bf16."""
        if self.config.grouped:
            raise ValueError(
                "moc_inference_optimized_global_after_gate_native requires ungrouped global MoC")
        ensure_native_ops_ready()
        self._ensure_down_weight_t()
        x_2d, shp = self._flatten_decode_input(x)
        x_2d = x_2d.contiguous()
        if x_2d.shape[0] <= 16 and x_2d.dtype == torch.bfloat16:
            # the gate GEMV and the after-gate kernel through one layer
            # entry (same results as the two steps below)
            y = K.global_decode(x_2d, self.gate_proj.weight, self.up_proj.weight,
                                self._down_weight_t, self.config.k,
                                workspace=self._global_decode_workspace(x_2d.shape[0], x_2d.device))
            return self._restore_output_shape(y, shp)
        if x_2d.shape[0] <= 16:
            gate_full = K.gemv(x_2d, self.gate_proj.weight)
        else:
            gate_full = K.linear(x_2d, self.gate_proj.weight)
        y = torch.ops.moc_native.optimized_global_after_gate_bf16.default(
            x_2d, gate_full, self.up_proj.weight, self._down_weight_t, self.config.k)
        return self._restore_output_shape(y, shp)

    def fused_decode_residual(self, x: torch.Tensor, norm_weight: torch.Tensor,
                              eps: float) -> torch.Tensor:
        """x + FFN(RMSNorm(x)) for a decoder layer's FFN half, <= 4 tokens,
        in two launches: the pre-norm runs inside the gate GEMV (global MoC)
        or the fused gate/up + top-2-of-8 kernel (MoC 2:8), the residual add
        inside the last step of the after-gate kernel or of the selected
        Down (the layer of benchmark_decode.py:303 with RMSNorm of
        :101-109).  Other shapes: the same result unfused."""
        x_2d, shp = self._flatten_decode_input(x)
        grouped28 = self.config.grouped and self.config.grouped_a == 2 and self.config.grouped_b == 8
        if grouped28 and x_2d.shape[0] <= 4 and x_2d.dtype == torch.bfloat16:
            ensure_native_ops_ready()
            self._ensure_down_weight_t()
            x_2d = x_2d.contiguous()
            c = self.config
            if K.moc28_decode_fits(x_2d.shape[0], c.intermediate_size, c.hidden_size, norm=True):
                y = K.moc28_decode(x_2d, self.gate_proj.weight, self.up_proj.weight, self._down_weight_t,
                                   norm_weight=norm_weight, eps=eps, residual=x_2d,
                                   workspace=self._moc28_decode_workspace(x_2d.shape[0], x_2d.device))
                return self._restore_output_shape(y, shp)
            idx, sz = K.grouped_top2_up_silu(x_2d, self.gate_proj.weight, self.up_proj.weight,
                                             norm_weight=norm_weight, eps=eps)
            y = K.selected_grouped_down(sz, idx, self._down_weight_t, residual=x_2d)
            return self._restore_output_shape(y, shp)
        if self.config.grouped or x_2d.shape[0] > 4 or x_2d.dtype != torch.bfloat16:
            xf = x_2d.float()
            xn = (xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + eps)).to(x_2d.dtype) * norm_weight
            return self._restore_output_shape(x_2d + self.forward(xn), shp)
        ensure_native_ops_ready()
        self._ensure_down_weight_t()
        x_2d = x_2d.contiguous()
        c = self.config
        if K.global_decode_rmsnorm_residual_fits(x_2d.shape[0], c.intermediate_size, c.k, c.hidden_size):
            y = K.global_decode_rmsnorm_residual(
                x_2d, norm_weight, eps, self.gate_proj.weight, self.up_proj.weight, self._down_weight_t, c.k,
                workspace=self._global_decode_workspace(x_2d.shape[0], x_2d.device))
            return self._restore_output_shape(y, shp)
        gate_full, xn = K.gemv_rmsnorm(x_2d, norm_weight, eps, self.gate_proj.weight)
        y = K.global_after_gate(xn, gate_full, self.up_proj.weight, self._down_weight_t,
                                self.config.k, residual=x_2d,
                                workspace=self._workspace(x_2d.shape[0], x_2d.device))
        return self._restore_output_shape(y, shp)

    def make_moc2_8_graph_runner(self, batch_size: int, gate_up_BLOCK_B: int | None = None,
                                 gate_up_BLOCK_G: int | None = None,
                                 gate_up_BLOCK_H: int | None = None,
                                 down_block_k: int | None = None,
                                 down_block_h: int | None = None):
        """Capture fused gate+up+top-2-of-8+SiLU and the selected Down in a HIP
        graph over persistent buffers (inference_ffn.py:205-279)."""
        if not (self.config.grouped and self.config.grouped_a == 2 and self.config.grouped_b == 8):
            raise ValueError("graph runner requires grouped MoC with grouped_a=2, grouped_b=8.")
        ensure_native_ops_ready()
        self._ensure_down_weight_t()
        h = self.config.hidden_size
        inter = self.config.intermediate_size
        k = (inter // 8) * 2
        device = self.gate_proj.weight.device
        dtype = self.gate_proj.weight.dtype
        x_buf = torch.zeros(batch_size, h, device=device, dtype=dtype)
        y_buf = torch.empty(batch_size, h, device=device, dtype=dtype)
        wg = self.gate_proj.weight.contiguous()
        wu = self.up_proj.weight.contiguous()
        if dtype == torch.bfloat16 and K.moc28_decode_fits(batch_size, inter, h):
            # decode batches: the gate/up GEMV pair, then the top-2-of-8 and
            # the selected Down in one launch (a workspace of the runner's own:
            # eager calls of the module never share it with the replays)
            ws = torch.empty(max(K.moc28_decode_workspace_bytes(batch_size, inter, h), 256),
                             dtype=torch.uint8, device=device)
            buffers = (x_buf, y_buf, ws)

            def _run():
                K.moc28_decode(x_buf, wg, wu, self._down_weight_t, workspace=ws, out=y_buf)
        elif batch_size > 64 and dtype == torch.bfloat16:
            # prefill batches: the selection travels 2:4-packed from the
            # gate/up epilogue to the structured-sparse Down
            ap, meta = K.packed28_buffers(batch_size, inter, device)
            ws = K.sparse28_down_workspace(batch_size, inter, h, device)
            buffers = (x_buf, y_buf, ap, meta, ws)

            def _run():
                K.grouped_top2_up_silu_packed(x_buf, wg, wu, ap, meta)
                K.sparse28_down(ap, meta, inter, self._down_weight_t, workspace=ws, out=y_buf)
        else:
            idx_buf = torch.empty(batch_size, k, device=device, dtype=torch.int64)
            sz_buf = torch.empty(batch_size, k, device=device, dtype=dtype)
            ws = torch.empty(max(1, K.selected_grouped_down_workspace_bytes(batch_size, k, inter, h)),
                             dtype=torch.uint8, device=device)
            buffers = (x_buf, y_buf, idx_buf, sz_buf, ws)

            def _run():
                fused_gate_top2of8_selected_up_silu_into(x_buf, wg, wu, topk_idx_out=idx_buf,
                                                         sparse_z_out=sz_buf)
                selected_down_from_sparse_z_into(sz_buf, idx_buf, self._down_weight_t, out=y_buf,
                                                 workspace=ws)

        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            for _ in range(3):
                _run()
        torch.cuda.current_stream().wait_stream(s)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            _run()

        def runner(x_in: torch.Tensor) -> torch.Tensor:
            x_2d, shp = self._flatten_decode_input(x_in)
            if x_2d.shape[0] != batch_size:
                raise ValueError(
                    f"MoC 2:8 graph runner built for batch_size={batch_size}, got {x_2d.shape[0]}")
            x_buf.copy_(x_2d)
            graph.replay()
            return self._restore_output_shape(y_buf, shp)

        runner.graph = graph
        # every buffer the graph reads or writes lives as long as the runner:
        # a freed one would be handed to other tensors while replays still
        # write it (and the sparse Down's workspace carries its zeroed
        # arrival counters from one replay to the next)
        runner.buffers = buffers
        return runner

    def moc_inference_grouped_top2of8(self, x: torch.Tensor) -> torch.Tensor:
        """MoC 2:8 through moc::fused_grouped_top2_up_silu + moc::selected_grouped_down."""
        if not (self.config.grouped and self.config.grouped_a == 2 and self.config.grouped_b == 8):
            raise ValueError(
                "moc_inference_grouped_top2of8 requires grouped MoC with grouped_a=2, grouped_b=8.")
        if self.config.intermediate_size % 8 != 0:
            raise ValueError(
                f"intermediate_size={self.config.intermediate_size} must be divisible by 8")
        ensure_native_ops_ready()
        self._ensure_down_weight_t()
        x_2d, shp = self._flatten_decode_input(x)
        c = self.config
        if x_2d.dtype == torch.bfloat16 and K.moc28_decode_fits(x_2d.shape[0], c.intermediate_size,
                                                                 c.hidden_size):
            # decode: the gate/up GEMV pair, then one launch that selects the
            # top 2 of every 8 channels and sums the selected Down rows
            x_2d = x_2d.contiguous()
            y = K.moc28_decode(x_2d, self.gate_proj.weight, self.up_proj.weight, self._down_weight_t,
                               workspace=self._moc28_decode_workspace(x_2d.shape[0], x_2d.device))
            return self._restore_output_shape(y, shp)
        if x_2d.shape[0] > 64 and x_2d.dtype == torch.bfloat16:
            # prefill: the gate/up epilogue writes the selection 2:4-packed and
            # the Down runs on the structured-sparse MFMA (no int64 indices)
            ap, meta, ws = self._packed28_state(x_2d.shape[0], x_2d.device)
            K.grouped_top2_up_silu_packed(x_2d, self.gate_proj.weight, self.up_proj.weight, ap, meta)
            y = K.sparse28_down(ap, meta, self.config.intermediate_size, self._down_weight_t,
                                workspace=ws)
            return self._restore_output_shape(y, shp)
        topk_idx, sparse_z = torch.ops.moc.fused_grouped_top2_up_silu.default(
            x_2d, self.gate_proj.weight, self.up_proj.weight)
        y = torch.ops.moc.selected_grouped_down.default(sparse_z, topk_idx, self._down_weight_t)
        return self._restore_output_shape(y, shp)

    def forward(self, x: torch.Tensor, mode: str = "auto") -> torch.Tensor:
        if mode == "auto":
            mode = ("moc_inference_grouped_top2of8" if self.config.grouped
                    else "moc_inference_optimized_global_after_gate_native")
        if mode == "dense_baseline":
            return self.dense_baseline(x)
        if mode == "masked_reference":
            return self.masked_reference(x)
        if mode == "moc_inference_optimized_global_after_gate_native":
            return self.moc_inference_optimized_global_after_gate_native(x)
        if mode == "moc_inference_grouped_top2of8":
            return self.moc_inference_grouped_top2of8(x)
        raise ValueError(f"unknown mode={mode}")
