"""Sparse MoE FFN with the expert loop replaced by grouped W8A8 (or W4A8) GEMMs.

Same constructor and routing as fni8serve/models/moe.py:25-113 (softmax or
sigmoid scoring, optional group-limited top-k, renormalisation, routed
scaling, optional shared expert).  The reference then loops over experts in
Python, with two host syncs per expert (moe.py:99-105); its docstring names
the grouped GEMM as the intended kernel (moe.py:9-11), and its graph runner
declines MoE layers for that reason (engine/cuda_graph.py:190-191).  On the
GPU this module runs instead, with no host sync, so a whole MoE layer can be
captured in a HIP graph:

    router GEMM       fp32 logits (torch)
    moe_route         scoring, group mask, top-k, weights in one launch
    moe_sort          stable counting sort of (token, slot) by expert
    quantize_rowwise  x quantized once per token (row-local, so every expert
                      reuses the same int8 row)
    grouped gate_up   one launch over all expert segments, rows gathered by token
    act_and_mul_quant the activation and the per-row quantization of the sorted
                      rows in one launch (bit-identical to act_and_mul then
                      quantize_rowwise)
    grouped down      one launch
    moe_combine       weighted fp16 sum in ascending expert id (index_add_ order)

Because quantization is row-local and the GEMM is exact, every int8 row, int32
accumulator and fp16 expert output equals what the per-expert loop computes.
CPU inputs run the reference's loop unchanged.

Experts of per_group_i4 int4 weights (as the reference's converter writes for
weight_bits=4, fni8serve/convert.py:130-131) run the same chain on the grouped
W4A8 GEMM when every expert of a projection shares one layout (shape, group
size 64-256, K a multiple of 256): again no host sync, and the arithmetic of
the per-expert W4A8 linears.  Other experts (mixed schemes or layouts) keep
their own GatedMLP modules (moe.py:56): on the GPU they run on the same device
routing and sort, then each non-empty expert's sorted rows go through its
GatedMLP and the same combine -- one host read of the segment offsets per
layer instead of the reference's two syncs per expert, and the same
per-expert arithmetic and index_add_ order.
"""
from __future__ import annotations

import torch
import torch.nn as nn
import torch.nn.functional as F

from .. import ops
from ..qtensor import QTensor
from .activation import fused_act, get_act_and_mul
from .mlp import GatedMLP


def _w4_stackable(qs: list[QTensor]) -> bool:
    """True when every QTensor is a per_group_i4 int4 weight of one shape and
    group size that the grouped W4A8 kernel takes (G in 64..256, K a multiple
    of 256, fp32 scales)."""
    q0 = qs[0]
    if q0.scheme != "per_group_i4" or q0.data.dim() != 2:
        return False
    N, Kh = q0.data.shape
    G = q0.group_size
    if G not in ops.W4_GROUPED_GROUPS or (2 * Kh) % 256 or (2 * Kh) % G:
        return False
    return all(q.scheme == "per_group_i4" and q.codebook == "int4" and q.group_size == G
               and q.data.dtype == torch.uint8 and tuple(q.data.shape) == (N, Kh)
               and q.scale is not None and q.scale.dtype == torch.float32
               and q.scale.numel() == N * (2 * Kh // G) and q.data.device == q0.data.device
               for q in qs)


class SparseMoE(nn.Module):
    def __init__(self, *, gate: torch.Tensor, experts: list[tuple[QTensor, QTensor]], top_k: int,
                 norm_topk_prob: bool = True, act: str = "silu",
                 shared_expert: tuple[QTensor, QTensor] | None = None,
                 shared_expert_gate: torch.Tensor | None = None, scoring_func: str = "softmax",
                 e_score_correction_bias: torch.Tensor | None = None,
                 routed_scaling_factor: float = 1.0, num_expert_groups: int | None = None,
                 topk_group: int | None = None):
        super().__init__()
        self.gate = nn.Parameter(gate)
        self.top_k = top_k
        self.norm_topk_prob = norm_topk_prob
        self.scoring_func = scoring_func
        self.routed_scaling_factor = routed_scaling_factor
        self.num_expert_groups = num_expert_groups
        self.topk_group = topk_group
        self.register_buffer(
            "e_score_bias",
            e_score_correction_bias.float() if e_score_correction_bias is not None else None,
            persistent=False)
        self.num_experts = len(experts)
        gu = [e[0] for e in experts]
        dn = [e[1] for e in experts]
        self.act_fn = get_act_and_mul(act)
        self.shared = GatedMLP(*shared_expert, act=act) if shared_expert else None
        self.shared_gate = (nn.Parameter(shared_expert_gate)
                            if shared_expert_gate is not None else None)
        self.grouped = all(q.scheme == "per_row_i8" for q in gu + dn)
        self.grouped_w4 = not self.grouped and _w4_stackable(gu) and _w4_stackable(dn)
        if self.grouped_w4:
            # per_group_i4 int4 experts of one layout per projection: stacked
            # packed weights [E, N, K/2] and group scales [E, N, K/G] for the
            # grouped W4A8 kernel; the per-expert modules keep views
            self.g_gate_up, self.g_down = gu[0].group_size, dn[0].group_size
            for name, qs in (("gate_up", gu), ("down", dn)):
                N, Kh = qs[0].data.shape
                G = qs[0].group_size
                self.register_buffer(f"w_{name}", torch.stack([q.data for q in qs]).contiguous(),
                                     persistent=False)
                self.register_buffer(
                    f"s_{name}",
                    torch.stack([q.scale.reshape(N, 2 * Kh // G) for q in qs]).contiguous(),
                    persistent=False)
            self.experts = nn.ModuleList([
                GatedMLP(QTensor(self.w_gate_up[e], self.s_gate_up[e], scheme="per_group_i4",
                                 group_size=self.g_gate_up, codebook="int4"),
                         QTensor(self.w_down[e], self.s_down[e], scheme="per_group_i4",
                                 group_size=self.g_down, codebook="int4"), act=act)
                for e in range(self.num_experts)])
            return
        if not self.grouped:
            # mixed experts, or int4 layouts the grouped kernel does not take:
            # one GatedMLP per expert on its own QTensors, as the reference
            # builds them (moe.py:56)
            self.experts = nn.ModuleList([GatedMLP(g_, d_, act=act) for g_, d_ in experts])
            return
        # Stacked expert weights [E, N, K] / scales [E, N] for the grouped kernel;
        # the per-expert modules keep views into the same storage.
        self.register_buffer("w_gate_up", torch.stack([q.data for q in gu]).contiguous(),
                             persistent=False)
        self.register_buffer("s_gate_up",
                             torch.stack([q.scale.reshape(-1).float() for q in gu]).contiguous(),
                             persistent=False)
        self.register_buffer("w_down", torch.stack([q.data for q in dn]).contiguous(),
                             persistent=False)
        self.register_buffer("s_down",
                             torch.stack([q.scale.reshape(-1).float() for q in dn]).contiguous(),
                             persistent=False)
        self.experts = nn.ModuleList([
            GatedMLP(QTensor(self.w_gate_up[e], self.s_gate_up[e], scheme="per_row_i8"),
                     QTensor(self.w_down[e], self.s_down[e], scheme="per_row_i8"), act=act)
            for e in range(self.num_experts)])

    def _gate_f32(self) -> torch.Tensor:
        """The router weight in fp32 (moe.py:64 converts it on every call); the
        copy is kept while the parameter's storage and version are unchanged."""
        w = self.gate
        key = (w.data_ptr(), w._version, w.device)
        if getattr(self, "_gate_key", None) != key:
            self._gate_cache = w.detach().float()
            self._gate_key = key
        return self._gate_cache

    def route(self, xf: torch.Tensor):
        """Router (moe.py:62-91): returns (topw in x.dtype [T, k], topi [T, k]).
        On the GPU the scoring, group mask, top-k and weights are one launch
        (`ops.moe_route`) after the fp32 router GEMM; on the CPU the
        reference's torch chain runs as written."""
        router_logits = F.linear(xf.float(), self._gate_f32())
        if xf.is_cuda:
            return ops.moe_route(router_logits, self.top_k, self.scoring_func, self.e_score_bias,
                                 self.num_expert_groups, self.topk_group, self.norm_topk_prob,
                                 self.routed_scaling_factor)
        if self.scoring_func == "sigmoid":
            scores = torch.sigmoid(router_logits)
            sel = scores + self.e_score_bias if self.e_score_bias is not None else scores
        else:
            scores = F.softmax(router_logits, dim=-1)
            sel = scores
        if self.num_expert_groups is not None and self.topk_group is not None:
            T = xf.shape[0]
            per_group = sel.shape[-1] // self.num_expert_groups
            group_scores = sel.view(T, self.num_expert_groups, per_group).amax(dim=-1)
            selected = group_scores.topk(self.topk_group, dim=-1)[1]
            offsets = torch.arange(per_group, device=sel.device).view(1, 1, per_group)
            expert_idx = (selected.unsqueeze(-1) * per_group + offsets).reshape(T, -1)
            mask = torch.full_like(sel, float("-inf"))
            mask.scatter_(1, expert_idx, 0.0)
            sel = sel + mask
        if self.scoring_func == "sigmoid":
            _, topi = torch.topk(sel, self.top_k, dim=-1)
            topw = scores.gather(-1, topi)
        else:
            topw, topi = torch.topk(sel, self.top_k, dim=-1)
        if self.norm_topk_prob:
            topw = topw / topw.sum(dim=-1, keepdim=True).clamp_min(1e-9)
        return (topw * self.routed_scaling_factor).to(xf.dtype), topi

    def experts_grouped(self, xf: torch.Tensor, topw: torch.Tensor, topi: torch.Tensor):
        """All routed experts in two grouped launches; returns out [T, H]."""
        T = xf.shape[0]
        R = T * self.top_k
        seg_off, row_token, pos = ops.moe_sort(topi, self.num_experts)
        xq, xs = ops.quantize_rowwise(xf)
        h = ops.gemm_w8a8_grouped(xq, xs, self.w_gate_up, self.s_gate_up, seg_off, R,
                                  row_index=row_token)
        act = fused_act(self.act_fn)
        if act is not None:
            aq, as_ = ops.act_and_mul_quant(h, act)
        else:
            aq, as_ = ops.quantize_rowwise(self.act_fn(h))
        y = ops.gemm_w8a8_grouped(aq, as_, self.w_down, self.s_down, seg_off, R)
        return ops.moe_combine(y, topi, topw, pos)

    def experts_grouped_w4(self, xf: torch.Tensor, topw: torch.Tensor, topi: torch.Tensor):
        """int4 experts in two grouped W4A8 launches; returns out [T, H].  The same
        chain as experts_grouped: per-token quantization once, the gate_up
        segments with rows gathered by token, the fused activation and
        quantization of the sorted rows, the down segments, the combine."""
        R = xf.shape[0] * self.top_k
        seg_off, row_token, pos = ops.moe_sort(topi, self.num_experts)
        xq, xs = ops.quantize_rowwise(xf)
        h = ops.gemm_w4a8_grouped(xq, xs, self.w_gate_up, self.s_gate_up, self.g_gate_up,
                                  seg_off, R, row_index=row_token)
        act = fused_act(self.act_fn)
        if act is not None:
            aq, as_ = ops.act_and_mul_quant(h, act)
        else:
            aq, as_ = ops.quantize_rowwise(self.act_fn(h))
        y = ops.gemm_w4a8_grouped(aq, as_, self.w_down, self.s_down, self.g_down, seg_off, R)
        return ops.moe_combine(y, topi, topw, pos)

    def experts_sorted(self, xf: torch.Tensor, topw: torch.Tensor, topi: torch.Tensor):
        """Experts that are not per_row_i8 (the W4A8 path): device sort, one host
        read of the segment offsets, each non-empty expert's GatedMLP on its
        sorted rows (ascending token, then slot: the rows nonzero() gives it at
        moe.py:103), then the device combine in ascending expert order."""
        R = xf.shape[0] * self.top_k
        seg_off, row_token, pos = ops.moe_sort(topi, self.num_experts)
        y = torch.empty((R, xf.shape[1]), dtype=xf.dtype, device=xf.device)
        bounds = seg_off.tolist()
        for e in range(self.num_experts):
            lo, hi = bounds[e], bounds[e + 1]
            if hi > lo:
                y[lo:hi] = self.experts[e](xf[row_token[lo:hi].long()])
        return ops.moe_combine(y, topi, topw, pos)

    def _experts_loop(self, xf: torch.Tensor, topw: torch.Tensor, topi: torch.Tensor):
        """The reference's per-expert loop (moe.py:97-105), for CPU inputs."""
        out = torch.zeros_like(xf)
        for e in range(self.num_experts):
            mask = topi == e
            if not mask.any():
                continue
            tok_idx, slot = mask.nonzero(as_tuple=True)
            contrib = self.experts[e](xf[tok_idx].unsqueeze(1)).squeeze(1)
            out.index_add_(0, tok_idx, contrib * topw[tok_idx, slot].unsqueeze(-1))
        return out

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        B, S, H = x.shape
        xf = x.reshape(-1, H)
        topw, topi = self.route(xf)
        if xf.is_cuda:
            if self.grouped:
                out = self.experts_grouped(xf, topw, topi)
            elif self.grouped_w4:
                out = self.experts_grouped_w4(xf, topw, topi)
            else:
                out = self.experts_sorted(xf, topw, topi)
        else:
            out = self._experts_loop(xf, topw, topi)
        if self.shared is not None:
            shared_out = self.shared(x).reshape(-1, H)
            if self.shared_gate is not None:
                g = torch.sigmoid(F.linear(xf.float(), self.shared_gate.float())).to(x.dtype)
                shared_out = shared_out * g
            out = out + shared_out
        return out.reshape(B, S, H)
