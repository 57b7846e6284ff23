"""Routed-MoE decode layer on the MI355X kernels (host driver, extension).

The reference routes on the host (D2H copy + stream sync per layer,
kernel/cpp-engine-mxfp4/routed.cu:169-208), packs the top-k experts with 36
device-to-device copies (routed.cu:266-283) and runs one grouped GEMV per
token (runtime/dsv4_engine_mxfp4.py:412-423). This layer keeps everything on
the device: gating (top-k + sigmoid renormalisation) in one launch, then the
expert-indexed grouped GEMV reads the routed experts in place from the
per-layer [n_experts, ...] tensors, one launch per projection, for all T
tokens at once. Buffers are allocated once, so a forward call allocates
nothing and can be captured in a HIP graph.

Per-layer weights (MXFP4, OCP MX v1.0 packing):
    W1, W3: packed [E, hidden, K/2], scale [E, hidden, K/32]
    W2:     packed [E, out_dim, hidden/2], scale [E, out_dim, hidden/32]
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import Dict, Optional, Tuple

import torch

from . import fill
from . import mxfp4_grouped_gemv_binding as gb
from . import synth


@dataclass
class MoEWeights:
    W1: Dict[str, torch.Tensor]
    W3: Dict[str, torch.Tensor]
    W2: Dict[str, torch.Tensor]

    @property
    def n_experts(self) -> int:
        return self.W1["packed"].shape[0]

    @property
    def hidden(self) -> int:
        return self.W1["packed"].shape[1]

    @property
    def K(self) -> int:
        return self.W1["packed"].shape[2] * 2

    @property
    def out_dim(self) -> int:
        return self.W2["packed"].shape[1]

    def nbytes_per_expert(self) -> int:
        return sum(w[k][0].numel() for w in (self.W1, self.W3, self.W2) for k in ("packed", "scale"))


# Stream seeds of a layer's six tensors; the packed stream of matrix m uses
# seed_base + 4*m and its scales seed_base + 4*m + 1 (see synth.mxfp4_weight).
def _seed(seed_base: int, m: int) -> int:
    return seed_base + 4 * m


def make_moe_weights(seed_base: int, n_experts: int, K: int, hidden: int, out_dim: int,
                     device) -> MoEWeights:
    """Allocate one layer's experts on `device` and fill them with the seeded
    synthetic distribution (bytes identical to synth.mxfp4_weight)."""
    def mat(m: int, rows: int, cols: int) -> Dict[str, torch.Tensor]:
        p = torch.empty(n_experts, rows, cols // 2, dtype=torch.uint8, device=device)
        s = torch.empty(n_experts, rows, cols // 32, dtype=torch.uint8, device=device)
        fill.fill_uniform_u8(p, _seed(seed_base, m))
        fill.fill_uniform_u8(s, _seed(seed_base, m) + 1, 0, synth.SCALE_LO, synth.SCALE_HI)
        return {"packed": p, "scale": s}

    return MoEWeights(W1=mat(0, hidden, K), W3=mat(1, hidden, K), W2=mat(2, out_dim, hidden))


def expert_host_weights(seed_base: int, e: int, K: int, hidden: int, out_dim: int):
    """Host (numpy) copy of expert e of make_moe_weights(seed_base, ...):
    returns ((W1p, W1s), (W3p, W3s), (W2p, W2s)) each [rows, cols/2], [rows, cols/32]."""
    out = []
    for m, (rows, cols) in enumerate(((hidden, K), (hidden, K), (out_dim, hidden))):
        p, s = synth.mxfp4_weight(_seed(seed_base, m), rows, cols, n_mats=1, first=e)
        out.append((p[0], s[0]))
    return tuple(out)


class RoutedMoELayer:
    """Device-resident routed MoE layer -> bf16 [T, out_dim]:
        forward(x, logits=...)          config gating (sigmoid top-k renormalised);
        forward(x, ids=..., weights=...) the caller's routing;
        forward(x)                      with router_gate [E, K] bf16 given: the
                                        reference engine's routing (router GEMV,
                                        sqrt-softplus top-k x routed_scale),
                                        kernel/cpp-engine-mxfp4/routed.cu:373-503."""

    def __init__(self, weights: MoEWeights, topk: int = 8, max_tokens: int = 16,
                 check: bool = True, router_gate: Optional[torch.Tensor] = None,
                 routed_scale: float = 1.5):
        self.w = weights
        self.check = check
        self.topk = topk
        self.max_tokens = max_tokens
        self.router_gate = router_gate
        self.routed_scale = routed_scale
        dev = weights.W1["packed"].device
        self.device = dev
        if router_gate is not None:
            ws = gb.dispatch_workspace_bytes(max_tokens, topk, weights.n_experts, weights.hidden)
        else:
            ws = gb.moe_workspace_bytes(max_tokens, topk, weights.n_experts, weights.hidden)
        self.workspace = torch.empty(ws, dtype=torch.uint8, device=dev)
        self.ids = torch.empty(max_tokens, topk, dtype=torch.int32, device=dev)
        self.weights = torch.empty(max_tokens, topk, dtype=torch.float32, device=dev)
        self.out = torch.empty(max_tokens, weights.out_dim, dtype=torch.bfloat16, device=dev)

    def route(self, logits: torch.Tensor) -> Tuple[torch.Tensor, torch.Tensor]:
        T = logits.shape[0]
        return gb.route_sigmoid_topk(logits, self.topk, self.ids[:T], self.weights[:T])

    def forward(self, x: torch.Tensor, logits: Optional[torch.Tensor] = None,
                ids: Optional[torch.Tensor] = None,
                weights: Optional[torch.Tensor] = None) -> torch.Tensor:
        if x.dim() == 1:
            x = x.view(1, -1)
        T = x.shape[0]
        if T > self.max_tokens:
            raise ValueError(f"T={T} > max_tokens={self.max_tokens}")
        if logits is not None:
            return gb.mxfp4_moe_layer(x, logits, self.w.W1, self.w.W3, self.w.W2, self.topk,
                                      out=self.out[:T], ids_out=self.ids[:T],
                                      weights_out=self.weights[:T], workspace=self.workspace,
                                      check=self.check)
        if ids is None and weights is None and self.router_gate is not None:
            return gb.mxfp4_moe_routed_dispatch(x, self.router_gate, self.w.W1, self.w.W3, self.w.W2,
                                                self.topk, self.routed_scale, out=self.out[:T],
                                                ids_out=self.ids[:T], weights_out=self.weights[:T],
                                                workspace=self.workspace)
        if ids is None or weights is None:
            raise ValueError("pass logits, or ids and weights (or build the layer with a router_gate)")
        return gb.mxfp4_moe_grouped_gemv(x, self.w.W1, self.w.W3, self.w.W2, ids, weights,
                                         out=self.out[:T], workspace=self.workspace)
