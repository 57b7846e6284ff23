"""ctypes binding of libmxfp4_grouped_gemv.so (routed MXFP4 SwiGLU MoE).

Drop-in API (same call contract as the reference binding
runtime/mxfp4_grouped_gemv_binding.py:95-174):

    mxfp4_grouped_gemv(W1, W3, W2, scales, x, r) -> out [out_dim] bf16

    W1, W3: {'packed': uint8 [n_exp, hidden, K_in/2], 'scale': uint8 [n_exp, hidden, K_in/32]}
    W2:     {'packed': uint8 [n_exp, out_dim, hidden/2], 'scale': uint8 [n_exp, out_dim, hidden/32]}
    scales: ignored (the scales live in W{1,3,2}['scale'])
    x:      bf16 [K_in];  r: float32 [n_exp]

Extensions (not in the reference):

    route_sigmoid_topk(logits [T, E] f32, topk) -> (ids [T, topk] int32, weights [T, topk] f32)
    route_topk(logits, topk, score_mode, routed_scale) -> (ids, weights)   (either gating)
    router_logits(x [T, K] bf16, W_gate [E, K] bf16) -> logits [T, E] f32
    mxfp4_moe_routed_dispatch(x, W_gate, W1, W3, W2, topk, routed_scale=1.5)
        the reference engine's routed dispatch (router GEMV + sqrt-softplus
        top-k + grouped GEMV) on the device
    mxfp4_moe_grouped_gemv(x [T, K_in], W1, W3, W2, ids, weights, out=None, workspace=None)
        experts read in place from per-layer tensors [n_experts, ...].

Errors: ValueError for device/dtype/shape/contiguity problems, RuntimeError for
a non-zero return code of the library. The library path is
$MXFP4_GROUPED_LIB or kernel/mxfp4-routed/libmxfp4_grouped_gemv.so.
"""
from __future__ import annotations

import ctypes
from typing import Any, Dict, Optional, Tuple

import torch

from . import _lib

MXFP4_BLOCK_ELEMS = 32

_c_int, _c_void_p, _c_size_t = ctypes.c_int, ctypes.c_void_p, ctypes.c_size_t
_LIB: Optional[ctypes.CDLL] = None


def lib_path() -> str:
    return _lib.lib_path("MXFP4_GROUPED_LIB", "mxfp4-routed", "libmxfp4_grouped_gemv.so")


def _load_lib() -> ctypes.CDLL:
    global _LIB
    if _LIB is not None:
        return _LIB
    lib = _lib.load(lib_path())
    lib.mxfp4_grouped_gemv_topk.restype = _c_int
    lib.mxfp4_grouped_gemv_topk.argtypes = [_c_void_p] * 8 + [_c_int] * 4 + [_c_void_p] * 3
    lib.mxfp4_grouped_workspace_bytes.restype = _c_size_t
    lib.mxfp4_grouped_workspace_bytes.argtypes = [_c_int] * 3
    lib.mxfp4_moe_route_sigmoid_topk.restype = _c_int
    lib.mxfp4_moe_route_sigmoid_topk.argtypes = [_c_void_p, _c_int, _c_int, _c_int,
                                                 _c_void_p, _c_void_p, _c_void_p]
    lib.mxfp4_moe_workspace_bytes.restype = _c_size_t
    lib.mxfp4_moe_workspace_bytes.argtypes = [_c_int] * 4
    lib.mxfp4_moe_grouped_gemv.restype = _c_int
    lib.mxfp4_moe_grouped_gemv.argtypes = ([_c_void_p] * 9 + [_c_int] * 6 + [_c_void_p] * 3)
    lib.mxfp4_moe_build_routing.restype = _c_int
    lib.mxfp4_moe_build_routing.argtypes = [_c_void_p] * 2 + [_c_int] * 4 + [_c_void_p] * 2
    lib.mxfp4_moe_swiglu.restype = _c_int
    lib.mxfp4_moe_swiglu.argtypes = [_c_void_p] * 5 + [_c_int] * 5 + [_c_void_p] * 2
    lib.mxfp4_moe_down.restype = _c_int
    lib.mxfp4_moe_down.argtypes = [_c_void_p] * 2 + [_c_int] * 5 + [_c_void_p] * 3
    lib.mxfp4_moe_layer.restype = _c_int
    lib.mxfp4_moe_layer.argtypes = [_c_void_p] * 8 + [_c_int] * 6 + [_c_void_p] * 5
    lib.mxfp4_moe_prefill_workspace_bytes.restype = _c_size_t
    lib.mxfp4_moe_prefill_workspace_bytes.argtypes = [_c_int] * 5
    lib.mxfp4_moe_prefill.restype = _c_int
    lib.mxfp4_moe_prefill.argtypes = [_c_void_p] * 9 + [_c_int] * 6 + [_c_void_p] * 3
    lib.mxfp4_moe_prefill_dequant_bf16.restype = _c_int
    lib.mxfp4_moe_prefill_dequant_bf16.argtypes = [_c_void_p] * 2 + [_c_int] * 2 + [_c_void_p] * 2
    lib.mxfp4_moe_route_topk.restype = _c_int
    lib.mxfp4_moe_route_topk.argtypes = [_c_void_p] + [_c_int] * 4 + [ctypes.c_float] + [_c_void_p] * 3
    lib.mxfp4_moe_router_logits.restype = _c_int
    lib.mxfp4_moe_router_logits.argtypes = [_c_void_p] * 2 + [_c_int] * 3 + [_c_void_p] * 2
    lib.mxfp4_moe_dispatch_workspace_bytes.restype = _c_size_t
    lib.mxfp4_moe_dispatch_workspace_bytes.argtypes = [_c_int] * 4
    lib.mxfp4_moe_gate_swiglu.restype = _c_int
    lib.mxfp4_moe_gate_swiglu.argtypes = [_c_void_p] * 6 + [_c_int] * 5 + [_c_void_p] * 4
    lib.mxfp4_moe_grouped_gemv_noalloc.restype = _c_int
    lib.mxfp4_moe_grouped_gemv_noalloc.argtypes = ([_c_void_p] * 9 + [_c_int] * 6 + [_c_void_p] * 2)
    lib.mxfp4_moe_routed_dispatch.restype = _c_int
    lib.mxfp4_moe_routed_dispatch.argtypes = ([_c_void_p] * 8 + [_c_int] * 6 + [ctypes.c_float] +
                                             [_c_void_p] * 5)
    _LIB = lib
    return lib


def _check(t: torch.Tensor, name: str, dtype: torch.dtype) -> None:
    if not t.is_cuda:
        raise ValueError(f"{name}: expected a GPU tensor, got device={t.device}")
    if t.dtype != dtype:
        raise ValueError(f"{name}: expected dtype {dtype}, got {t.dtype}")
    if not t.is_contiguous():
        raise ValueError(f"{name}: tensor must be contiguous")


def _check_mats(W1, W3, W2) -> None:
    for name, w in (("W1", W1), ("W3", W3), ("W2", W2)):
        if "packed" not in w or "scale" not in w:
            raise ValueError(f"{name} must contain 'packed' and 'scale' tensors")
        _check(w["packed"], f"{name}.packed", torch.uint8)
        _check(w["scale"], f"{name}.scale", torch.uint8)
        if w["packed"].dim() != 3 or w["scale"].dim() != 3:
            raise ValueError(f"{name}: packed/scale must be 3-D [experts, rows, cols]")


def _shapes(W1, W3, W2, K_in: int) -> Tuple[int, int, int]:
    n_exp, hidden = W1["packed"].shape[0], W1["packed"].shape[1]
    out_dim = W2["packed"].shape[1]
    if tuple(W3["packed"].shape) != tuple(W1["packed"].shape):
        raise ValueError(f"W3.packed shape {tuple(W3['packed'].shape)} != W1.packed shape "
                         f"{tuple(W1['packed'].shape)}")
    if W1["packed"].shape[2] != K_in // 2:
        raise ValueError(f"W1.packed last dim {W1['packed'].shape[2]} != K_in/2={K_in // 2}")
    want = (n_exp, hidden, K_in // MXFP4_BLOCK_ELEMS)
    if tuple(W1["scale"].shape) != want or tuple(W3["scale"].shape) != want:
        raise ValueError(f"W1/W3.scale shape must be {want}")
    if W2["packed"].shape[0] != n_exp or W2["packed"].shape[2] != hidden // 2:
        raise ValueError(f"W2.packed shape {tuple(W2['packed'].shape)} != "
                         f"({n_exp}, out_dim, {hidden // 2})")
    want2 = (n_exp, out_dim, hidden // MXFP4_BLOCK_ELEMS)
    if tuple(W2["scale"].shape) != want2:
        raise ValueError(f"W2.scale shape {tuple(W2['scale'].shape)} != {want2}")
    return n_exp, hidden, out_dim


def workspace_bytes(n_exp: int, hidden: int, out_dim: int) -> int:
    return int(_load_lib().mxfp4_grouped_workspace_bytes(n_exp, hidden, out_dim))


def mxfp4_grouped_gemv(
    W1: Dict[str, torch.Tensor],
    W3: Dict[str, torch.Tensor],
    W2: Dict[str, torch.Tensor],
    scales: Any,
    x: torch.Tensor,
    r: torch.Tensor,
    out: Optional[torch.Tensor] = None,
    workspace: Optional[torch.Tensor] = None,
) -> torch.Tensor:
    """Routed SwiGLU over the n_exp packed experts for one token; returns bf16 [out_dim].

    `out` and `workspace` may be passed to avoid per-call allocation (the
    reference allocates both on every call).
    """
    del scales
    lib = _load_lib()
    _check(x, "x", torch.bfloat16)
    _check(r, "r", torch.float32)
    _check_mats(W1, W3, W2)
    K_in = x.numel()
    n_exp, hidden, out_dim = _shapes(W1, W3, W2, K_in)
    if tuple(r.shape) != (n_exp,):
        raise ValueError(f"r shape {tuple(r.shape)} != ({n_exp},)")
    if out is None:
        out = torch.empty(out_dim, dtype=torch.bfloat16, device=x.device)
    else:
        _check(out, "out", torch.bfloat16)
        if out.numel() != out_dim:
            raise ValueError(f"out numel {out.numel()} != {out_dim}")
    ws_bytes = lib.mxfp4_grouped_workspace_bytes(n_exp, hidden, out_dim)
    if workspace is None:
        workspace = torch.empty(ws_bytes, dtype=torch.uint8, device=x.device)
    elif workspace.numel() * workspace.element_size() < ws_bytes:
        raise ValueError(f"workspace smaller than {ws_bytes} bytes")
    rc = lib.mxfp4_grouped_gemv_topk(
        _lib.vp(x), _lib.vp(W1["packed"]), _lib.vp(W3["packed"]), _lib.vp(W2["packed"]),
        _lib.vp(W1["scale"]), _lib.vp(W3["scale"]), _lib.vp(W2["scale"]), _lib.vp(r),
        K_in, hidden, out_dim, n_exp, _lib.vp(out), _lib.vp(workspace),
        ctypes.c_void_p(_lib.stream_ptr(x.device)))
    if rc != 0:
        raise RuntimeError(f"mxfp4_grouped_gemv_topk returned {rc}")
    return out


def route_sigmoid_topk(logits: torch.Tensor, topk: int,
                       ids: Optional[torch.Tensor] = None,
                       weights: Optional[torch.Tensor] = None) -> Tuple[torch.Tensor, torch.Tensor]:
    """Device gating: top-k of logits [T, E] with sigmoid weights renormalised to 1."""
    lib = _load_lib()
    _check(logits, "logits", torch.float32)
    if logits.dim() != 2:
        raise ValueError("logits must be [T, n_experts]")
    T, E = logits.shape
    if ids is None:
        ids = torch.empty(T, topk, dtype=torch.int32, device=logits.device)
    if weights is None:
        weights = torch.empty(T, topk, dtype=torch.float32, device=logits.device)
    _check(ids, "ids", torch.int32)
    _check(weights, "weights", torch.float32)
    rc = lib.mxfp4_moe_route_sigmoid_topk(_lib.vp(logits), T, E, topk, _lib.vp(ids),
                                          _lib.vp(weights),
                                          ctypes.c_void_p(_lib.stream_ptr(logits.device)))
    if rc != 0:
        raise RuntimeError(f"mxfp4_moe_route_sigmoid_topk returned {rc}")
    return ids, weights


SCORE_SIGMOID = 0          # benchmark configuration gating
SCORE_SQRT_SOFTPLUS = 1    # the reference engine's router (routed.cu:156-208)


def route_topk(logits: torch.Tensor, topk: int, score_mode: int = SCORE_SQRT_SOFTPLUS,
               routed_scale: float = 1.5, ids: Optional[torch.Tensor] = None,
               weights: Optional[torch.Tensor] = None) -> Tuple[torch.Tensor, torch.Tensor]:
    """Device gating of logits [T, E] with a choice of scoring (SCORE_SIGMOID or
    SCORE_SQRT_SOFTPLUS with routed_scale); returns (ids, weights) [T, topk]."""
    lib = _load_lib()
    _check(logits, "logits", torch.float32)
    if logits.dim() != 2:
        raise ValueError("logits must be [T, n_experts]")
    T, E = logits.shape
    if ids is None:
        ids = torch.empty(T, topk, dtype=torch.int32, device=logits.device)
    if weights is None:
        weights = torch.empty(T, topk, dtype=torch.float32, device=logits.device)
    _check(ids, "ids", torch.int32)
    _check(weights, "weights", torch.float32)
    rc = lib.mxfp4_moe_route_topk(_lib.vp(logits), T, E, topk, int(score_mode), float(routed_scale),
                                  _lib.vp(ids), _lib.vp(weights),
                                  ctypes.c_void_p(_lib.stream_ptr(logits.device)))
    if rc != 0:
        raise RuntimeError(f"mxfp4_moe_route_topk returned {rc}")
    return ids, weights


def router_logits(x: torch.Tensor, W_gate: torch.Tensor, out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Router gate GEMV: logits [T, E] fp32 = x [T, K] bf16 @ W_gate [E, K] bf16 ^T."""
    lib = _load_lib()
    _check(x, "x", torch.bfloat16)
    _check(W_gate, "W_gate", torch.bfloat16)
    if x.dim() == 1:
        x = x.view(1, -1)
    T, K = x.shape
    if W_gate.dim() != 2 or W_gate.shape[1] != K:
        raise ValueError(f"W_gate shape {tuple(W_gate.shape)} != (n_experts, {K})")
    E = W_gate.shape[0]
    if out is None:
        out = torch.empty(T, E, dtype=torch.float32, device=x.device)
    _check(out, "out", torch.float32)
    if out.numel() != T * E:
        raise ValueError(f"out numel {out.numel()} != {T * E}")
    rc = lib.mxfp4_moe_router_logits(_lib.vp(x), _lib.vp(W_gate), T, E, K, _lib.vp(out),
                                     ctypes.c_void_p(_lib.stream_ptr(x.device)))
    if rc != 0:
        raise RuntimeError(f"mxfp4_moe_router_logits returned {rc}")
    return out


def dispatch_workspace_bytes(T: int, topk: int, n_experts: int, hidden: int) -> int:
    return int(_load_lib().mxfp4_moe_dispatch_workspace_bytes(T, topk, n_experts, hidden))


def mxfp4_moe_routed_dispatch(
    x: torch.Tensor,
    W_gate: torch.Tensor,
    W1: Dict[str, torch.Tensor],
    W3: Dict[str, torch.Tensor],
    W2: Dict[str, torch.Tensor],
    topk: int,
    routed_scale: float = 1.5,
    out: Optional[torch.Tensor] = None,
    ids_out: Optional[torch.Tensor] = None,
    weights_out: Optional[torch.Tensor] = None,
    workspace: Optional[torch.Tensor] = None,
) -> torch.Tensor:
    """The reference engine's routed dispatch on the device (router GEMV,
    sqrt-softplus top-k x routed_scale, expert-indexed grouped GEMV) for
    x [T, K_in]; returns bf16 [T, out_dim]."""
    lib = _load_lib()
    _check(x, "x", torch.bfloat16)
    _check(W_gate, "W_gate", torch.bfloat16)
    _check_mats(W1, W3, W2)
    if x.dim() == 1:
        x = x.view(1, -1)
    T, K_in = x.shape
    n_experts, hidden, out_dim = _shapes(W1, W3, W2, K_in)
    if tuple(W_gate.shape) != (n_experts, K_in):
        raise ValueError(f"W_gate shape {tuple(W_gate.shape)} != ({n_experts}, {K_in})")
    if out is None:
        out = torch.empty(T, out_dim, dtype=torch.bfloat16, device=x.device)
    _check(out, "out", torch.bfloat16)
    if out.numel() != T * out_dim:
        raise ValueError(f"out numel {out.numel()} != {T * out_dim}")
    need = lib.mxfp4_moe_dispatch_workspace_bytes(T, topk, n_experts, hidden)
    if workspace is None:
        workspace = torch.empty(need, dtype=torch.uint8, device=x.device)
    elif workspace.numel() * workspace.element_size() < need:
        raise ValueError(f"workspace smaller than {need} bytes")
    for name, t, dt in (("ids_out", ids_out, torch.int32), ("weights_out", weights_out, torch.float32)):
        if t is not None:
            _check(t, name, dt)
            if t.numel() != T * topk:
                raise ValueError(f"{name} numel {t.numel()} != {T * topk}")
    rc = lib.mxfp4_moe_routed_dispatch(
        _lib.vp(x), _lib.vp(W_gate), _lib.vp(W1["packed"]), _lib.vp(W3["packed"]), _lib.vp(W2["packed"]),
        _lib.vp(W1["scale"]), _lib.vp(W3["scale"]), _lib.vp(W2["scale"]), T, topk, n_experts, K_in, hidden,
        out_dim, float(routed_scale), _lib.vp(out), None if ids_out is None else _lib.vp(ids_out),
        None if weights_out is None else _lib.vp(weights_out), _lib.vp(workspace),
        ctypes.c_void_p(_lib.stream_ptr(x.device)))
    if rc != 0:
        raise RuntimeError(f"mxfp4_moe_routed_dispatch returned {rc}")
    return out


def prefill_dequant(W_packed: torch.Tensor, W_scale: torch.Tensor) -> torch.Tensor:
    """Debug: [N, K/2] + [N, K/32] -> bf16 [N, K] with the prefill GEMMs' decode."""
    lib = _load_lib()
    _check(W_packed, "W_packed", torch.uint8)
    _check(W_scale, "W_scale", torch.uint8)
    N, K = W_packed.shape[0], W_packed.shape[1] * 2
    if tuple(W_scale.shape) != (N, K // MXFP4_BLOCK_ELEMS):
        raise ValueError(f"W_scale shape {tuple(W_scale.shape)} != ({N}, {K // MXFP4_BLOCK_ELEMS})")
    out = torch.empty(N, K, dtype=torch.bfloat16, device=W_packed.device)
    rc = lib.mxfp4_moe_prefill_dequant_bf16(_lib.vp(W_packed), _lib.vp(W_scale), K, N, _lib.vp(out),
                                            ctypes.c_void_p(_lib.stream_ptr(W_packed.device)))
    if rc != 0:
        raise RuntimeError(f"mxfp4_moe_prefill_dequant_bf16 returned {rc}")
    return out


def moe_workspace_bytes(T: int, topk: int, n_experts: int, hidden: int) -> int:
    return int(_load_lib().mxfp4_moe_workspace_bytes(T, topk, n_experts, hidden))


def mxfp4_moe_grouped_gemv(
    x: torch.Tensor,
    W1: Dict[str, torch.Tensor],
    W3: Dict[str, torch.Tensor],
    W2: Dict[str, torch.Tensor],
    ids: torch.Tensor,
    weights: torch.Tensor,
    out: Optional[torch.Tensor] = None,
    workspace: Optional[torch.Tensor] = None,
) -> torch.Tensor:
    """Expert-indexed routed SwiGLU for T tokens; returns bf16 [T, out_dim]."""
    lib = _load_lib()
    _check(x, "x", torch.bfloat16)
    _check(ids, "ids", torch.int32)
    _check(weights, "weights", torch.float32)
    _check_mats(W1, W3, W2)
    if x.dim() == 1:
        x = x.view(1, -1)
    T, K_in = x.shape
    n_experts, hidden, out_dim = _shapes(W1, W3, W2, K_in)
    if ids.dim() != 2 or ids.shape[0] != T or tuple(weights.shape) != tuple(ids.shape):
        raise ValueError(f"ids/weights must both be [T={T}, topk]")
    topk = ids.shape[1]
    if out is None:
        out = torch.empty(T, out_dim, dtype=torch.bfloat16, device=x.device)
    else:
        _check(out, "out", torch.bfloat16)
        if out.numel() != T * out_dim:
            raise ValueError(f"out numel {out.numel()} != {T * out_dim}")
    ws_bytes = lib.mxfp4_moe_workspace_bytes(T, topk, n_experts, hidden)
    if workspace is None:
        workspace = torch.empty(ws_bytes, dtype=torch.uint8, device=x.device)
    elif workspace.numel() * workspace.element_size() < ws_bytes:
        raise ValueError(f"workspace smaller than {ws_bytes} bytes")
    rc = lib.mxfp4_moe_grouped_gemv(
        _lib.vp(x), _lib.vp(W1["packed"]), _lib.vp(W3["packed"]), _lib.vp(W2["packed"]),
        _lib.vp(W1["scale"]), _lib.vp(W3["scale"]), _lib.vp(W2["scale"]),
        _lib.vp(ids), _lib.vp(weights), T, topk, n_experts, K_in, hidden, out_dim,
        _lib.vp(out), _lib.vp(workspace), ctypes.c_void_p(_lib.stream_ptr(x.device)))
    if rc != 0:
        raise RuntimeError(f"mxfp4_moe_grouped_gemv returned {rc}")
    return out


def prefill_workspace_bytes(T: int, topk: int, n_experts: int, hidden: int, out_dim: int) -> int:
    return int(_load_lib().mxfp4_moe_prefill_workspace_bytes(T, topk, n_experts, hidden, out_dim))


def mxfp4_moe_prefill(
    x: torch.Tensor,
    W1: Dict[str, torch.Tensor],
    W3: Dict[str, torch.Tensor],
    W2: Dict[str, torch.Tensor],
    ids: torch.Tensor,
    weights: torch.Tensor,
    out: Optional[torch.Tensor] = None,
    workspace: Optional[torch.Tensor] = None,
) -> torch.Tensor:
    """Routed SwiGLU for a prefill chunk of T tokens on the matrix cores
    (same result as mxfp4_moe_grouped_gemv); returns bf16 [T, out_dim]."""
    lib = _load_lib()
    _check(x, "x", torch.bfloat16)
    _check(ids, "ids", torch.int32)
    _check(weights, "weights", torch.float32)
    _check_mats(W1, W3, W2)
    if x.dim() == 1:
        x = x.view(1, -1)
    T, K_in = x.shape
    n_experts, hidden, out_dim = _shapes(W1, W3, W2, K_in)
    if ids.dim() != 2 or ids.shape[0] != T or tuple(weights.shape) != tuple(ids.shape):
        raise ValueError(f"ids/weights must both be [T={T}, topk]")
    topk = ids.shape[1]
    if out is None:
        out = torch.empty(T, out_dim, dtype=torch.bfloat16, device=x.device)
    else:
        _check(out, "out", torch.bfloat16)
        if out.numel() != T * out_dim:
            raise ValueError(f"out numel {out.numel()} != {T * out_dim}")
    ws_bytes = prefill_workspace_bytes(T, topk, n_experts, hidden, out_dim)
    if ws_bytes == 0:
        raise ValueError(f"unsupported prefill shape T={T} topk={topk} E={n_experts} "
                         f"K={K_in} H={hidden} O={out_dim}")
    if workspace is None:
        workspace = torch.empty(ws_bytes, dtype=torch.uint8, device=x.device)
    elif workspace.numel() * workspace.element_size() < ws_bytes:
        raise ValueError(f"workspace smaller than {ws_bytes} bytes")
    rc = lib.mxfp4_moe_prefill(
        _lib.vp(x), _lib.vp(W1["packed"]), _lib.vp(W3["packed"]), _lib.vp(W2["packed"]),
        _lib.vp(W1["scale"]), _lib.vp(W3["scale"]), _lib.vp(W2["scale"]),
        _lib.vp(ids), _lib.vp(weights), T, topk, n_experts, K_in, hidden, out_dim,
        _lib.vp(out), _lib.vp(workspace), ctypes.c_void_p(_lib.stream_ptr(x.device)))
    if rc != 0:
        raise RuntimeError(f"mxfp4_moe_prefill returned {rc}")
    return out


def mxfp4_moe_layer(
    x: torch.Tensor,
    logits: torch.Tensor,
    W1: Dict[str, torch.Tensor],
    W3: Dict[str, torch.Tensor],
    W2: Dict[str, torch.Tensor],
    topk: int,
    out: Optional[torch.Tensor] = None,
    ids_out: Optional[torch.Tensor] = None,
    weights_out: Optional[torch.Tensor] = None,
    workspace: Optional[torch.Tensor] = None,
    check: bool = True,
) -> torch.Tensor:
    """Routed-MoE layer at decode in one library call: device gating of logits
    [T, E] + expert-indexed grouped GEMV; returns bf16 [T, out_dim].
    `check=False` skips the Python-side validation (the library still
    validates shapes) for callers that reuse checked buffers in a loop."""
    lib = _load_lib()
    if x.dim() == 1:
        x = x.view(1, -1)
    T, K_in = x.shape
    n_experts, hidden = W1["packed"].shape[0], W1["packed"].shape[1]
    out_dim = W2["packed"].shape[1]
    if check:
        _check(x, "x", torch.bfloat16)
        _check(logits, "logits", torch.float32)
        _check_mats(W1, W3, W2)
        _shapes(W1, W3, W2, K_in)
        if tuple(logits.shape) != (T, n_experts):
            raise ValueError(f"logits shape {tuple(logits.shape)} != ({T}, {n_experts})")
    if out is None:
        out = torch.empty(T, out_dim, dtype=torch.bfloat16, device=x.device)
    if workspace is None:
        workspace = torch.empty(lib.mxfp4_moe_workspace_bytes(T, topk, n_experts, hidden),
                                dtype=torch.uint8, device=x.device)
    if check:
        _check(out, "out", torch.bfloat16)
        if out.numel() != T * out_dim:
            raise ValueError(f"out numel {out.numel()} != {T * out_dim}")
        need = lib.mxfp4_moe_workspace_bytes(T, topk, n_experts, hidden)
        if workspace.numel() * workspace.element_size() < need:
            raise ValueError(f"workspace smaller than {need} bytes")
        for name, t, dt in (("ids_out", ids_out, torch.int32), ("weights_out", weights_out, torch.float32)):
            if t is not None:
                _check(t, name, dt)
                if t.numel() != T * topk:
                    raise ValueError(f"{name} numel {t.numel()} != {T * topk}")
    rc = lib.mxfp4_moe_layer(
        _lib.vp(x), _lib.vp(logits), _lib.vp(W1["packed"]), _lib.vp(W3["packed"]),
        _lib.vp(W2["packed"]), _lib.vp(W1["scale"]), _lib.vp(W3["scale"]), _lib.vp(W2["scale"]),
        T, topk, n_experts, K_in, hidden, out_dim, _lib.vp(out),
        None if ids_out is None else _lib.vp(ids_out),
        None if weights_out is None else _lib.vp(weights_out),
        _lib.vp(workspace), ctypes.c_void_p(_lib.stream_ptr(x.device)))
    if rc != 0:
        raise RuntimeError(f"mxfp4_moe_layer returned {rc}")
    return out


class MoEStages:
    """The three launches of the general mxfp4_moe_grouped_gemv path (routing
    kernel, stage A, stage B), callable one by one on a fixed workspace
    (preallocated here): build_routing(ids, weights) -> swiglu(x) -> down(out).
    At T = 1 mxfp4_moe_grouped_gemv itself runs two launches (stage A forms the
    routing) with the same results."""

    def __init__(self, W1, W3, W2, T: int, topk: int, device):
        self.lib = _load_lib()
        _check_mats(W1, W3, W2)
        self.W1, self.W3, self.W2 = W1, W3, W2
        self.n_experts, self.hidden = W1["packed"].shape[0], W1["packed"].shape[1]
        self.K = W1["packed"].shape[2] * 2
        self.out_dim = W2["packed"].shape[1]
        self.T, self.topk = T, topk
        ws = self.lib.mxfp4_moe_workspace_bytes(T, topk, self.n_experts, self.hidden)
        self.workspace = torch.empty(ws, dtype=torch.uint8, device=device)

    def _rc(self, name: str, rc: int) -> None:
        if rc != 0:
            raise RuntimeError(f"{name} returned {rc}")

    def build_routing(self, ids: torch.Tensor, weights: torch.Tensor) -> None:
        self._rc("mxfp4_moe_build_routing", self.lib.mxfp4_moe_build_routing(
            _lib.vp(ids), _lib.vp(weights), self.T, self.topk, self.n_experts, self.hidden,
            _lib.vp(self.workspace), ctypes.c_void_p(_lib.stream_ptr(ids.device))))

    def swiglu(self, x: torch.Tensor) -> None:
        self._rc("mxfp4_moe_swiglu", self.lib.mxfp4_moe_swiglu(
            _lib.vp(x), _lib.vp(self.W1["packed"]), _lib.vp(self.W3["packed"]),
            _lib.vp(self.W1["scale"]), _lib.vp(self.W3["scale"]), self.T, self.topk,
            self.n_experts, self.K, self.hidden, _lib.vp(self.workspace),
            ctypes.c_void_p(_lib.stream_ptr(x.device))))

    def gate_swiglu(self, x: torch.Tensor, logits: torch.Tensor, ids_out: Optional[torch.Tensor] = None,
                    weights_out: Optional[torch.Tensor] = None) -> None:
        """Gating of logits [T, E] and stage A (the first part of
        mxfp4_moe_layer); down() completes the layer."""
        self._rc("mxfp4_moe_gate_swiglu", self.lib.mxfp4_moe_gate_swiglu(
            _lib.vp(x), _lib.vp(logits), _lib.vp(self.W1["packed"]), _lib.vp(self.W3["packed"]),
            _lib.vp(self.W1["scale"]), _lib.vp(self.W3["scale"]), self.T, self.topk, self.n_experts, self.K,
            self.hidden, None if ids_out is None else _lib.vp(ids_out),
            None if weights_out is None else _lib.vp(weights_out), _lib.vp(self.workspace),
            ctypes.c_void_p(_lib.stream_ptr(x.device))))

    def down(self, out: torch.Tensor) -> torch.Tensor:
        self._rc("mxfp4_moe_down", self.lib.mxfp4_moe_down(
            _lib.vp(self.W2["packed"]), _lib.vp(self.W2["scale"]), self.T, self.topk,
            self.n_experts, self.hidden, self.out_dim, _lib.vp(out), _lib.vp(self.workspace),
            ctypes.c_void_p(_lib.stream_ptr(out.device))))
        return out


__all__ = ["mxfp4_grouped_gemv", "MoEStages", "mxfp4_moe_layer", "MXFP4_BLOCK_ELEMS", "route_sigmoid_topk",
           "mxfp4_moe_grouped_gemv", "moe_workspace_bytes", "workspace_bytes", "route_topk", "router_logits",
           "mxfp4_moe_routed_dispatch", "dispatch_workspace_bytes", "prefill_dequant", "SCORE_SIGMOID",
           "SCORE_SQRT_SOFTPLUS"]
