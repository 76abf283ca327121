"""Torch-facing wrappers of the C ABI in include/moe_mi355x.h.

Tensors are device tensors; bf16 data is carried as ``torch.bfloat16``,
expert indices as ``torch.int32`` (the ABI's uint32 values are < 2**31), packed
weights as ``torch.int32`` / ``torch.uint32`` (bit patterns).  Every call runs
on the current HIP stream of the tensor's device and is asynchronous.
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass
from typing import Optional

import torch

from . import BlockAux, BlockDesc, QWeightC, RouterParams, check, lib

_NULL = ctypes.c_void_p(0)


def _p(t: Optional[torch.Tensor]) -> ctypes.c_void_p:
    return _NULL if t is None else ctypes.c_void_p(t.data_ptr())


def _stream(device: torch.device) -> ctypes.c_void_p:
    return ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)


def _need(cond: bool, msg: str) -> None:
    if not cond:
        raise ValueError(msg)


def _dev(t: torch.Tensor, dtype: torch.dtype, name: str) -> None:
    _need(t.is_cuda, f"{name} must be a device tensor")
    _need(t.dtype == dtype, f"{name} must be {dtype}, got {t.dtype}")
    _need(t.is_contiguous(), f"{name} must be contiguous")


@dataclass
class QuantizedWeight:
    """One stacked projection [experts, N, K] in MLX affine layout.

    ``w`` int32/uint32 [E, N, K*bits/32]; ``scales``/``biases`` bf16
    [E, N, K/group_size].  (reference include/mlx-lm/common/quantized_linear.h:16-21)
    """

    w: torch.Tensor
    scales: torch.Tensor
    biases: Optional[torch.Tensor]
    group_size: int
    bits: int
    linear_bias: Optional[torch.Tensor] = None  # bf16 [E, N]: SwitchLinear's bias (switch_layers.cpp:111-114)

    def __post_init__(self):
        _need(self.w.dim() == 3, "w must be [E, N, K*bits/32]")
        _need(self.w.element_size() == 4, "w must hold 32-bit words")
        self.experts, self.N = int(self.w.shape[0]), int(self.w.shape[1])
        self.K = int(self.w.shape[2]) * 32 // self.bits
        _need(tuple(self.scales.shape) == (self.experts, self.N, self.K // self.group_size),
              "scales must be [E, N, K/group_size]")
        if self.biases is not None:
            _need(self.biases.shape == self.scales.shape, "biases must match scales")
        if self.linear_bias is not None:
            _need(tuple(self.linear_bias.shape) == (self.experts, self.N) and
                  self.linear_bias.dtype == torch.bfloat16 and self.linear_bias.is_contiguous(),
                  "linear_bias must be a contiguous bf16 [E, N]")

    def c(self) -> QWeightC:
        return QWeightC(self.w.data_ptr(), self.scales.data_ptr(),
                        self.biases.data_ptr() if self.biases is not None else None,
                        self.experts, self.N, self.K, self.group_size, self.bits,
                        self.linear_bias.data_ptr() if self.linear_bias is not None else None)

    @classmethod
    def from_numpy(cls, w, scales, biases, group_size: int, bits: int, device,
                   linear_bias=None) -> "QuantizedWeight":
        import numpy as np

        def bf(a):
            return None if a is None else \
                torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).to(device).view(torch.bfloat16)
        return cls(torch.from_numpy(np.ascontiguousarray(w).view(np.int32)).to(device), bf(scales), bf(biases),
                   group_size, bits, bf(linear_bias))


def router_logits(x: torch.Tensor, wg: torch.Tensor, bias: Optional[torch.Tensor] = None) -> torch.Tensor:
    """logits [T, E] = bf16(x [T, H] . wg [E, H]^T (+ bias [E])), linear_forward's dense branch."""
    _dev(x, torch.bfloat16, "x")
    _dev(wg, torch.bfloat16, "wg")
    T, H = x.shape
    E = wg.shape[0]
    if bias is not None:
        _dev(bias, torch.bfloat16, "bias")
        _need(bias.numel() == E, "bias must hold E values")
    out = torch.empty((T, E), dtype=torch.bfloat16, device=x.device)
    check(lib().moe_router_logits(_p(x), _p(wg), _p(bias), T, H, E, _p(out), _stream(x.device)),
          "moe_router_logits")
    return out


def make_router_params(variant: int, num_experts: int, top_k: int, norm_topk_prob: bool = True,
                       n_group: int = 1, topk_group: int = 1,
                       routed_scaling_factor: float = 1.0) -> RouterParams:
    return RouterParams(variant, num_experts, top_k, int(bool(norm_topk_prob)), n_group, topk_group,
                        routed_scaling_factor)


def route(logits: torch.Tensor, params: RouterParams, score_bias: Optional[torch.Tensor] = None):
    """(inds int32 [T, k] canonical slot order, scores fp32 [T, k])."""
    _dev(logits, torch.bfloat16, "logits")
    if score_bias is not None:
        _dev(score_bias, torch.float32, "score_bias")
    T = logits.shape[0]
    k = params.top_k
    inds = torch.empty((T, k), dtype=torch.int32, device=logits.device)
    scores = torch.empty((T, k), dtype=torch.float32, device=logits.device)
    check(lib().moe_route(_p(logits), _p(score_bias), T, ctypes.byref(params), _p(inds), _p(scores),
                          _stream(logits.device)), "moe_route")
    return inds, scores


def bucket(inds: torch.Tensor, num_experts: int):
    """(perm, inv_perm, sorted_expert, offsets[E+1]) of the stable expert sort."""
    _dev(inds, torch.int32, "inds")
    T, k = inds.shape
    P = T * k
    dev = inds.device
    perm = torch.empty(P, dtype=torch.int32, device=dev)
    inv = torch.empty(P, dtype=torch.int32, device=dev)
    se = torch.empty(P, dtype=torch.int32, device=dev)
    offs = torch.empty(num_experts + 1, dtype=torch.int32, device=dev)
    wsz = lib().moe_bucket_workspace_size(T, k, num_experts)
    ws = torch.empty(max(wsz, 1), dtype=torch.uint8, device=dev)
    check(lib().moe_bucket(_p(inds), T, k, num_experts, _p(perm), _p(inv), _p(se), _p(offs), _p(ws),
                           wsz, _stream(dev)), "moe_bucket")
    return perm, inv, se, offs


def _out_buffer(out: Optional[torch.Tensor], shape, device) -> torch.Tensor:
    if out is None:
        return torch.empty(shape, dtype=torch.bfloat16, device=device)
    _dev(out, torch.bfloat16, "out")
    _need(tuple(out.shape) == tuple(shape), f"out must be {tuple(shape)}")
    return out


def gather_qmm(x: torch.Tensor, w: QuantizedWeight, lhs: Optional[torch.Tensor],
               rhs: torch.Tensor, M: int = 1, sorted_indices: bool = False,
               out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """out [batch, M, N] = x[lhs[b]] . dequant(w[rhs[b]])^T  (switch_layers.cpp:94-102).  A row whose
    rhs[b] is not below the expert count is written as zeros."""
    _dev(x, torch.bfloat16, "x")
    _dev(rhs, torch.int32, "rhs")
    if lhs is not None:
        _dev(lhs, torch.int32, "lhs")
        _need(lhs.numel() == rhs.numel(), "lhs and rhs must be broadcast to the same length")
    batch = rhs.numel()
    _need(x.shape[-1] == w.K, "x last dim must equal K")
    out = _out_buffer(out, (batch, M, w.N), x.device)
    wsz = lib().moe_gather_qmm_workspace_size(batch, M, w.experts)
    ws = torch.empty(max(wsz, 1), dtype=torch.uint8, device=x.device)
    qc = w.c()
    check(lib().moe_gather_qmm(_p(x), ctypes.byref(qc), _p(lhs), _p(rhs), batch, M, int(sorted_indices),
                               _p(out), _p(ws), wsz, _stream(x.device)), "moe_gather_qmm")
    return out


def gather_mm(x: torch.Tensor, w: torch.Tensor, lhs: Optional[torch.Tensor], rhs: torch.Tensor, M: int = 1,
              linear_bias: Optional[torch.Tensor] = None, sorted_indices: bool = False,
              out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """out [batch, M, N] = x[lhs[b]] . w[rhs[b]]^T (+ linear_bias[rhs[b]]): SwitchLinear's dense branch,
    gather_mm(x, swapaxes(w, -1, -2), lhs, rhs) (switch_layers.cpp:103-115); w bf16 [E, N, K].  A row
    whose rhs[b] is not below E is written as zeros."""
    _dev(x, torch.bfloat16, "x")
    _dev(w, torch.bfloat16, "w")
    _dev(rhs, torch.int32, "rhs")
    _need(w.dim() == 3 and x.shape[-1] == w.shape[2], "w must be [E, N, K] with K = x's last dim")
    E, N, K = (int(v) for v in w.shape)
    if lhs is not None:
        _dev(lhs, torch.int32, "lhs")
        _need(lhs.numel() == rhs.numel(), "lhs and rhs must be broadcast to the same length")
    if linear_bias is not None:
        _dev(linear_bias, torch.bfloat16, "linear_bias")
        _need(tuple(linear_bias.shape) == (E, N), "linear_bias must be [E, N]")
    batch = rhs.numel()
    out = _out_buffer(out, (batch, M, N), x.device)
    wsz = lib().moe_gather_mm_workspace_size(batch, M, E)
    ws = torch.empty(max(wsz, 1), dtype=torch.uint8, device=x.device)
    check(lib().moe_gather_mm(_p(x), _p(w), _p(linear_bias), E, N, K, _p(lhs), _p(rhs), batch, M,
                              int(sorted_indices), _p(out), _p(ws), wsz, _stream(x.device)), "moe_gather_mm")
    return out


def swiglu(g: torch.Tensor, u: torch.Tensor) -> torch.Tensor:
    _dev(g, torch.bfloat16, "gate")
    _dev(u, torch.bfloat16, "up")
    _need(g.shape == u.shape, "gate and up must have the same shape")
    h = torch.empty_like(g)
    check(lib().moe_swiglu(_p(g), _p(u), g.numel(), _p(h), _stream(g.device)), "moe_swiglu")
    return h


def gptoss_swiglu(x_linear: torch.Tensor, x_glu: torch.Tensor) -> torch.Tensor:
    """GPT-OSS's clipped SwiGLU swiglu(x_linear, x_glu) (gptoss.cpp:50-58); its MoE MLP calls it
    as swiglu(x_gate, x_up) (:158).  bf16 out."""
    _dev(x_linear, torch.bfloat16, "x_linear")
    _dev(x_glu, torch.bfloat16, "x_glu")
    _need(x_linear.shape == x_glu.shape, "x_linear and x_glu must have the same shape")
    h = torch.empty_like(x_linear)
    check(lib().moe_gptoss_swiglu(_p(x_linear), _p(x_glu), x_linear.numel(), _p(h), _stream(x_linear.device)),
          "moe_gptoss_swiglu")
    return h


def add_rms_norm(a: torch.Tensor, b: torch.Tensor, weight: torch.Tensor, eps: float):
    """(a + b, rms_norm(a + b) * weight) for [T, H] bf16 rows: the residual add and the norm that
    produce the MoE input (add_rms_norm, src/common/gated_delta.cpp:313-345)."""
    _dev(a, torch.bfloat16, "a")
    _dev(b, torch.bfloat16, "b")
    _dev(weight, torch.bfloat16, "weight")
    _need(a.shape == b.shape and a.dim() == 2 and weight.shape == (a.shape[1],), "a, b [T, H]; weight [H]")
    s, n = torch.empty_like(a), torch.empty_like(a)
    check(lib().moe_add_rms_norm(_p(a), _p(b), _p(weight), float(eps), a.shape[0], a.shape[1], _p(s), _p(n),
                                 _stream(a.device)), "moe_add_rms_norm")
    return s, n


def combine(Y: torch.Tensor, scores: torch.Tensor, inv_perm: Optional[torch.Tensor] = None) -> torch.Tensor:
    """y [T, H] = sum_j scores[t, j] * Y[row(t, j)]; Y is [T*k, H] (sorted if inv_perm given)."""
    _dev(Y, torch.bfloat16, "Y")
    _dev(scores, torch.float32, "scores")
    T, k = scores.shape
    H = Y.shape[-1]
    if inv_perm is not None:
        _dev(inv_perm, torch.int32, "inv_perm")
    y = torch.empty((T, H), dtype=torch.bfloat16, device=Y.device)
    check(lib().moe_combine(_p(Y), _p(inv_perm), _p(scores), T, k, H, _p(y), _stream(Y.device)),
          "moe_combine")
    return y


def take_rows(src: torch.Tensor, rows: torch.Tensor, divisor: int = 1) -> torch.Tensor:
    """dst[i] = src[rows[i] // divisor] over src's leading axis (zero row if out of range).

    divisor = k with rows = a sorted pair order is gather_sort's take(x_flat, order // k);
    divisor = 1 with rows = the inverse order is scatter_unsort (switch_layers.cpp:17-46)."""
    _need(src.is_cuda and src.is_contiguous(), "src must be a contiguous device tensor")
    _dev(rows, torch.int32, "rows")
    n = rows.numel()
    row_bytes = src[0].numel() * src.element_size() if src.shape[0] > 0 else 0
    dst = torch.empty((n,) + tuple(src.shape[1:]), dtype=src.dtype, device=src.device)
    check(lib().moe_take_rows(_p(src), src.shape[0], _p(rows), n, divisor, row_bytes, _p(dst),
                              _stream(src.device)), "moe_take_rows")
    return dst


def add_expert_bias(out: torch.Tensor, bias: torch.Tensor, rhs: torch.Tensor) -> torch.Tensor:
    """out [batch, M, N] += bias [E, N][rhs[b]] in place (bf16 rounding), switch_layers.cpp:111-114."""
    _dev(out, torch.bfloat16, "out")
    _dev(bias, torch.bfloat16, "bias")
    _dev(rhs, torch.int32, "rhs")
    batch, M, N = out.shape
    _need(rhs.numel() == batch and bias.shape[-1] == N, "shapes of out, bias and rhs disagree")
    check(lib().moe_add_expert_bias(_p(out), _p(bias), _p(rhs), batch, M, N, bias.shape[0],
                                    _stream(out.device)), "moe_add_expert_bias")
    return out


def switch_glu(x: torch.Tensor, inds: torch.Tensor, gate: QuantizedWeight, up: QuantizedWeight,
               down: QuantizedWeight, activation: int = 0) -> torch.Tensor:
    """SwitchGLU::operator() (switch_layers.cpp:200-245): [T, H] x, [T, k] inds -> [T, k, H].
    activation: moe_activation of h (0 SwiGLU; 1 / 2 GPT-OSS's clipped SwiGLU, gptoss.cpp:50-58)."""
    _dev(x, torch.bfloat16, "x")
    _dev(inds, torch.int32, "inds")
    T, k = inds.shape
    _need(x.shape == (T, gate.K), "x must be [T, H]")
    out = torch.empty((T, k, down.N), dtype=torch.bfloat16, device=x.device)
    g, u, d = gate.c(), up.c(), down.c()
    wsz = lib().moe_switch_glu_workspace_size(ctypes.byref(g), ctypes.byref(d), T, k)
    ws = torch.empty(max(wsz, 1), dtype=torch.uint8, device=x.device)
    check(lib().moe_switch_glu(ctypes.byref(g), ctypes.byref(u), ctypes.byref(d), _p(x), _p(inds), T, k,
                               int(activation), _p(out), _p(ws), wsz, _stream(x.device)), "moe_switch_glu")
    return out


def switch_mlp_relu2(x: torch.Tensor, inds: torch.Tensor, up: QuantizedWeight,
                     down: QuantizedWeight) -> torch.Tensor:
    """NemotronHSwitchMLP::operator() (nemotron_h.cpp:484-511): fc1, relu^2, fc2; [T, H] x, [T, k] inds
    -> [T, k, H]."""
    _dev(x, torch.bfloat16, "x")
    _dev(inds, torch.int32, "inds")
    T, k = inds.shape
    _need(x.shape == (T, up.K), "x must be [T, H]")
    out = torch.empty((T, k, down.N), dtype=torch.bfloat16, device=x.device)
    u, d = up.c(), down.c()
    wsz = lib().moe_switch_mlp_workspace_size(ctypes.byref(u), ctypes.byref(d), T, k)
    ws = torch.empty(max(wsz, 1), dtype=torch.uint8, device=x.device)
    check(lib().moe_switch_mlp_relu2(ctypes.byref(u), ctypes.byref(d), _p(x), _p(inds), T, k, _p(out), _p(ws), wsz,
                                     _stream(x.device)), "moe_switch_mlp_relu2")
    return out


def _block_io(block: "MoeBlock", x: torch.Tensor, out: Optional[torch.Tensor]) -> None:
    """x [T, hidden] and out (when given) of the same shape, bf16, contiguous, on x's device.
    The C ABI cannot see buffer sizes, so a short x or out would be read or written out of
    bounds on the device: shapes are checked before anything else."""
    _need(x.dim() == 2 and x.shape[1] == block.hidden, f"x must be [T, {block.hidden}], got {tuple(x.shape)}")
    if out is not None:
        _need(tuple(out.shape) == tuple(x.shape), f"out must be {tuple(x.shape)}, got {tuple(out.shape)}")
    _dev(x, torch.bfloat16, "x")
    _need(x.device == block.device, f"x is on {x.device}, the block's weights on {block.device}")
    if out is not None:
        _dev(out, torch.bfloat16, "out")
        _need(out.device == x.device, "out must be on x's device")


class BlockGraph:
    """A captured moe_block_forward over fixed buffers; keeps them (and its workspace) alive."""

    def __init__(self, block: "MoeBlock", x: torch.Tensor, out: torch.Tensor):
        self.handle = None
        _need(out is not None, "out is required")
        _block_io(block, x, out)
        T = x.shape[0]
        n = block.workspace_size(T)
        self.keep = (block, x, out, torch.empty(max(n, 1), dtype=torch.uint8, device=x.device))
        self.handle = ctypes.c_void_p()
        check(lib().moe_block_graph_create(ctypes.byref(block.desc), _p(x), T, _p(out), _p(self.keep[3]), n,
                                           ctypes.byref(self.handle)), "moe_block_graph_create")

    def launch(self):
        check(lib().moe_block_graph_launch(self.handle, _stream(self.keep[1].device)), "moe_block_graph_launch")

    def __del__(self):
        if getattr(self, "handle", None) is not None and self.handle.value:
            lib().moe_block_graph_destroy(self.handle)
            self.handle = ctypes.c_void_p()


class MoeBlock:
    """The model-level MoE block: router -> top-k -> SwitchGLU -> combine (+ shared expert).

    Mirrors Qwen3MoESparseMoeBlock / Qwen3NextSparseMoeBlock / PhiMoESparseMoeBlock /
    DeepseekV3MoE ``operator()`` (src/llm/models/qwen3_moe.cpp:155-175,
    qwen3_next.cpp:452-490, phimoe.cpp:93-105, deepseek_v3.cpp:371-381).
    """

    def __init__(self, router: RouterParams, router_weight: Optional[torch.Tensor], gate: QuantizedWeight,
                 up: QuantizedWeight, down: QuantizedWeight, score_bias: Optional[torch.Tensor] = None,
                 shared: Optional[tuple] = None, router_q: Optional[QuantizedWeight] = None,
                 router_bias: Optional[torch.Tensor] = None, activation: int = 0):
        E = router.num_experts
        self.hidden, self.intermediate, self.num_experts = gate.K, gate.N, E
        self.router = router
        self.router_weight, self.score_bias, self.router_bias = router_weight, score_bias, router_bias
        self.shared_gate_weight = shared[3] if shared is not None else None
        self.router_q = router_q
        self.tensors = [router_weight, score_bias, router_bias]
        self.weights = [gate, up, down]
        d = BlockDesc()
        d.hidden, d.intermediate, d.num_experts = gate.K, gate.N, E
        d.router = router
        d.router_weight = router_weight.data_ptr() if router_weight is not None else None
        d.score_bias = score_bias.data_ptr() if score_bias is not None else None
        d.gate, d.up, d.down = gate.c(), up.c(), down.c()
        d.shared_intermediate = 0
        if shared is not None:  # (gate, up, down, sigmoid gate: bf16 [1, H], a QuantizedWeight [1][1, H] or None)
            sg, su, sd, sgw = shared
            self.weights += [sg, su, sd]
            self.tensors.append(sgw)
            d.shared_intermediate = sg.N
            d.shared_gate, d.shared_up, d.shared_down = sg.c(), su.c(), sd.c()
            if isinstance(sgw, QuantizedWeight):
                d.shared_gate_q = sgw.c()
            else:
                d.shared_gate_weight = sgw.data_ptr() if sgw is not None else None
        if router_q is not None:  # quantized router projection (linear_forward's quantized branch)
            self.weights.append(router_q)
            d.router_q = router_q.c()
        d.router_bias = router_bias.data_ptr() if router_bias is not None else None
        d.activation = int(activation)
        self.desc = d
        self.device = gate.w.device
        self._ws = None

    @classmethod
    def from_host(cls, layer, device="cuda:0") -> "MoeBlock":
        """Upload a workloads.HostLayer (numpy) to the device."""
        import numpy as np

        def qw(h):
            return QuantizedWeight.from_numpy(h.w, h.scales, h.biases, h.group_size, h.bits, device,
                                              getattr(h, "linear_bias", None))

        def bf(a):
            return torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).to(device).view(torch.bfloat16)

        bias = None if layer.score_bias is None else torch.from_numpy(layer.score_bias).to(device)
        shared = None
        if layer.shared is not None:
            sg, su, sd, sgw = layer.shared
            gate = None if sgw is None else bf(sgw) if isinstance(sgw, np.ndarray) else qw(sgw)
            shared = (qw(sg), qw(su), qw(sd), gate)
        rq = None if getattr(layer, "router_q", None) is None else qw(layer.router_q)
        rw = None if layer.router_weight is None else bf(layer.router_weight)
        rb = None if getattr(layer, "router_bias", None) is None else bf(layer.router_bias)
        return cls(layer.cfg.router_params(), rw, qw(layer.gate), qw(layer.up),
                   qw(layer.down), bias, shared, rq, rb, getattr(layer.cfg, "activation", 0))

    def graph(self, x: torch.Tensor, out: torch.Tensor) -> "BlockGraph":
        """The block over the buffers x [T, H] -> out as one captured graph (moe_block_graph_create):
        refill x in place and call .launch() per decode step.  Uses a workspace of its own."""
        return BlockGraph(self, x, out)

    def workspace_size(self, T: int) -> int:
        n = lib().moe_block_workspace_size(ctypes.byref(self.desc), T)
        if n == 0 and T > 0:
            raise ValueError("invalid MoE block description")
        return n

    def workspace(self, T: int) -> torch.Tensor:
        n = self.workspace_size(T)
        if self._ws is None or self._ws.numel() < n:
            self._ws = torch.empty(max(n, 1), dtype=torch.uint8, device=self.device)
        return self._ws

    def _aux(self, T: int, device):
        k, E = self.router.top_k, self.num_experts
        auxd = dict(
            logits=torch.empty((T, E), dtype=torch.bfloat16, device=device),
            inds=torch.empty((T, k), dtype=torch.int32, device=device),
            scores=torch.empty((T, k), dtype=torch.float32, device=device),
            perm=torch.empty(T * k, dtype=torch.int32, device=device),
            inv_perm=torch.empty(T * k, dtype=torch.int32, device=device),
            offsets=torch.empty(E + 1, dtype=torch.int32, device=device),
        )
        aux = BlockAux(*(auxd[n].data_ptr() for n in ("logits", "inds", "scores", "perm", "inv_perm", "offsets")))
        return aux, auxd

    def forward(self, x: torch.Tensor, out: Optional[torch.Tensor] = None, return_aux: bool = False):
        _block_io(self, x, out)
        T = x.shape[0]
        if out is None:
            out = torch.empty_like(x)
        ws = self.workspace(T)
        aux, auxd = self._aux(T, x.device) if return_aux else (None, {})
        check(lib().moe_block_forward(ctypes.byref(self.desc), _p(x), T, _p(out),
                                      ctypes.byref(aux) if aux is not None else None, _p(ws), ws.numel(),
                                      _stream(x.device)), "moe_block_forward")
        if return_aux:
            return out, auxd
        return out

    def forward_add_norm(self, a: torch.Tensor, b: torch.Tensor, norm_weight: torch.Tensor, eps: float,
                         out: Optional[torch.Tensor] = None, return_aux: bool = False):
        """The decode layer's residual add + RMSNorm and the block in one call
        (moe_block_forward_add_norm): returns (sum, normed, out[, aux]) with sum = a + b and normed
        = rms_norm(sum) * norm_weight, the block's input; the results of add_rms_norm followed by
        forward, bit for bit."""
        _block_io(self, a, out)
        _block_io(self, b, None)
        _dev(norm_weight, torch.bfloat16, "norm_weight")
        _need(a.shape == b.shape and norm_weight.shape == (a.shape[1],), "a, b [T, H]; norm_weight [H]")
        T = a.shape[0]
        if out is None:
            out = torch.empty_like(a)
        s, n = torch.empty_like(a), torch.empty_like(a)
        ws = self.workspace(T)
        aux, auxd = self._aux(T, a.device) if return_aux else (None, {})
        check(lib().moe_block_forward_add_norm(ctypes.byref(self.desc), _p(a), _p(b), _p(norm_weight), float(eps), T,
                                               _p(s), _p(n), _p(out),
                                               ctypes.byref(aux) if aux is not None else None, _p(ws), ws.numel(),
                                               _stream(a.device)), "moe_block_forward_add_norm")
        if return_aux:
            return s, n, out, auxd
        return s, n, out

    __call__ = forward
