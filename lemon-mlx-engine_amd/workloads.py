"""Synthetic MoE layers of the benchmark configurations, generated on the host.

All tensors come from the library's seeded counter-based generator
(``moe_synth_normal_*``) and are quantized with ``moe_quantize_affine`` (the
MLX affine format), so the HIP path and the CPU checker consume identical
bytes.  The seed of a config is ``0 + config id``.

Tensor ids: 1 router weight, 2/3/4 expert gate/up/down, 5/6/7 shared-expert
gate/up/down, 8 shared-expert sigmoid gate, 9 score-correction bias, 10/11/12
expert linear biases (gate/up/down), 13 router bias, 100 tokens.
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass, field
from typing import Dict, Optional, Sequence

import numpy as np

from . import (ROUTE_GLM4_SIGMOID, ROUTE_GLM4_SOFTMAX, ROUTE_LFM2, ROUTE_SIGMOID_CORRECTED, ROUTE_SIGMOID_GROUP, ROUTE_SIGMOID_GROUP_DROP_BEST, ROUTE_SOFTMAX_TOPK,
               ROUTE_TOPK_LOGITS, ROUTE_TOPK_PROBS, RouterParams, check, lib)


@dataclass(frozen=True)
class MoeConfig:
    name: str
    config_id: int
    hidden: int
    intermediate: int
    num_experts: int
    top_k: int
    variant: int
    norm_topk_prob: bool
    bits: int
    group_size: int = 64
    n_group: int = 1
    topk_group: int = 1
    routed_scaling_factor: float = 1.0
    shared_intermediate: int = 0
    shared_gated: bool = False
    tokens: Sequence[int] = field(default_factory=tuple)
    w_std: float = 0.02
    bias_std: float = 0.01
    activation: int = 0        # moe_activation of the routed experts (0: SwiGLU)

    @property
    def seed(self) -> int:
        return self.config_id

    def router_params(self) -> RouterParams:
        return RouterParams(self.variant, self.num_experts, self.top_k, int(self.norm_topk_prob),
                            self.n_group, self.topk_group, self.routed_scaling_factor)


# The five configurations of the benchmark definition (configs[0..4]).
CONFIGS: Dict[str, MoeConfig] = {
    "tiny": MoeConfig("tiny", 0, 512, 1024, 8, 2, ROUTE_TOPK_LOGITS, True, 4, tokens=(16,)),
    "qwen3_30b_a3b": MoeConfig("qwen3_30b_a3b", 1, 2048, 768, 128, 8, ROUTE_TOPK_LOGITS, True, 4,
                               tokens=(1, 8, 64, 8192)),
    "qwen3_next_80b": MoeConfig("qwen3_next_80b", 2, 2048, 512, 512, 10, ROUTE_TOPK_PROBS, True, 4,
                                shared_intermediate=512, shared_gated=True, tokens=(1, 32, 4096)),
    "mixtral_8x7b": MoeConfig("mixtral_8x7b", 3, 4096, 14336, 8, 2, ROUTE_SOFTMAX_TOPK, False, 8,
                              tokens=(1, 16, 8192)),
    "deepseek_v3": MoeConfig("deepseek_v3", 4, 7168, 2048, 256, 8, ROUTE_SIGMOID_GROUP, True, 4,
                             n_group=8, topk_group=4, routed_scaling_factor=2.5,
                             shared_intermediate=2048, shared_gated=False, tokens=(1, 64, 4096)),
}

TID_ROUTER, TID_GATE, TID_UP, TID_DOWN = 1, 2, 3, 4
TID_SH_GATE, TID_SH_UP, TID_SH_DOWN, TID_SH_GATE_W, TID_BIAS, TID_X = 5, 6, 7, 8, 9, 100
TID_LB_GATE, TID_LB_UP, TID_LB_DOWN, TID_ROUTER_BIAS = 10, 11, 12, 13


def _vp(a: np.ndarray) -> ctypes.c_void_p:
    return ctypes.c_void_p(a.ctypes.data)


def normal_bf16(seed: int, tid: int, n: int, std: float, first: int = 0, mean: float = 0.0) -> np.ndarray:
    out = np.empty(n, dtype=np.uint16)
    check(lib().moe_synth_normal_bf16(seed, tid, mean, std, first, n, _vp(out)), "moe_synth_normal_bf16")
    return out


def normal_f32(seed: int, tid: int, n: int, std: float, first: int = 0, mean: float = 0.0) -> np.ndarray:
    out = np.empty(n, dtype=np.float32)
    check(lib().moe_synth_normal_f32(seed, tid, mean, std, first, n, _vp(out)), "moe_synth_normal_f32")
    return out


def quantize(w_bf16: np.ndarray, rows: int, K: int, group_size: int, bits: int):
    """MLX affine quantize of a [rows, K] bf16 matrix -> (packed u32, scales bf16, biases bf16)."""
    wq = np.empty(rows * K * bits // 32, dtype=np.uint32)
    sc = np.empty(rows * (K // group_size), dtype=np.uint16)
    bi = np.empty_like(sc)
    check(lib().moe_quantize_affine(_vp(np.ascontiguousarray(w_bf16)), rows, K, group_size, bits, _vp(wq),
                                    _vp(sc), _vp(bi)), "moe_quantize_affine")
    return wq, sc, bi


@dataclass
class HostQWeight:
    w: np.ndarray        # uint32 [E, N, K*bits/32]
    scales: np.ndarray   # uint16 (bf16) [E, N, K/gs]
    biases: np.ndarray   # uint16 (bf16) [E, N, K/gs]
    experts: int
    N: int
    K: int
    group_size: int
    bits: int
    linear_bias: Optional[np.ndarray] = None  # bf16 [E, N]: SwitchLinear's bias (switch_layers.cpp:111-114)


def make_qweight(seed: int, tid: int, experts: int, N: int, K: int, std: float, group_size: int,
                 bits: int) -> HostQWeight:
    """Generate W ~ N(0, std) [experts, N, K] slice by slice and quantize it."""
    per = N * K
    w = np.empty((experts, N, K * bits // 32), dtype=np.uint32)
    s = np.empty((experts, N, K // group_size), dtype=np.uint16)
    b = np.empty_like(s)
    for e in range(experts):
        dense = normal_bf16(seed, tid, per, std, first=e * per)
        wq, sc, bi = quantize(dense, N, K, group_size, bits)
        w[e] = wq.reshape(N, -1)
        s[e] = sc.reshape(N, -1)
        b[e] = bi.reshape(N, -1)
    return HostQWeight(w, s, b, experts, N, K, group_size, bits)


@dataclass
class HostLayer:
    cfg: MoeConfig
    router_weight: Optional[np.ndarray]  # bf16 [E, H] (None: router_q only)
    gate: HostQWeight
    up: HostQWeight
    down: HostQWeight
    score_bias: Optional[np.ndarray] = None   # fp32 [E]
    shared: Optional[tuple] = None            # (gate, up, down, sigmoid gate: bf16 [1, H], a quantized
                                              #  HostQWeight [1][1, H], or None)
    router_q: Optional[HostQWeight] = None    # quantized router [1][E, H] (used instead of router_weight)
    router_bias: Optional[np.ndarray] = None  # bf16 [E]: the router projection's bias (GPT-OSS)


def make_layer(cfg: MoeConfig, router_bits: Optional[int] = None, linear_bias: bool = False,
               shared_gate_bits: Optional[int] = None, glu_bias_std: float = 0.1) -> HostLayer:
    """router_bits: also quantize the router weight (same values, gs 64) and
    route with it, as a checkpoint with a quantized mlp.gate does.
    shared_gate_bits: quantize the shared expert's sigmoid gate (gs 64), as MLX
    conversions of Qwen3-Next do.
    linear_bias: give the expert projections SwitchLinear biases and the router
    a bias ~ N(0, 0.1) bf16, as GPT-OSS's block has (gptoss.cpp:120-131); the
    gate and up biases ~ N(0, glu_bias_std) (a few units put GPT-OSS's clipped
    SwiGLU inputs on both sides of its limits)."""
    H, I, E = cfg.hidden, cfg.intermediate, cfg.num_experts
    sd, gs, bits = cfg.seed, cfg.group_size, cfg.bits
    rw = normal_bf16(sd, TID_ROUTER, E * H, cfg.w_std).reshape(E, H)
    gate = make_qweight(sd, TID_GATE, E, I, H, cfg.w_std, gs, bits)
    up = make_qweight(sd, TID_UP, E, I, H, cfg.w_std, gs, bits)
    down = make_qweight(sd, TID_DOWN, E, H, I, cfg.w_std, gs, bits)
    bias = None
    if cfg.variant in (ROUTE_SIGMOID_GROUP, ROUTE_SIGMOID_GROUP_DROP_BEST, ROUTE_SIGMOID_CORRECTED,
                       ROUTE_GLM4_SIGMOID, ROUTE_GLM4_SOFTMAX, ROUTE_LFM2):
        bias = normal_f32(sd, TID_BIAS, E, cfg.bias_std)
    shared = None
    if cfg.shared_intermediate > 0:
        Is = cfg.shared_intermediate
        sg = make_qweight(sd, TID_SH_GATE, 1, Is, H, cfg.w_std, gs, bits)
        su = make_qweight(sd, TID_SH_UP, 1, Is, H, cfg.w_std, gs, bits)
        sdn = make_qweight(sd, TID_SH_DOWN, 1, H, Is, cfg.w_std, gs, bits)
        sgw = normal_bf16(sd, TID_SH_GATE_W, H, cfg.w_std).reshape(1, H) if cfg.shared_gated else None
        if cfg.shared_gated and shared_gate_bits:
            sgw = make_qweight(sd, TID_SH_GATE_W, 1, 1, H, cfg.w_std, 64, shared_gate_bits)
        shared = (sg, su, sdn, sgw)
    rq = make_qweight(sd, TID_ROUTER, 1, E, H, cfg.w_std, 64, router_bits) if router_bits else None
    rb = None
    if linear_bias:
        for q, tid, std in ((gate, TID_LB_GATE, glu_bias_std), (up, TID_LB_UP, glu_bias_std),
                            (down, TID_LB_DOWN, 0.1)):
            q.linear_bias = normal_bf16(sd, tid, q.experts * q.N, std).reshape(q.experts, q.N)
        rb = normal_bf16(sd, TID_ROUTER_BIAS, E, 0.1)
    return HostLayer(cfg, rw, gate, up, down, bias, shared, rq, rb)


def make_tokens(cfg: MoeConfig, T: int) -> np.ndarray:
    """x ~ N(0, 1) bf16 [T, H]; a smaller T is a prefix of a larger one."""
    return normal_bf16(cfg.seed, TID_X, T * cfg.hidden, 1.0).reshape(T, cfg.hidden)


def layer_bytes(cfg: MoeConfig, distinct_experts: int, T: int) -> int:
    """Algorithmic HBM bytes of one block call: routed expert weights (packed +
    bf16 scale and bias per group), shared expert, router weight, x in and y out."""
    bpp = cfg.bits / 8 + 4 / cfg.group_size
    b = distinct_experts * 3 * cfg.intermediate * cfg.hidden * bpp
    b += 3 * cfg.shared_intermediate * cfg.hidden * bpp
    b += cfg.num_experts * cfg.hidden * 2
    b += 2 * T * cfg.hidden * 2
    return int(b)


def layer_flops(cfg: MoeConfig, T: int) -> int:
    return int(2 * T * cfg.top_k * 3 * cfg.intermediate * cfg.hidden + 2 * T * cfg.hidden * cfg.num_experts
               + 2 * T * 3 * cfg.shared_intermediate * cfg.hidden)
