"""checkpoint.py -- one MoE layer of an MLX-format checkpoint directory (safetensors)
as a ``workloads.HostLayer``, ready for ``MoeBlock.from_host``.

Follows the reference's ingestion steps:

* files: ``load_safetensors_from_directory`` (src/common/safetensors.cpp:23-77) --
  ``model.safetensors.index.json`` shards first, then ``model.safetensors``, else
  every ``*.safetensors`` of the directory;
* per-expert tensors ``<block>.experts.{e}.<proj>.*`` are stacked into the
  ``<block>.switch_mlp.*`` layout [E, N, ...] for ``.weight``, ``.scales`` and
  ``.biases`` (``Qwen3MoEModel::sanitize_impl``, src/llm/models/qwen3_moe.cpp:291-318;
  ``DeepseekV3Model::sanitize_impl``, src/llm/models/deepseek_v3.cpp:531-555;
  ``PhiMoEModel::sanitize_impl``, src/llm/models/phimoe.cpp:208-235, which also renames
  ``w1/w2/w3`` to ``gate_proj/down_proj/up_proj``);
* a tensor is quantized iff ``<prefix>.scales`` exists; its bits and group size are
  the config's ``quantization`` defaults (64, 4) unless the ``quantization`` entry
  names the prefix itself (``register_quantized_weights``,
  src/common/quantize_utils.cpp:14-104; the per-prefix overrides of
  src/common/base_config.cpp:28-73, with a ``language_model.`` prefix stripped).

Tensor data are memory-mapped; only the tensors of the requested layer are read.
Models (``_MODELS``): Qwen3-MoE (``qwen3_moe``: top-k of logits), Qwen3-Next
(``qwen3_next``: top-k of probabilities, gated shared expert), DeepSeek-V3
(``deepseek_v3``: sigmoid router with ``e_score_correction_bias``, ungated shared experts
of ``moe_intermediate_size * n_shared_experts``; src/llm/models/deepseek_v3.cpp:21-62,
294-381) and PhiMoE (``phimoe``: ``block_sparse_moe``, softmax over the k selected
logits; src/llm/models/phimoe.cpp:11-30, 85-105).
"""
from __future__ import annotations

import json
import os
import struct
from dataclasses import dataclass
from typing import Dict, Optional, Tuple

import numpy as np

from . import (ROUTE_SIGMOID, ROUTE_SIGMOID_GROUP, ROUTE_SOFTMAX_TOPK, ROUTE_TOPK_LOGITS,
               ROUTE_TOPK_PROBS)
from .workloads import HostLayer, HostQWeight, MoeConfig

_DTYPES = {"BF16": np.uint16, "F16": np.float16, "F32": np.float32, "U32": np.uint32, "I32": np.int32,
           "U8": np.uint8, "U16": np.uint16}

_PROJS = (("gate_proj", "gate_proj"), ("up_proj", "up_proj"), ("down_proj", "down_proj"))


@dataclass(frozen=True)
class _Naming:
    """Where one model family keeps its MoE block: config keys (with the reference's
    defaults), the block's module name and the per-expert projection names."""
    variant: int
    block: str = "mlp"                              # model.layers.{l}.<block>
    experts_key: str = "num_experts"
    experts_default: Optional[int] = None
    topk_default: Optional[int] = None
    intermediate_key: str = "moe_intermediate_size"
    intermediate_default: Optional[int] = None
    projs: Tuple[Tuple[str, str], ...] = _PROJS     # (per-expert name, switch_mlp name)
    shared: Optional[str] = None                    # shared expert module under the block
    shared_gate: Optional[str] = None               # its sigmoid gate (Qwen3-Next)
    score_bias: bool = False                        # gate.e_score_correction_bias (DeepSeek)


_MODELS = {
    # qwen3_moe.cpp:17-47, 155-175
    "qwen3_moe": _Naming(ROUTE_TOPK_LOGITS),
    # qwen3_next.cpp:452-490: shared_expert + shared_expert_gate
    "qwen3_next": _Naming(ROUTE_TOPK_PROBS, shared="shared_expert", shared_gate="shared_expert_gate"),
    # deepseek_v3.cpp:21-62 (config), 294-381 (gate, shared_experts, combine)
    "deepseek_v3": _Naming(ROUTE_SIGMOID, experts_key="n_routed_experts", experts_default=1, topk_default=1,
                           shared="shared_experts", score_bias=True),
    # phimoe.cpp:11-30 (config defaults), 85-105 (block), 208-235 (w1/w2/w3 renames)
    "phimoe": _Naming(ROUTE_SOFTMAX_TOPK, block="block_sparse_moe", experts_key="num_local_experts",
                      experts_default=16, topk_default=2, intermediate_key="intermediate_size",
                      intermediate_default=6400,
                      projs=(("w1", "gate_proj"), ("w3", "up_proj"), ("w2", "down_proj"))),
}


def read_header(path: str) -> Tuple[Dict[str, dict], int]:
    """-> ({name: {dtype, shape, data_offsets}}, offset of the data section)."""
    with open(path, "rb") as f:
        (n,) = struct.unpack("<Q", f.read(8))
        header = json.loads(f.read(n))
    header.pop("__metadata__", None)
    return header, 8 + n


def checkpoint_files(directory: str) -> list:
    index = os.path.join(directory, "model.safetensors.index.json")
    if os.path.exists(index):
        with open(index) as f:
            wm = json.load(f).get("weight_map")
        if wm:
            files = [os.path.join(directory, s) for s in sorted(set(wm.values()))]
            for p in files:
                if not os.path.exists(p):
                    raise FileNotFoundError(f"Missing shard file: {p}")
            return files
    single = os.path.join(directory, "model.safetensors")
    if os.path.exists(single) and os.path.getsize(single) > 1024:
        return [single]
    files = sorted(os.path.join(directory, n) for n in os.listdir(directory) if n.endswith(".safetensors"))
    if not files:
        raise FileNotFoundError(f"No .safetensors files found in {directory}")
    return files


class Checkpoint:
    """Tensor index of a checkpoint directory (headers only until a tensor is read)."""

    def __init__(self, directory: str, config: Optional[dict] = None):
        if config is None:
            with open(os.path.join(directory, "config.json")) as f:
                config = json.load(f)
        self.config = config
        self.index: Dict[str, tuple] = {}
        for path in checkpoint_files(directory):
            header, base = read_header(path)
            for name, info in header.items():
                self.index[name] = (path, base, info)  # later files win, as in the reference
        q = config.get("quantization") or {}
        self.default_q = (int(q.get("bits", 4)), int(q.get("group_size", 64)))
        self.overrides = {}
        for key, v in q.items():
            if key in ("group_size", "bits", "mode", "quant_method", "linear_class", "quantization_mode"):
                continue
            key = key[len("language_model."):] if key.startswith("language_model.") else key
            if isinstance(v, dict):
                self.overrides[key] = (int(v.get("bits", self.default_q[0])),
                                       int(v.get("group_size", self.default_q[1])))

    def has(self, name: str) -> bool:
        return name in self.index

    def get(self, name: str) -> np.ndarray:
        path, base, info = self.index[name]
        dt = _DTYPES.get(info["dtype"])
        if dt is None:
            raise ValueError(f"{name}: unsupported dtype {info['dtype']}")
        b, e = info["data_offsets"]
        shape = tuple(info["shape"])
        mm = np.memmap(path, dtype=np.uint8, mode="r", offset=base + b, shape=(e - b,))
        return np.array(mm.view(dt).reshape(shape))

    def quant_for(self, prefix: str) -> Tuple[int, int]:
        return self.overrides.get(prefix, self.default_q)

    def get_f32(self, name: str) -> np.ndarray:
        """A floating-point tensor (BF16, F16 or F32) as float32."""
        dt = self.index[name][2]["dtype"]
        a = self.get(name)
        if dt == "BF16":
            return (a.astype(np.uint32) << 16).view(np.float32)
        if dt in ("F16", "F32"):
            return a.astype(np.float32)
        raise ValueError(f"{name}: {dt} is not a floating-point dtype")

    def _tensor(self, prefix: str, suffix: str, experts: Optional[int],
                source: Optional[str] = None) -> Optional[np.ndarray]:
        """prefix.suffix, or the per-expert tensors stacked (prefix = '...switch_mlp.<proj>';
        source = the per-expert projection's own name, default <proj>)."""
        if self.has(f"{prefix}.{suffix}"):
            return self.get(f"{prefix}.{suffix}")
        if experts is None:
            return None
        head, proj = prefix.rsplit(".switch_mlp.", 1)
        keys = [f"{head}.experts.{e}.{source or proj}.{suffix}" for e in range(experts)]
        if not self.has(keys[0]):
            return None
        missing = [k for k in keys if not self.has(k)]
        if missing:
            raise ValueError(f"{prefix}: {len(missing)} of {experts} per-expert tensors missing ({missing[0]})")
        return np.stack([self.get(k) for k in keys])

    def qweight(self, prefix: str, experts: Optional[int] = None,
                source: Optional[str] = None) -> Optional[HostQWeight]:
        """A quantized projection (stacked [E, N, K*bits/32] or one [N, K*bits/32]
        matrix as experts = 1), or None when the tensor is not quantized."""
        s = self._tensor(prefix, "scales", experts, source)
        if s is None:
            return None
        w = self._tensor(prefix, "weight", experts, source)
        b = self._tensor(prefix, "biases", experts, source)
        if w is None:
            raise ValueError(f"{prefix}: scales without a weight")
        if w.ndim == 2:
            w, s = w[None], s[None]
            b = None if b is None else b[None]
        # the override key is the stacked name: the reference registers after sanitize
        # (src/llm/llm_factory.cpp:110-116)
        bits, gs = self.quant_for(prefix)
        E, N, words = w.shape
        K = words * 32 // bits
        if s.shape != (E, N, K // gs):
            raise ValueError(f"{prefix}: scales {s.shape} do not match {bits}-bit codes {w.shape}, group {gs}")
        return HostQWeight(np.ascontiguousarray(w, np.uint32), np.ascontiguousarray(s),
                           None if b is None else np.ascontiguousarray(b), E, N, K, gs, bits)


def _cfg_int(c: dict, key: str, default: Optional[int]) -> int:
    v = c.get(key)
    if v is None:
        if default is None:
            raise ValueError(f"config.json: missing {key!r}")
        return default
    return int(v)


def load_moe_layer(directory: str, layer: int, config: Optional[dict] = None,
                   router_variant: Optional[int] = None) -> HostLayer:
    """The MoE block of decoder layer `layer` (router, stacked experts, shared expert).

    router_variant overrides the model family's router (for DeepSeek-V3: the default
    ROUTE_SIGMOID follows deepseek_v3.cpp:304-350 as written; ROUTE_SIGMOID_GROUP applies
    the correction bias and the group limit, the "noaux_tc" rule of nemotron_h.cpp:405-468)."""
    ck = Checkpoint(directory, config)
    c = ck.config
    mt = c.get("model_type", "qwen3_moe")
    if mt not in _MODELS:
        raise ValueError(f"model_type {mt!r}: MoE naming not supported (have {sorted(_MODELS)})")
    nm = _MODELS[mt]
    H = int(c["hidden_size"])
    I = _cfg_int(c, nm.intermediate_key, nm.intermediate_default)
    E = _cfg_int(c, nm.experts_key, nm.experts_default)
    k = _cfg_int(c, "num_experts_per_tok", nm.topk_default)
    if mt == "deepseek_v3":
        # deepseek_v3.cpp:402-404: dense MLP below first_k_dense_replace and off moe_layer_freq
        if layer < int(c.get("first_k_dense_replace", 0)) or layer % int(c.get("moe_layer_freq", 1)) != 0:
            raise ValueError(f"deepseek_v3 layer {layer} is a dense MLP, not an MoE block")
    p = f"model.layers.{layer}.{nm.block}"
    if any(n.endswith("weight_scale_inv") for n in ck.index if n.startswith(p + ".")):
        raise ValueError(f"{p}: block-fp8 (weight_scale_inv) tensors are not MLX affine quantized")
    q = {dst: ck.qweight(f"{p}.switch_mlp.{dst}", E, src) for src, dst in nm.projs}
    gate, up, down = q["gate_proj"], q["up_proj"], q["down_proj"]
    if gate is None or up is None or down is None:
        raise ValueError(f"{p}: expert projections are not quantized (MLX affine) in this checkpoint")
    if (gate.N, gate.K, down.N, down.K, gate.experts) != (I, H, H, I, E):
        raise ValueError(f"{p}: expert shapes do not match hidden {H}, intermediate {I}, {E} experts")
    router_q = ck.qweight(f"{p}.gate")
    router_w = None if router_q is not None else ck.get(f"{p}.gate.weight")
    score_bias = None
    if nm.score_bias and ck.has(f"{p}.gate.e_score_correction_bias"):
        score_bias = np.ascontiguousarray(ck.get_f32(f"{p}.gate.e_score_correction_bias"))
    shared, Is = None, 0
    if nm.shared and ck.has(f"{p}.{nm.shared}.gate_proj.weight"):
        sg, su, sd = (ck.qweight(f"{p}.{nm.shared}.{n}_proj") for n in ("gate", "up", "down"))
        if sg is None or su is None or sd is None:
            raise ValueError(f"{p}: shared expert projections are not quantized")
        sgw = None
        if nm.shared_gate:
            # the sigmoid gate: quantized [1][1, H] (MLX conversions) or bf16 [1, H]
            sgw = ck.qweight(f"{p}.{nm.shared_gate}")
            if sgw is None and ck.has(f"{p}.{nm.shared_gate}.weight"):
                sgw = ck.get(f"{p}.{nm.shared_gate}.weight")
        if mt == "deepseek_v3" and sg.N != I * _cfg_int(c, "n_shared_experts", 1):
            raise ValueError(f"{p}: shared expert width {sg.N} != moe_intermediate_size * n_shared_experts")
        shared, Is = (sg, su, sd, sgw), sg.N
    variant = nm.variant if router_variant is None else int(router_variant)
    if variant >= ROUTE_SIGMOID_GROUP and score_bias is None:
        score_bias = np.zeros(E, np.float32)  # the gate's initial value (deepseek_v3.cpp:301)
    group_kw = {}
    if mt == "deepseek_v3":
        group_kw = dict(n_group=int(c.get("n_group", 1)), topk_group=int(c.get("topk_group") or 1),
                        routed_scaling_factor=float(c.get("routed_scaling_factor", 1.0)))
    cfg = MoeConfig(name=f"{mt}:layer{layer}", config_id=0, hidden=H, intermediate=I, num_experts=E, top_k=k,
                    variant=variant, norm_topk_prob=bool(c.get("norm_topk_prob", False)), bits=gate.bits,
                    group_size=gate.group_size, shared_intermediate=Is,
                    shared_gated=shared is not None and shared[3] is not None, **group_kw)
    return HostLayer(cfg, router_w, gate, up, down, score_bias if variant >= ROUTE_SIGMOID_GROUP else None,
                     shared, router_q)
