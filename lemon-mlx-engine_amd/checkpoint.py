"""checkpoint.py -- one MoE layer of an MLX-format checkpoint directory (safetensors)
as a ``workloads.HostLayer``, ready for ``MoeBlock.from_host``.

Follows the reference's ingestion steps:

* files: ``load_safetensors_from_directory`` (src/common/safetensors.cpp:23-77) --
  ``model.safetensors.index.json`` shards first, then ``model.safetensors``, else
  every ``*.safetensors`` of the directory;
* per-expert tensors ``mlp.experts.{e}.{gate,up,down}_proj.*`` are stacked into the
  ``mlp.switch_mlp.*`` layout [E, N, ...] (``Qwen3MoEModel::sanitize_impl``,
  src/llm/models/qwen3_moe.cpp:291-318; stacked here for ``.scales`` and ``.biases``
  as well, which a per-expert quantized checkpoint holds);
* a tensor is quantized iff ``<prefix>.scales`` exists; its bits and group size are
  the config's ``quantization`` defaults (64, 4) unless the ``quantization`` entry
  names the prefix itself (``register_quantized_weights``,
  src/common/quantize_utils.cpp:14-104; the per-prefix overrides of
  src/common/base_config.cpp:28-73, with a ``language_model.`` prefix stripped).

Tensor data are memory-mapped; only the tensors of the requested layer are read.
Models: Qwen3-MoE (``qwen3_moe``: top-k of logits) and Qwen3-Next (``qwen3_next``:
top-k of probabilities, gated shared expert) naming.
"""
from __future__ import annotations

import json
import os
import struct
from typing import Dict, Optional, Tuple

import numpy as np

from . import ROUTE_TOPK_LOGITS, ROUTE_TOPK_PROBS
from .workloads import HostLayer, HostQWeight, MoeConfig

_DTYPES = {"BF16": np.uint16, "F16": np.float16, "F32": np.float32, "U32": np.uint32, "I32": np.int32,
           "U8": np.uint8, "U16": np.uint16}
_MODELS = {"qwen3_moe": ROUTE_TOPK_LOGITS, "qwen3_next": ROUTE_TOPK_PROBS}


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

    def _tensor(self, prefix: str, suffix: str, experts: Optional[int]) -> Optional[np.ndarray]:
        """prefix.suffix, or the per-expert tensors stacked (prefix = '...switch_mlp.<proj>')."""
        if self.has(f"{prefix}.{suffix}"):
            return self.get(f"{prefix}.{suffix}")
        if experts is None:
            return None
        head, proj = prefix.rsplit(".switch_mlp.", 1)
        keys = [f"{head}.experts.{e}.{proj}.{suffix}" for e in range(experts)]
        if not all(self.has(k) for k in keys):
            return None
        return np.stack([self.get(k) for k in keys])

    def qweight(self, prefix: str, experts: Optional[int] = None) -> Optional[HostQWeight]:
        """A quantized projection (stacked [E, N, K*bits/32] or one [N, K*bits/32]
        matrix as experts = 1), or None when the tensor is not quantized."""
        s = self._tensor(prefix, "scales", experts)
        if s is None:
            return None
        w = self._tensor(prefix, "weight", experts)
        b = self._tensor(prefix, "biases", experts)
        if w.ndim == 2:
            w, s = w[None], s[None]
            b = None if b is None else b[None]
        key = prefix if self.has(f"{prefix}.scales") else prefix.replace(".switch_mlp.", ".experts.0.")
        bits, gs = self.quant_for(key)
        E, N, words = w.shape
        K = words * 32 // bits
        if s.shape != (E, N, K // gs):
            raise ValueError(f"{prefix}: scales {s.shape} do not match {bits}-bit codes {w.shape}, group {gs}")
        return HostQWeight(np.ascontiguousarray(w, np.uint32), np.ascontiguousarray(s),
                           None if b is None else np.ascontiguousarray(b), E, N, K, gs, bits)


def load_moe_layer(directory: str, layer: int, config: Optional[dict] = None) -> HostLayer:
    """The MoE block of decoder layer `layer` (router, stacked experts, shared expert)."""
    ck = Checkpoint(directory, config)
    c = ck.config
    mt = c.get("model_type", "qwen3_moe")
    if mt not in _MODELS:
        raise ValueError(f"model_type {mt!r}: MoE naming not supported (have {sorted(_MODELS)})")
    H, I = int(c["hidden_size"]), int(c["moe_intermediate_size"])
    E, k = int(c["num_experts"]), int(c["num_experts_per_tok"])
    p = f"model.layers.{layer}.mlp"
    gate, up, down = (ck.qweight(f"{p}.switch_mlp.{n}_proj", E) for n in ("gate", "up", "down"))
    if gate is None or up is None or down is None:
        raise ValueError(f"{p}: expert projections are not quantized (MLX affine) in this checkpoint")
    if (gate.N, gate.K, down.N, down.K, gate.experts) != (I, H, H, I, E):
        raise ValueError(f"{p}: expert shapes do not match hidden {H}, intermediate {I}, {E} experts")
    router_q = ck.qweight(f"{p}.gate")
    router_w = None if router_q is not None else ck.get(f"{p}.gate.weight")
    shared, Is = None, 0
    if ck.has(f"{p}.shared_expert.gate_proj.weight"):
        sg, su, sd = (ck.qweight(f"{p}.shared_expert.{n}_proj") for n in ("gate", "up", "down"))
        if sg is None or su is None or sd is None:
            raise ValueError(f"{p}: shared expert projections are not quantized")
        # the sigmoid gate: quantized [1][1, H] (MLX conversions) or bf16 [1, H]
        sgw = ck.qweight(f"{p}.shared_expert_gate")
        if sgw is None and ck.has(f"{p}.shared_expert_gate.weight"):
            sgw = ck.get(f"{p}.shared_expert_gate.weight")
        shared, Is = (sg, su, sd, sgw), sg.N
    cfg = MoeConfig(name=f"{mt}:layer{layer}", config_id=0, hidden=H, intermediate=I, num_experts=E, top_k=k,
                    variant=_MODELS[mt], norm_topk_prob=bool(c.get("norm_topk_prob", False)), bits=gate.bits,
                    group_size=gate.group_size, shared_intermediate=Is,
                    shared_gated=shared is not None and shared[3] is not None)
    return HostLayer(cfg, router_w, gate, up, down, None, shared, router_q)
