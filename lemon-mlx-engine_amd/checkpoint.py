"""checkpoint.py -- one MoE layer of an MLX-format checkpoint directory (safetensors)
as a ``workloads.HostLayer``, ready for ``MoeBlock.from_host``.

Follows the reference's ingestion steps:

* files: ``load_safetensors_from_directory`` (src/common/safetensors.cpp:23-77) --
  ``model.safetensors.index.json`` shards first, then ``model.safetensors``, else
  every ``*.safetensors`` of the directory;
* names: a VLM checkpoint's text model is renamed the way ``Qwen35MoEModel::sanitize_impl``
  does (src/llm/models/qwen35_moe.cpp:1046-1078): ``language_model.`` stripped,
  ``model.language_model.`` -> ``model.``, vision tensors skipped;
* per-expert tensors ``<block>.experts.{e}.<proj>.*`` are stacked into the
  ``<block>.switch_mlp.*`` layout [E, N, ...] for ``.weight``, ``.scales`` and
  ``.biases`` (``Qwen3MoEModel::sanitize_impl``, src/llm/models/qwen3_moe.cpp:291-318;
  ``DeepseekV3Model::sanitize_impl``, src/llm/models/deepseek_v3.cpp:531-555;
  ``PhiMoEModel::sanitize_impl``, src/llm/models/phimoe.cpp:208-235, which also renames
  ``w1/w2/w3`` to ``gate_proj/down_proj/up_proj``; qwen35_moe.cpp:1110-1160);
* a fused ``experts.gate_up_proj`` is split into gate and up: at the middle row for
  Qwen3.5-MoE (qwen35_moe.cpp:1080-1107), even rows -> gate and odd rows -> up for GPT-OSS,
  with its ``gate_up_proj_bias`` split the same way (``GPTOSSModel::sanitize_impl``,
  src/llm/models/gptoss.cpp:305-350; ``down_proj`` / ``down_proj_bias`` become
  ``down_proj.weight`` / ``down_proj.bias``).  The reference splits the bare (unquantized)
  tensor; its quantized form (``.weight`` / ``.scales`` / ``.biases``, split row for row
  alike) is read too;
* a tensor is quantized iff ``<prefix>.scales`` exists; its bits and group size are
  the config's ``quantization`` defaults (64, 4) unless the ``quantization`` entry
  names the prefix itself (``register_quantized_weights``,
  src/common/quantize_utils.cpp:14-104; the per-prefix overrides of
  src/common/base_config.cpp:28-73, with a ``language_model.`` prefix stripped).

Tensor data are memory-mapped; only the tensors of the requested layer are read.
Models (``_MODELS``): Qwen3-MoE (``qwen3_moe``: top-k of logits), Qwen3-Next
(``qwen3_next``: top-k of probabilities, gated shared expert), Qwen3.5-MoE (``qwen3_5_moe``,
``qwen3_5``: ``moe_route`` -- softmax over the top-k logits -- when ``norm_topk_prob``
(default true), else top-k of logits with the softmax over all; gated shared expert;
config under ``text_config``; qwen35_moe.cpp:25-70, 680-725), DeepSeek-V3 (``deepseek_v3``:
sigmoid router with ``e_score_correction_bias``, ungated shared experts of
``moe_intermediate_size * n_shared_experts``; src/llm/models/deepseek_v3.cpp:21-62, 294-381),
PhiMoE (``phimoe``: ``block_sparse_moe``, softmax over the k selected logits;
src/llm/models/phimoe.cpp:11-30, 85-105) and GPT-OSS (``gpt_oss``: stacked ``mlp.experts``
with SwitchLinear biases, ``mlp.router`` with a bias, softmax over the k selected logits, the
clipped SwiGLU; src/llm/models/gptoss.cpp:11-38, 118-178).  Only dense MLX-affine
quantized experts are read; unquantized (bf16) experts raise.
"""
from __future__ import annotations

import json
import os
import struct
from dataclasses import dataclass
from typing import Dict, Optional, Tuple

import numpy as np

from . import (ACT_GPTOSS, ACT_SWIGLU, ROUTE_SIGMOID, ROUTE_SIGMOID_GROUP, ROUTE_SOFTMAX_TOPK,
               ROUTE_TOPK_LOGITS, ROUTE_TOPK_PROBS)
from .workloads import HostLayer, HostQWeight, MoeConfig

_DTYPES = {"BF16": np.uint16, "F16": np.float16, "F32": np.float32, "U32": np.uint32, "I32": np.int32,
           "U8": np.uint8, "U16": np.uint16}

_PROJS = (("gate_proj", "gate_proj"), ("up_proj", "up_proj"), ("down_proj", "down_proj"))


@dataclass(frozen=True)
class _Naming:
    """Where one model family keeps its MoE block: config keys (with the reference's
    defaults), the block's module names and the per-expert projection names."""
    variant: int
    block: str = "mlp"                              # model.layers.{l}.<block>
    experts_key: str = "num_experts"
    experts_default: Optional[int] = None
    topk_default: Optional[int] = None
    intermediate_key: str = "moe_intermediate_size"
    intermediate_default: Optional[int] = None
    projs: Tuple[Tuple[str, str], ...] = _PROJS     # (per-expert name, stacked name)
    shared: Optional[str] = None                    # shared expert module under the block
    shared_gate: Optional[str] = None               # its sigmoid gate (Qwen3-Next, Qwen3.5)
    score_bias: bool = False                        # gate.e_score_correction_bias (DeepSeek)
    stacked: str = "switch_mlp"                     # module of the stacked experts
    router: str = "gate"                            # module of the router projection
    linear_bias: bool = False                       # SwitchLinear biases and a router bias (GPT-OSS)
    activation: int = ACT_SWIGLU                    # moe_activation of the experts
    fused: Optional[str] = None                     # experts.gate_up_proj split: "halves" / "interleaved"
    vlm: bool = False                               # text_config nesting and language_model. names
    variant_norm: Optional[int] = None              # router variant when norm_topk_prob is set
    norm_default: bool = False                      # norm_topk_prob when the config omits it


_MODELS = {
    # qwen3_moe.cpp:17-47, 155-175
    "qwen3_moe": _Naming(ROUTE_TOPK_LOGITS),
    # qwen3_next.cpp:452-490: shared_expert + shared_expert_gate
    "qwen3_next": _Naming(ROUTE_TOPK_PROBS, shared="shared_expert", shared_gate="shared_expert_gate"),
    # qwen35_moe.cpp:25-70 (config, text_config, norm_topk_prob default true), 680-725 (block:
    # moe_route if norm_topk_prob, else argpartition + softmax over all), 1046-1160 (sanitize)
    "qwen3_5_moe": _Naming(ROUTE_TOPK_LOGITS, shared="shared_expert", shared_gate="shared_expert_gate",
                           fused="halves", vlm=True, variant_norm=ROUTE_SOFTMAX_TOPK, norm_default=True),
    # deepseek_v3.cpp:21-62 (config), 294-381 (gate, shared_experts, combine)
    "deepseek_v3": _Naming(ROUTE_SIGMOID, experts_key="n_routed_experts", experts_default=1, topk_default=1,
                           shared="shared_experts", score_bias=True),
    # phimoe.cpp:11-30 (config defaults), 85-105 (block), 208-235 (w1/w2/w3 renames)
    "phimoe": _Naming(ROUTE_SOFTMAX_TOPK, block="block_sparse_moe", experts_key="num_local_experts",
                      experts_default=16, topk_default=2, intermediate_key="intermediate_size",
                      intermediate_default=6400,
                      projs=(("w1", "gate_proj"), ("w3", "up_proj"), ("w2", "down_proj"))),
    # gptoss.cpp:11-38 (config), 118-178 (MLP: router with bias, top-k of logits + softmax over the
    # k, SwitchLinear(bias=true) x3 under mlp.experts, swiglu(x_gate, x_up)), 305-350 (sanitize)
    "gpt_oss": _Naming(ROUTE_SOFTMAX_TOPK, experts_key="num_local_experts", intermediate_key="intermediate_size",
                       stacked="experts", router="router", linear_bias=True, activation=ACT_GPTOSS,
                       fused="interleaved"),
}
_MODELS["qwen3_5"] = _MODELS["qwen3_5_moe"]  # llm_factory.cpp:143-145: the same model class


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


def vlm_name(key: str) -> Optional[str]:
    """A VLM checkpoint's tensor name as the text model's (None: a vision tensor, skipped);
    qwen35_moe.cpp:1046-1078."""
    if key.startswith("vision_tower") or key.startswith("model.visual"):
        return None
    if key.startswith("language_model."):
        key = key[len("language_model."):]
    if key.startswith("model.language_model."):
        key = "model." + key[len("model.language_model."):]
    return key


class Checkpoint:
    """Tensor index of a checkpoint directory (headers only until a tensor is read).
    vlm: index the tensors under their text-model names (vlm_name)."""

    def __init__(self, directory: str, config: Optional[dict] = None, vlm: bool = False):
        if config is None:
            with open(os.path.join(directory, "config.json")) as f:
                config = json.load(f)
        self.config = config
        self.index: Dict[str, tuple] = {}
        for path in checkpoint_files(directory):
            header, base = read_header(path)
            for name, info in header.items():
                key = vlm_name(name) if vlm else name
                if key is not None:
                    self.index[key] = (path, base, info)  # later files win, as in the reference
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
        """prefix.suffix, or the per-expert tensors stacked (prefix = '...<stacked>.<proj>';
        source = the per-expert projection's own name, default <proj>)."""
        if self.has(f"{prefix}.{suffix}"):
            return self.get(f"{prefix}.{suffix}")
        if experts is None or ".switch_mlp." not in prefix:
            return None
        head, proj = prefix.rsplit(".switch_mlp.", 1)
        keys = [f"{head}.experts.{e}.{source or proj}.{suffix}" for e in range(experts)]
        if not self.has(keys[0]):
            return None
        missing = [k for k in keys if not self.has(k)]
        if missing:
            raise ValueError(f"{prefix}: {len(missing)} of {experts} per-expert tensors missing ({missing[0]})")
        return np.stack([self.get(k) for k in keys])

    def make_qweight(self, prefix: str, w, s, b) -> HostQWeight:
        """A HostQWeight from the packed codes, scales and biases of `prefix` (stacked [E, N, ...] or one
        [N, ...] matrix as experts = 1); bits and group size from the quantization entry of `prefix`."""
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

    def qweight(self, prefix: str, experts: Optional[int] = None,
                source: Optional[str] = None) -> Optional[HostQWeight]:
        """A quantized projection (stacked [E, N, K*bits/32] or one [N, K*bits/32]
        matrix as experts = 1), or None when the tensor is not quantized."""
        s = self._tensor(prefix, "scales", experts, source)
        if s is None:
            return None
        return self.make_qweight(prefix, self._tensor(prefix, "weight", experts, source), s,
                                 self._tensor(prefix, "biases", experts, source))


def _cfg_int(c: dict, key: str, default: Optional[int]) -> int:
    v = c.get(key)
    if v is None:
        if default is None:
            raise ValueError(f"config.json: missing {key!r}")
        return default
    return int(v)


def _split_rows(a: np.ndarray, how: str) -> Tuple[np.ndarray, np.ndarray]:
    """Rows (axis -2 of [E, 2I, ...], axis -1 of a bias [E, 2I]) of a fused gate|up tensor ->
    (gate, up): halves (qwen35_moe.cpp:1088-1102) or even / odd rows (gptoss.cpp:315-318, 330-332)."""
    ax = a.ndim - 2 if a.ndim >= 3 else a.ndim - 1
    n = a.shape[ax]
    if n % 2:
        raise ValueError(f"fused gate|up tensor with an odd row count {n}")
    idx_g = np.arange(0, n // 2) if how == "halves" else np.arange(0, n, 2)
    idx_u = np.arange(n // 2, n) if how == "halves" else np.arange(1, n, 2)
    return np.ascontiguousarray(np.take(a, idx_g, axis=ax)), np.ascontiguousarray(np.take(a, idx_u, axis=ax))


def _expert_projs(ck: Checkpoint, nm: _Naming, p: str, E: int) -> Dict[str, Optional[HostQWeight]]:
    """gate_proj / up_proj / down_proj of the block at p, quantized, or None where not quantized:
    stacked under <stacked>, per-expert, or (nm.fused) a fused experts.gate_up_proj."""
    sp = f"{p}.{nm.stacked}"
    q = {dst: ck.qweight(f"{sp}.{dst}", E, src) for src, dst in nm.projs}
    fp = f"{p}.experts.gate_up_proj"
    if nm.fused and q["gate_proj"] is None and (ck.has(fp) or ck.has(f"{fp}.weight")):
        if not ck.has(f"{fp}.scales"):
            return {"gate_proj": None, "up_proj": None, "down_proj": q["down_proj"]}  # unquantized
        w, s = ck.get(f"{fp}.weight"), ck.get(f"{fp}.scales")
        b = ck.get(f"{fp}.biases") if ck.has(f"{fp}.biases") else None
        # one quantization entry for both halves: the fused tensor's own, else the stacked names'
        halves = [_split_rows(a, nm.fused) if a is not None else (None, None) for a in (w, s, b)]
        for i, dst in enumerate(("gate_proj", "up_proj")):
            name = fp if fp in ck.overrides else f"{sp}.{dst}"
            q[dst] = ck.make_qweight(name, halves[0][i], halves[1][i], halves[2][i])
    if q["down_proj"] is None and nm.fused and ck.has(f"{p}.experts.down_proj.scales"):
        q["down_proj"] = ck.qweight(f"{p}.experts.down_proj")
    return q


def _linear_biases(ck: Checkpoint, nm: _Naming, p: str, q: Dict[str, HostQWeight]) -> None:
    """SwitchLinear biases [E, N] (GPT-OSS: <stacked>.<proj>.bias, or the fused experts.gate_up_proj_bias
    split as its weight, and experts.down_proj_bias) onto the projections."""
    sp = f"{p}.{nm.stacked}"
    fb = f"{p}.experts.gate_up_proj_bias"
    if ck.has(fb) and not ck.has(f"{sp}.gate_proj.bias"):
        g, u = _split_rows(ck.get(fb), nm.fused or "interleaved")
        q["gate_proj"].linear_bias, q["up_proj"].linear_bias = g, u
    for dst in ("gate_proj", "up_proj", "down_proj"):
        if ck.has(f"{sp}.{dst}.bias"):
            q[dst].linear_bias = ck.get(f"{sp}.{dst}.bias")
    if q["down_proj"].linear_bias is None and ck.has(f"{p}.experts.down_proj_bias"):
        q["down_proj"].linear_bias = ck.get(f"{p}.experts.down_proj_bias")
    for dst, w in q.items():
        lb = w.linear_bias
        if lb is not None and (lb.shape != (w.experts, w.N) or lb.dtype != np.uint16):
            raise ValueError(f"{p}: {dst} bias must be bf16 [{w.experts}, {w.N}], got {lb.dtype} {lb.shape}")


def load_moe_layer(directory: str, layer: int, config: Optional[dict] = None,
                   router_variant: Optional[int] = None) -> HostLayer:
    """The MoE block of decoder layer `layer` (router, stacked experts, shared expert).

    router_variant overrides the model family's router (for DeepSeek-V3: the default
    ROUTE_SIGMOID follows deepseek_v3.cpp:304-350 as written; ROUTE_SIGMOID_GROUP applies
    the correction bias and the group limit, the "noaux_tc" rule of nemotron_h.cpp:405-468)."""
    if config is None:
        with open(os.path.join(directory, "config.json")) as f:
            config = json.load(f)
    mt = config.get("model_type", "qwen3_moe")
    if mt not in _MODELS:
        raise ValueError(f"model_type {mt!r}: MoE naming not supported (have {sorted(_MODELS)})")
    nm = _MODELS[mt]
    ck = Checkpoint(directory, config, vlm=nm.vlm)
    c = config.get("text_config", config) if nm.vlm else config
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
    q = _expert_projs(ck, nm, p, E)
    gate, up, down = q["gate_proj"], q["up_proj"], q["down_proj"]
    if gate is None or up is None or down is None:
        raise ValueError(f"{p}: expert projections are not quantized (MLX affine) in this checkpoint")
    if (gate.N, gate.K, down.N, down.K, gate.experts) != (I, H, H, I, E):
        raise ValueError(f"{p}: expert shapes do not match hidden {H}, intermediate {I}, {E} experts")
    if nm.linear_bias:
        _linear_biases(ck, nm, p, q)
    rp = f"{p}.{nm.router}"
    router_q = ck.qweight(rp)
    router_w = None if router_q is not None else ck.get(f"{rp}.weight")
    router_b = None
    if nm.linear_bias and ck.has(f"{rp}.bias"):
        if router_q is not None:
            router_q.linear_bias = ck.get(f"{rp}.bias").reshape(1, E)
        else:
            router_b = ck.get(f"{rp}.bias")
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
    norm = bool(c.get("norm_topk_prob", nm.norm_default))
    variant = nm.variant_norm if nm.variant_norm is not None and norm else nm.variant
    variant = variant if router_variant is None else int(router_variant)
    if variant >= ROUTE_SIGMOID_GROUP and score_bias is None:
        score_bias = np.zeros(E, np.float32)  # the gate's initial value (deepseek_v3.cpp:301)
    group_kw = {}
    if mt == "deepseek_v3":
        group_kw = dict(n_group=int(c.get("n_group", 1)), topk_group=int(c.get("topk_group") or 1),
                        routed_scaling_factor=float(c.get("routed_scaling_factor", 1.0)))
    cfg = MoeConfig(name=f"{mt}:layer{layer}", config_id=0, hidden=H, intermediate=I, num_experts=E, top_k=k,
                    variant=variant, norm_topk_prob=norm, bits=gate.bits, group_size=gate.group_size,
                    shared_intermediate=Is, shared_gated=shared is not None and shared[3] is not None,
                    activation=nm.activation, **group_kw)
    return HostLayer(cfg, router_w, gate, up, down, score_bias if variant >= ROUTE_SIGMOID_GROUP else None,
                     shared, router_q, router_b)
