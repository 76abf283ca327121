"""MI355X-native quantized mixture-of-experts block (lemon-mlx-engine's MoE path).

This module binds the C ABI of ``libmoe_mi355x.so`` (declared in
``include/moe_mi355x.h``) with ctypes.  The arithmetic runs in the library's
hand-written HIP kernels for gfx950; torch is used here only to own device
memory and to name the current HIP stream.  There is no CPU fallback: if the
shared library is missing, every call raises.

The operator names and argument meanings follow the reference:

* ``router_logits``  -- ``linear_forward(x, gate_weight)``,
  include/mlx-lm/common/quantized_linear.h:73-96
* ``route``          -- the per-model routers (qwen3_moe.cpp:155-168,
  qwen3_next.cpp:452-469, phimoe.cpp:93-101, deepseek_v3.cpp:304-350,
  nemotron_h.cpp:405-468) and ``moe_route`` (gated_delta.cpp:973-998)
* ``bucket``         -- ``gather_sort``'s argsort / inverse, switch_layers.cpp:17-30
* ``gather_qmm``     -- the call at switch_layers.cpp:94-102
* ``swiglu``         -- activations.h:22-30
* ``combine``        -- ``scatter_unsort`` + ``sum(y * scores, -2)``,
  switch_layers.cpp:32-46 and qwen3_moe.cpp:173-174
* ``take_rows``      -- the row gathers of ``gather_sort`` / ``scatter_unsort``,
  switch_layers.cpp:17-46
* ``add_expert_bias`` -- SwitchLinear's linear bias, switch_layers.cpp:111-114
* ``switch_glu``     -- ``SwitchGLU::operator()``, switch_layers.cpp:200-245
* ``MoeBlock``       -- the model MoE blocks' ``operator()``
"""
from __future__ import annotations

import ctypes
from pathlib import Path

_HERE = Path(__file__).resolve().parent
LIB_PATH = _HERE / "libmoe_mi355x.so"

MOE_OK = 0
MOE_E_INVALID_ARG = -1
MOE_E_UNSUPPORTED = -2
MOE_E_WORKSPACE = -3
MOE_E_HIP = -4
MOE_E_INDEX = -6

ROUTE_TOPK_LOGITS = 1
ROUTE_TOPK_PROBS = 2
ROUTE_SOFTMAX_TOPK = 3
ROUTE_SIGMOID = 5
ROUTE_SIGMOID_GROUP = 6
ROUTE_SIGMOID_GROUP_DROP_BEST = 7  # R6 as nemotron_h.cpp:425-447 writes it (drops the best groups)
ROUTE_SIGMOID_CORRECTED = 8        # Bailing: weights from the corrected scores
ROUTE_GLM4_SIGMOID = 9             # GLM4-MoE gate, scoring_func "sigmoid" (no group limit, no epsilon)
ROUTE_GLM4_SOFTMAX = 10            # GLM4-MoE gate, scoring_func "softmax"
ROUTE_LFM2 = 11                    # LFM2-MoE gate (fp32 softmax + expert bias, weights the biased probs)

# moe_activation (the routed experts' GLU activation)
ACT_SWIGLU = 0
ACT_GPTOSS = 1            # gptoss.cpp:50-58 as called at :158, swiglu(x_gate, x_up)
ACT_GPTOSS_UPSTREAM = 2   # the same function with the upstream roles (x_linear = up, x_glu = gate)

# MOE_ABI_VERSION of include/moe_mi355x.h this binding's structs and signatures follow
ABI_VERSION = 3


class MoeError(RuntimeError):
    """A non-zero status from the C ABI."""

    def __init__(self, status: int, where: str, detail: str = ""):
        self.status = status
        msg = f"{where}: {_status_string(status)} ({status})"
        if detail:
            msg += f": {detail}"
        super().__init__(msg)


class MoeArgumentError(MoeError, ValueError):
    """Invalid or unsupported arguments (the reference throws std::invalid_argument)."""


class RouterParams(ctypes.Structure):
    _fields_ = [
        ("variant", ctypes.c_int32),
        ("num_experts", ctypes.c_int32),
        ("top_k", ctypes.c_int32),
        ("norm_topk_prob", ctypes.c_int32),
        ("n_group", ctypes.c_int32),
        ("topk_group", ctypes.c_int32),
        ("routed_scaling_factor", ctypes.c_float),
    ]


class QWeightC(ctypes.Structure):
    _fields_ = [
        ("w", ctypes.c_void_p),
        ("scales", ctypes.c_void_p),
        ("biases", ctypes.c_void_p),
        ("experts", ctypes.c_int32),
        ("N", ctypes.c_int32),
        ("K", ctypes.c_int32),
        ("group_size", ctypes.c_int32),
        ("bits", ctypes.c_int32),
        ("linear_bias", ctypes.c_void_p),
    ]


class BlockDesc(ctypes.Structure):
    _fields_ = [
        ("hidden", ctypes.c_int32),
        ("intermediate", ctypes.c_int32),
        ("num_experts", ctypes.c_int32),
        ("router", RouterParams),
        ("router_weight", ctypes.c_void_p),
        ("score_bias", ctypes.c_void_p),
        ("gate", QWeightC),
        ("up", QWeightC),
        ("down", QWeightC),
        ("shared_intermediate", ctypes.c_int32),
        ("shared_gate", QWeightC),
        ("shared_up", QWeightC),
        ("shared_down", QWeightC),
        ("shared_gate_weight", ctypes.c_void_p),
        ("router_q", QWeightC),
        ("router_bias", ctypes.c_void_p),
        ("shared_gate_q", QWeightC),
        ("activation", ctypes.c_int32),
    ]


class BlockAux(ctypes.Structure):
    _fields_ = [
        ("logits", ctypes.c_void_p),
        ("inds", ctypes.c_void_p),
        ("scores", ctypes.c_void_p),
        ("perm", ctypes.c_void_p),
        ("inv_perm", ctypes.c_void_p),
        ("offsets", ctypes.c_void_p),
    ]


_VP = ctypes.c_void_p
_I32 = ctypes.c_int32
_I64 = ctypes.c_int64
_U64 = ctypes.c_uint64
_SZ = ctypes.c_size_t
_F = ctypes.c_float

# name -> (restype, argtypes); every symbol declared in include/moe_mi355x.h
SIGNATURES = {
    "moe_version": (ctypes.c_int, []),
    "moe_status_string": (ctypes.c_char_p, [ctypes.c_int]),
    "moe_last_error": (ctypes.c_char_p, []),
    "moe_router_logits": (ctypes.c_int, [_VP, _VP, _VP, _I64, _I32, _I32, _VP, _VP]),
    "moe_route": (ctypes.c_int, [_VP, _VP, _I64, ctypes.POINTER(RouterParams), _VP, _VP, _VP]),
    "moe_bucket_workspace_size": (_SZ, [_I64, _I32, _I32]),
    "moe_bucket": (ctypes.c_int, [_VP, _I64, _I32, _I32, _VP, _VP, _VP, _VP, _VP, _SZ, _VP]),
    "moe_gather_qmm_workspace_size": (_SZ, [_I64, _I32, _I32]),
    "moe_gather_qmm": (ctypes.c_int, [_VP, ctypes.POINTER(QWeightC), _VP, _VP, _I64, _I32, _I32, _VP,
                                      _VP, _SZ, _VP]),
    "moe_gather_mm_workspace_size": (_SZ, [_I64, _I32, _I32]),
    "moe_gather_mm": (ctypes.c_int, [_VP, _VP, _VP, _I32, _I32, _I32, _VP, _VP, _I64, _I32, _I32, _VP, _VP, _SZ,
                                     _VP]),
    "moe_swiglu": (ctypes.c_int, [_VP, _VP, _I64, _VP, _VP]),
    "moe_gptoss_swiglu": (ctypes.c_int, [_VP, _VP, _I64, _VP, _VP]),
    "moe_add_rms_norm": (ctypes.c_int, [_VP, _VP, _VP, ctypes.c_float, _I64, _I32, _VP, _VP, _VP]),
    "moe_combine": (ctypes.c_int, [_VP, _VP, _VP, _I64, _I32, _I32, _VP, _VP]),
    "moe_take_rows": (ctypes.c_int, [_VP, _I64, _VP, _I64, _I32, _I64, _VP, _VP]),
    "moe_add_expert_bias": (ctypes.c_int, [_VP, _VP, _VP, _I64, _I32, _I32, _I32, _VP]),
    "moe_switch_glu_workspace_size": (_SZ, [ctypes.POINTER(QWeightC), ctypes.POINTER(QWeightC), _I64, _I32]),
    "moe_switch_mlp_workspace_size": (_SZ, [ctypes.POINTER(QWeightC), ctypes.POINTER(QWeightC), _I64, _I32]),
    "moe_switch_mlp_relu2": (ctypes.c_int, [ctypes.POINTER(QWeightC), ctypes.POINTER(QWeightC), _VP, _VP, _I64,
                                            _I32, _VP, _VP, _SZ, _VP]),
    "moe_switch_glu": (ctypes.c_int, [ctypes.POINTER(QWeightC), ctypes.POINTER(QWeightC),
                                      ctypes.POINTER(QWeightC), _VP, _VP, _I64, _I32, _I32, _VP, _VP, _SZ, _VP]),
    "moe_block_workspace_size": (_SZ, [ctypes.POINTER(BlockDesc), _I64]),
    "moe_block_graph_create": (ctypes.c_int, [ctypes.POINTER(BlockDesc), _VP, _I64, _VP, _VP, _SZ,
                                              ctypes.POINTER(ctypes.c_void_p)]),
    "moe_block_graph_launch": (ctypes.c_int, [ctypes.c_void_p, _VP]),
    "moe_block_graph_destroy": (ctypes.c_int, [ctypes.c_void_p]),
    "moe_block_forward": (ctypes.c_int, [ctypes.POINTER(BlockDesc), _VP, _I64, _VP,
                                         ctypes.POINTER(BlockAux), _VP, _SZ, _VP]),
    "moe_block_forward_noalloc": (ctypes.c_int, [ctypes.POINTER(BlockDesc), _VP, _I64, _VP,
                                                 ctypes.POINTER(BlockAux), _VP]),
    "moe_block_forward_add_norm": (ctypes.c_int, [ctypes.POINTER(BlockDesc), _VP, _VP, _VP, ctypes.c_float, _I64,
                                                  _VP, _VP, _VP, ctypes.POINTER(BlockAux), _VP, _SZ, _VP]),
    "moe_profile_enable": (ctypes.c_int, [ctypes.c_int]),
    "moe_profile_count": (ctypes.c_int, []),
    "moe_profile_record": (ctypes.c_int, [ctypes.c_int, ctypes.POINTER(ctypes.c_char_p),
                                          ctypes.POINTER(ctypes.c_float)]),
    "moe_synth_normal_bf16": (ctypes.c_int, [_U64, _U64, _F, _F, _I64, _I64, _VP]),
    "moe_synth_normal_f32": (ctypes.c_int, [_U64, _U64, _F, _F, _I64, _I64, _VP]),
    "moe_quantize_affine": (ctypes.c_int, [_VP, _I64, _I32, _I32, _I32, _VP, _VP, _VP]),
}

_lib = None


def lib() -> ctypes.CDLL:
    """The loaded HIP library.  Raises if it has not been built."""
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise ImportError(
                f"{LIB_PATH} is missing: build it with __graft_entry__.build() "
                "(there is no CPU fallback for the MoE kernels)")
        handle = ctypes.CDLL(str(LIB_PATH), mode=ctypes.RTLD_GLOBAL)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(handle, name)
            fn.restype = res
            fn.argtypes = args
        built = handle.moe_version()
        if built != ABI_VERSION:
            raise ImportError(f"{LIB_PATH} implements ABI version {built}, this binding version {ABI_VERSION}: "
                              "rebuild the library (__graft_entry__.build())")
        _lib = handle
    return _lib


def _status_string(status: int) -> str:
    try:
        return lib().moe_status_string(status).decode()
    except Exception:  # library missing while formatting an error
        return "status"


def check(status: int, where: str) -> None:
    if status == MOE_OK:
        return
    detail = ""
    if status == MOE_E_HIP:
        detail = lib().moe_last_error().decode()
    if status in (MOE_E_INVALID_ARG, MOE_E_UNSUPPORTED, MOE_E_INDEX):
        raise MoeArgumentError(status, where, detail)
    raise MoeError(status, where, detail)


from . import ops  # noqa: E402  (torch-facing wrappers)
from .ops import (  # noqa: E402,F401
    MoeBlock,
    QuantizedWeight,
    add_expert_bias,
    bucket,
    combine,
    gather_mm,
    gather_qmm,
    route,
    router_logits,
    swiglu,
    gptoss_swiglu,
    add_rms_norm,
    switch_glu,
    switch_mlp_relu2,
    take_rows,
)
