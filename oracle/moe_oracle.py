"""ctypes binding of the CPU checker ``build/libmoe_oracle.so``.

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py, never by the product.  Arrays are numpy; bf16 is
carried as uint16 bit patterns.  See moe_oracle.h for what each function
restates and how it is pinned.
"""
from __future__ import annotations

import ctypes
from pathlib import Path
from typing import Optional

import numpy as np

LIB_PATH = Path(__file__).resolve().parent / "build" / "libmoe_oracle.so"

R_TOPK_LOGITS, R_TOPK_PROBS, R_SOFTMAX_TOPK, R_SIGMOID, R_SIGMOID_GROUP = 1, 2, 3, 5, 6
R_SIGMOID_GROUP_DROP_BEST, R_SIGMOID_CORRECTED = 7, 8
R_GLM4_SIGMOID, R_GLM4_SOFTMAX = 9, 10
R_LFM2 = 11
ACT_SWIGLU, ACT_GPTOSS, ACT_GPTOSS_UPSTREAM = 0, 1, 2


class ORouter(ctypes.Structure):
    _fields_ = [("variant", ctypes.c_int32), ("num_experts", ctypes.c_int32), ("top_k", ctypes.c_int32),
                ("norm_topk_prob", ctypes.c_int32), ("n_group", ctypes.c_int32),
                ("topk_group", ctypes.c_int32), ("routed_scaling_factor", ctypes.c_float)]


class OQWeight(ctypes.Structure):
    _fields_ = [("w", ctypes.c_void_p), ("scales", ctypes.c_void_p), ("biases", ctypes.c_void_p),
                ("experts", ctypes.c_int32), ("N", ctypes.c_int32), ("K", ctypes.c_int32),
                ("group_size", ctypes.c_int32), ("bits", ctypes.c_int32), ("linear_bias", ctypes.c_void_p)]


class OBlock(ctypes.Structure):
    _fields_ = [("hidden", ctypes.c_int32), ("intermediate", ctypes.c_int32), ("num_experts", ctypes.c_int32),
                ("router", ORouter), ("router_weight", ctypes.c_void_p), ("score_bias", ctypes.c_void_p),
                ("gate", OQWeight), ("up", OQWeight), ("down", OQWeight),
                ("shared_intermediate", ctypes.c_int32), ("shared_gate", OQWeight), ("shared_up", OQWeight),
                ("shared_down", OQWeight), ("shared_gate_weight", ctypes.c_void_p), ("router_q", OQWeight),
                ("router_bias", ctypes.c_void_p), ("shared_gate_q", OQWeight),
                ("activation", ctypes.c_int32), ("hidden_f32", ctypes.c_int32)]


_lib = None


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise ImportError(f"{LIB_PATH} missing: run `make -C oracle` (or __graft_entry__.build())")
        L = ctypes.CDLL(str(LIB_PATH))
        vp, i32, i64 = ctypes.c_void_p, ctypes.c_int32, ctypes.c_int64
        sig = {
            "oracle_num_threads": (ctypes.c_int, []),
            "oracle_set_num_threads": (None, [ctypes.c_int]),
            "oracle_canon_expf": (ctypes.c_float, [ctypes.c_float]),
            "oracle_dequant": (None, [vp, vp, vp, i64, i32, i32, i32, vp]),
            "oracle_router_logits": (ctypes.c_int, [vp, vp, vp, i64, i32, i32, vp]),
            "oracle_route": (ctypes.c_int, [vp, vp, i64, ctypes.POINTER(ORouter), vp, vp, vp]),
            "oracle_bucket": (ctypes.c_int, [vp, i64, i32, i32, vp, vp, vp, vp]),
            "oracle_gather_qmm": (ctypes.c_int, [vp, ctypes.POINTER(OQWeight), vp, vp, i64, i32, vp]),
            "oracle_gather_mm": (ctypes.c_int, [vp, vp, vp, i32, i32, i32, vp, vp, i64, i32, vp]),
            "oracle_swiglu": (None, [vp, vp, i64, vp]),
            "oracle_gptoss_swiglu": (None, [vp, vp, i64, vp, vp]),
            "oracle_gather_qmm_f32x": (ctypes.c_int, [vp, ctypes.POINTER(OQWeight), vp, vp, i64, i32, vp]),
            "oracle_add_rms_norm": (None, [vp, vp, vp, ctypes.c_float, i64, i32, vp, vp]),
            "oracle_combine": (None, [vp, vp, i64, i32, i32, vp]),
            "oracle_moe_experts": (ctypes.c_int, [ctypes.POINTER(OBlock), vp, i64, vp, vp, vp, vp]),
            "oracle_block_forward": (ctypes.c_int, [ctypes.POINTER(OBlock), vp, i64, vp, vp, vp, vp]),
        }
        for n, (r, a) in sig.items():
            f = getattr(L, n)
            f.restype = r
            f.argtypes = a
        _lib = L
    return _lib


def _p(a: Optional[np.ndarray]):
    return None if a is None else ctypes.c_void_p(a.ctypes.data)


def _c(a, dtype):
    return np.ascontiguousarray(a, dtype=dtype)


def num_threads() -> int:
    return lib().oracle_num_threads()


def set_num_threads(n: int) -> None:
    lib().oracle_set_num_threads(n)


def canon_expf(x: float) -> float:
    return lib().oracle_canon_expf(x)


def dequant(w, scales, biases, rows: int, K: int, group_size: int, bits: int) -> np.ndarray:
    w, s = _c(w, np.uint32), _c(scales, np.uint16)
    b = None if biases is None else _c(biases, np.uint16)
    out = np.empty((rows, K), dtype=np.float32)
    lib().oracle_dequant(_p(w), _p(s), _p(b), rows, K, group_size, bits, _p(out))
    return out


def router_logits(x, wg, bias=None) -> np.ndarray:
    x, wg = _c(x, np.uint16), _c(wg, np.uint16)
    b = None if bias is None else _c(bias, np.uint16)
    T, H = x.shape
    E = wg.shape[0]
    out = np.empty((T, E), dtype=np.uint16)
    assert lib().oracle_router_logits(_p(x), _p(wg), _p(b), T, H, E, _p(out)) == 0
    return out


def make_router(variant, E, k, norm=True, n_group=1, topk_group=1, rsf=1.0) -> ORouter:
    return ORouter(variant, E, k, int(bool(norm)), n_group, topk_group, rsf)


def route(logits, params: ORouter, bias=None):
    """-> (inds uint32 [T,k], scores f32 [T,k], sel f32 [T,E])."""
    logits = _c(logits, np.uint16)
    T, E = logits.shape
    k = params.top_k
    b = None if bias is None else _c(bias, np.float32)
    inds = np.empty((T, k), dtype=np.uint32)
    scores = np.empty((T, k), dtype=np.float32)
    sel = np.empty((T, E), dtype=np.float32)
    rc = lib().oracle_route(_p(logits), _p(b), T, ctypes.byref(params), _p(inds), _p(scores), _p(sel))
    if rc != 0:
        raise ValueError(f"oracle_route rc={rc}")
    return inds, scores, sel


def bucket(inds, E: int):
    inds = _c(inds, np.uint32)
    T, k = inds.shape
    P = T * k
    perm = np.empty(P, np.int32)
    inv = np.empty(P, np.int32)
    se = np.empty(P, np.uint32)
    offs = np.empty(E + 1, np.int32)
    rc = lib().oracle_bucket(_p(inds), T, k, E, _p(perm), _p(inv), _p(se), _p(offs))
    if rc != 0:
        raise ValueError(f"oracle_bucket rc={rc}")
    return perm, inv, se, offs


def qweight(q, keep: list) -> OQWeight:
    """OQWeight view of an object with w/scales/biases/experts/N/K/group_size/bits (and optionally
    linear_bias, SwitchLinear's bias [experts, N] bf16)."""
    w, s = _c(q.w, np.uint32), _c(q.scales, np.uint16)
    b = None if q.biases is None else _c(q.biases, np.uint16)
    lb = getattr(q, "linear_bias", None)
    lb = None if lb is None else _c(lb, np.uint16)
    keep += [w, s, b, lb]
    return OQWeight(w.ctypes.data, s.ctypes.data, None if b is None else b.ctypes.data, q.experts, q.N, q.K,
                    q.group_size, q.bits, None if lb is None else lb.ctypes.data)


def gather_qmm(x, q, lhs, rhs, M: int = 1) -> np.ndarray:
    keep = []
    qw = qweight(q, keep)
    x = _c(x, np.uint16)
    rhs = _c(rhs, np.uint32)
    lhs = None if lhs is None else _c(lhs, np.uint32)
    batch = rhs.size
    out = np.empty((batch, M, q.N), np.uint16)
    rc = lib().oracle_gather_qmm(_p(x), ctypes.byref(qw), _p(lhs), _p(rhs), batch, M, _p(out))
    if rc != 0:
        raise ValueError(f"oracle_gather_qmm rc={rc}")
    return out


def gather_qmm_f32x(x, q, lhs, rhs, M: int = 1) -> np.ndarray:
    """gather_qmm of fp32 activations x [*, M, K] -> fp32 [batch, M, N] (bias added in fp32)."""
    keep = []
    qw = qweight(q, keep)
    x = _c(x, np.float32)
    rhs = _c(rhs, np.uint32)
    lhs = None if lhs is None else _c(lhs, np.uint32)
    batch = rhs.size
    out = np.empty((batch, M, q.N), np.float32)
    rc = lib().oracle_gather_qmm_f32x(_p(x), ctypes.byref(qw), _p(lhs), _p(rhs), batch, M, _p(out))
    if rc != 0:
        raise ValueError(f"oracle_gather_qmm_f32x rc={rc}")
    return out


def gather_mm(x, w, lhs, rhs, M: int = 1, linear_bias=None) -> np.ndarray:
    """Dense gather_mm: w bf16 [E, N, K]; -> out bf16 [batch, M, N]."""
    x, w = _c(x, np.uint16), _c(w, np.uint16)
    E, N, K = w.shape
    rhs = _c(rhs, np.uint32)
    lhs = None if lhs is None else _c(lhs, np.uint32)
    lb = None if linear_bias is None else _c(linear_bias, np.uint16)
    batch = rhs.size
    out = np.empty((batch, M, N), np.uint16)
    rc = lib().oracle_gather_mm(_p(x), _p(w), _p(lb), E, N, K, _p(lhs), _p(rhs), batch, M, _p(out))
    if rc != 0:
        raise ValueError(f"oracle_gather_mm rc={rc}")
    return out


def add_rms_norm(a, b, w, eps):
    """-> (sum_out, normed) bf16 [T, H]."""
    a, b, w = _c(a, np.uint16), _c(b, np.uint16), _c(w, np.uint16)
    T, H = a.shape
    s, n = np.empty_like(a), np.empty_like(a)
    lib().oracle_add_rms_norm(_p(a), _p(b), _p(w), float(eps), T, H, _p(s), _p(n))
    return s, n


def swiglu(g, u) -> np.ndarray:
    g, u = _c(g, np.uint16), _c(u, np.uint16)
    h = np.empty_like(g)
    lib().oracle_swiglu(_p(g), _p(u), g.size, _p(h))
    return h


def gptoss_swiglu(x_linear, x_glu):
    """-> (h bf16, h fp32) of GPT-OSS's swiglu(x_linear, x_glu) (gptoss.cpp:50-58)."""
    a, b = _c(x_linear, np.uint16), _c(x_glu, np.uint16)
    h = np.empty_like(a)
    hf = np.empty(a.shape, np.float32)
    lib().oracle_gptoss_swiglu(_p(a), _p(b), a.size, _p(h), _p(hf))
    return h, hf


def combine(Y, scores) -> np.ndarray:
    scores = _c(scores, np.float32)
    T, k = scores.shape
    Y = _c(Y, np.uint16)
    H = Y.shape[-1]
    y = np.empty((T, H), np.uint16)
    lib().oracle_combine(_p(Y), _p(scores), T, k, H, _p(y))
    return y


def block(layer, keep: list, hidden_f32: bool = False) -> OBlock:
    """OBlock view of a workloads.HostLayer.  hidden_f32: the routed experts' h and Y stay fp32
    (the reference's GPT-OSS promotion, see moe_oracle.h)."""
    cfg = layer.cfg
    b = OBlock()
    b.activation = getattr(cfg, "activation", ACT_SWIGLU)
    b.hidden_f32 = int(bool(hidden_f32))
    b.hidden, b.intermediate, b.num_experts = cfg.hidden, cfg.intermediate, cfg.num_experts
    b.router = make_router(cfg.variant, cfg.num_experts, cfg.top_k, cfg.norm_topk_prob, cfg.n_group,
                           cfg.topk_group, cfg.routed_scaling_factor)
    if layer.router_weight is not None:
        rw = _c(layer.router_weight, np.uint16)
        keep.append(rw)
        b.router_weight = rw.ctypes.data
    if layer.score_bias is not None:
        sb = _c(layer.score_bias, np.float32)
        keep.append(sb)
        b.score_bias = sb.ctypes.data
    b.gate, b.up, b.down = qweight(layer.gate, keep), qweight(layer.up, keep), qweight(layer.down, keep)
    b.shared_intermediate = 0
    if layer.shared is not None:
        sg, su, sd, sgw = layer.shared
        b.shared_intermediate = sg.N
        b.shared_gate, b.shared_up, b.shared_down = qweight(sg, keep), qweight(su, keep), qweight(sd, keep)
        if sgw is not None and not isinstance(sgw, np.ndarray):  # a quantized gate [1][1, H]
            b.shared_gate_q = qweight(sgw, keep)
        elif sgw is not None:
            a = _c(sgw, np.uint16)
            keep.append(a)
            b.shared_gate_weight = a.ctypes.data
    if getattr(layer, "router_q", None) is not None:
        b.router_q = qweight(layer.router_q, keep)
    if getattr(layer, "router_bias", None) is not None:
        rb = _c(layer.router_bias, np.uint16)
        keep.append(rb)
        b.router_bias = rb.ctypes.data
    return b


def moe_experts(layer, x, inds, scores, with_terms: bool = False, hidden_f32: bool = False):
    """-> out bf16 [T,H] (and, with_terms, the f32 [T,H] magnitude of the summed terms)."""
    keep = []
    b = block(layer, keep, hidden_f32)
    x = _c(x, np.uint16)
    inds, scores = _c(inds, np.uint32), _c(scores, np.float32)
    out = np.empty_like(x)
    terms = np.empty(x.shape, np.float32) if with_terms else None
    rc = lib().oracle_moe_experts(ctypes.byref(b), _p(x), x.shape[0], _p(inds), _p(scores), _p(out),
                                  _p(terms))
    if rc != 0:
        raise ValueError(f"oracle_moe_experts rc={rc}")
    return (out, terms) if with_terms else out


def block_forward(layer, x, hidden_f32: bool = False):
    """-> (out bf16 [T,H], logits bf16 [T,E], inds u32 [T,k], scores f32 [T,k])."""
    keep = []
    b = block(layer, keep, hidden_f32)
    x = _c(x, np.uint16)
    T = x.shape[0]
    E, k = layer.cfg.num_experts, layer.cfg.top_k
    out = np.empty_like(x)
    logits = np.empty((T, E), np.uint16)
    inds = np.empty((T, k), np.uint32)
    scores = np.empty((T, k), np.float32)
    rc = lib().oracle_block_forward(ctypes.byref(b), _p(x), T, _p(out), _p(logits), _p(inds), _p(scores))
    if rc != 0:
        raise ValueError(f"oracle_block_forward rc={rc}")
    return out, logits, inds, scores


def bf16_to_f32(a) -> np.ndarray:
    return (np.asarray(a, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def f32_to_bf16(a) -> np.ndarray:
    """Round to nearest even."""
    u = np.ascontiguousarray(a, dtype=np.float32).view(np.uint32).astype(np.uint64)
    r = (u + 0x7FFF + ((u >> 16) & 1)) >> 16
    return r.astype(np.uint16)
