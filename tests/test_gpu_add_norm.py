"""moe_block_forward_add_norm: the decode layer's residual add + RMSNorm and the block in one call,
against moe_add_rms_norm followed by moe_block_forward on the same inputs -- the sum, the normed
block input, the block output and every routing / bucketing output bit for bit.  Up to 16 tokens
with a bf16 router the add + norm runs inside the router projection's launch (every workgroup
finds its rows' scales itself, with add_rms_norm's lane order); T = 64, prefill-sized T and a
quantized router take the launch of its own.  H = 7168 (a DeepSeek-V3-wide row, 14 chunks per
lane) runs on a small synthetic layer."""
import gc

import numpy as np
import pytest

from helpers import load_pkg

torch = pytest.importorskip("torch")
moe = load_pkg()
from lemon_mlx_engine_amd import workloads as W  # noqa: E402

pytestmark = pytest.mark.gpu
DEV = "cuda:0"
EPS = 1e-6

WIDE = W.MoeConfig("h7168_small", 61, 7168, 256, 16, 4, moe.ROUTE_TOPK_LOGITS, True, 4)
CASES = [("tiny", 1, None), ("tiny", 16, None),
         ("qwen3_30b_a3b", 1, None), ("qwen3_30b_a3b", 5, None), ("qwen3_30b_a3b", 16, None),
         ("qwen3_30b_a3b", 64, None), ("qwen3_30b_a3b", 600, None), ("qwen3_30b_a3b", 1, 8),
         ("qwen3_next_80b", 1, None), ("qwen3_next_80b", 8, None),
         ("h7168_small", 1, None), ("h7168_small", 12, None)]

_cache = {}


def _block(name, router_bits):
    key = (name, router_bits)
    if key not in _cache:
        _cache.clear()
        gc.collect()
        torch.cuda.empty_cache()
        cfg = WIDE if name == WIDE.name else W.CONFIGS[name]
        _cache[key] = moe.MoeBlock.from_host(W.make_layer(cfg, router_bits=router_bits), DEV)
    return _cache[key]


def _bf(seed, n, std, mean=0.0):
    v = W.normal_bf16(seed, 7, n, std, mean=mean)
    return torch.from_numpy(v.view(np.int16)).to(DEV).view(torch.bfloat16)


def _same(a, b):
    if a.dtype == torch.float32:
        return torch.equal(a.view(torch.int32), b.view(torch.int32))
    if a.dtype == torch.bfloat16:
        return torch.equal(a.view(torch.int16), b.view(torch.int16))
    return torch.equal(a, b)


@pytest.mark.timeout(300)
@pytest.mark.parametrize("name,T,router_bits", CASES, ids=[f"{n}-T{t}{'-q' if q else ''}" for n, t, q in CASES])
def test_add_norm_matches_sequence(name, T, router_bits):
    blk = _block(name, router_bits)
    H = blk.hidden
    print(f"add_norm {name} T={T} router_bits={router_bits}", flush=True)
    a = _bf(300 + T, T * H, 1.0).reshape(T, H)
    b = _bf(400 + T, T * H, 0.5).reshape(T, H)
    w = _bf(500, H, 0.1, mean=1.0)
    s_ref, n_ref = moe.add_rms_norm(a, b, w, EPS)
    out_ref, aux_ref = blk.forward(n_ref, return_aux=True)
    s, n, out, aux = blk.forward_add_norm(a, b, w, EPS, return_aux=True)
    torch.cuda.synchronize()
    assert _same(s, s_ref), f"{name} T={T}: sum differs"
    assert _same(n, n_ref), f"{name} T={T}: normed input differs"
    assert _same(out, out_ref), f"{name} T={T}: block output differs"
    for key in aux_ref:
        assert _same(aux[key], aux_ref[key]), f"{name} T={T}: {key} differs"


def test_add_norm_validation():
    """Null inputs and a negative eps are refused before any launch."""
    blk = _block("tiny", None)
    L = moe.lib()
    x = torch.zeros((4, blk.hidden), dtype=torch.bfloat16, device=DEV)
    w = torch.ones(blk.hidden, dtype=torch.bfloat16, device=DEV)
    ws = blk.workspace(4)
    p = x.data_ptr()
    args = [p, p, w.data_ptr(), 1e-6, 4, p, p, p, None, ws.data_ptr(), ws.numel(), None]
    import ctypes
    for i in (0, 1, 2, 5, 6):
        bad = list(args)
        bad[i] = None
        assert L.moe_block_forward_add_norm(ctypes.byref(blk.desc), *bad) == moe.MOE_E_INVALID_ARG
    bad = list(args)
    bad[3] = -1.0
    assert L.moe_block_forward_add_norm(ctypes.byref(blk.desc), *bad) == moe.MOE_E_INVALID_ARG
    bad = list(args)
    bad[10] = 16
    assert L.moe_block_forward_add_norm(ctypes.byref(blk.desc), *bad) == moe.MOE_E_WORKSPACE
