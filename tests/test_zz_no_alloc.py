"""moe_block_forward_noalloc: the block with its workspace in the library's static
device scratch, called through the C ABI, against moe_block_forward with a caller
workspace (same kernels, so bit-identical outputs and routing), two calls in a row
with the second smaller; a T beyond the scratch is refused before any launch."""
import ctypes
import gc

import numpy as np
import pytest

from helpers import load_pkg

torch = pytest.importorskip("torch")
moe = load_pkg()
from lemon_mlx_engine_amd import workloads as W  # noqa: E402

pytestmark = pytest.mark.gpu
DEV = "cuda:0"
NOALLOC_BYTES = 64 << 20


def _p(t):
    return ctypes.c_void_p(0 if t is None else t.data_ptr())


def _stream():
    return ctypes.c_void_p(torch.cuda.current_stream(torch.device(DEV)).cuda_stream)


def _aux(blk, T):
    k, E = blk.router.top_k, blk.num_experts
    t = dict(logits=torch.full((T, E), -1, dtype=torch.int16, device=DEV),
             inds=torch.full((T, k), -1, dtype=torch.int32, device=DEV),
             scores=torch.full((T, k), -1, dtype=torch.float32, device=DEV),
             perm=torch.full((T * k,), -1, dtype=torch.int32, device=DEV),
             inv_perm=torch.full((T * k,), -1, dtype=torch.int32, device=DEV),
             offsets=torch.full((E + 1,), -1, dtype=torch.int32, device=DEV))
    c = moe.BlockAux(*(t[n].data_ptr() for n in ("logits", "inds", "scores", "perm", "inv_perm", "offsets")))
    return t, c


def _run(blk, x, noalloc):
    T = x.shape[0]
    out = torch.full_like(x, float("nan"))
    aux, auxc = _aux(blk, T)
    L = moe.lib()
    if noalloc:
        st = L.moe_block_forward_noalloc(ctypes.byref(blk.desc), _p(x), T, _p(out), ctypes.byref(auxc), _stream())
    else:
        n = L.moe_block_workspace_size(ctypes.byref(blk.desc), T)
        ws = torch.empty(n, dtype=torch.uint8, device=DEV)
        st = L.moe_block_forward(ctypes.byref(blk.desc), _p(x), T, _p(out), ctypes.byref(auxc), _p(ws), n,
                                 _stream())
    assert st == moe.MOE_OK, (st, L.moe_last_error())
    torch.cuda.synchronize()
    return out, aux


def _tokens(cfg, T, seed):
    x = W.normal_bf16(200 + seed, 100, T * cfg.hidden, 1.0).reshape(T, cfg.hidden)
    return torch.from_numpy(x.view(np.int16)).to(DEV).view(torch.bfloat16)


@pytest.mark.timeout(300)
@pytest.mark.parametrize("name,T1,T2", [("tiny", 16, 5), ("qwen3_30b_a3b", 64, 8), ("qwen3_next_80b", 32, 1),
                                        ("deepseek_v3", 64, 1)])
def test_noalloc_matches_workspace_entry(name, T1, T2):
    gc.collect()
    torch.cuda.empty_cache()
    cfg = W.CONFIGS[name]
    blk = moe.MoeBlock.from_host(W.make_layer(cfg), DEV)
    for i, T in enumerate((T1, T2)):  # the second call is smaller and finds the first one's scratch contents
        print(f"noalloc {name} T={T}", flush=True)
        x = _tokens(cfg, T, i)
        ref, ra = _run(blk, x, noalloc=False)
        got, ga = _run(blk, x, noalloc=True)
        assert torch.equal(got.view(torch.int16), ref.view(torch.int16)), f"{name} T={T}: outputs differ"
        for key in ra:  # bit patterns (scores are fp32)
            a, b = ga[key], ra[key]
            if a.dtype == torch.float32:
                a, b = a.view(torch.int32), b.view(torch.int32)
            assert torch.equal(a, b), f"{name} T={T}: {key} differs"
    del blk


@pytest.mark.timeout(300)
@pytest.mark.parametrize("name,T", [("qwen3_30b_a3b", 8), ("qwen3_next_80b", 1)])
def test_noalloc_captured_replays(name, T):
    """After an eager call has resolved the scratch address, a call captured into a graph
    (torch.cuda.graph, thread-local capture) replays with new tokens written in place; every replay,
    with eager calls of both entry points and synchronisations between, equals moe_block_forward
    with a caller workspace bit for bit."""
    gc.collect()
    torch.cuda.empty_cache()
    cfg = W.CONFIGS[name]
    blk = moe.MoeBlock.from_host(W.make_layer(cfg), DEV)
    L = moe.lib()
    x = _tokens(cfg, T, 0)
    _run(blk, x, noalloc=True)  # eager: resolves the scratch address on this device
    out = torch.zeros_like(x)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, capture_error_mode="thread_local"):
        st = L.moe_block_forward_noalloc(ctypes.byref(blk.desc), _p(x), T, _p(out), None, _stream())
    assert st == moe.MOE_OK, (st, L.moe_last_error())
    for i in range(3):
        print(f"noalloc replay {name} T={T} #{i}", flush=True)
        xi = _tokens(cfg, T, 10 + i)
        x.copy_(xi)
        g.replay()
        torch.cuda.synchronize()
        got = out.clone()
        ref, _ = _run(blk, xi, noalloc=False)
        eager, _ = _run(blk, xi, noalloc=True)
        assert torch.equal(got.view(torch.int16), ref.view(torch.int16)), f"replay {i} differs"
        assert torch.equal(eager.view(torch.int16), ref.view(torch.int16)), f"eager call {i} differs"
    del g, blk


def test_noalloc_refuses_oversize():
    """A T whose workspace exceeds the static scratch returns MOE_E_WORKSPACE and leaves out untouched."""
    blk = moe.MoeBlock.from_host(W.make_layer(W.CONFIGS["tiny"]), DEV)
    L = moe.lib()
    T = 16384
    assert L.moe_block_workspace_size(ctypes.byref(blk.desc), T) > NOALLOC_BYTES
    x = _tokens(W.CONFIGS["tiny"], T, 0)
    out = torch.zeros_like(x)
    st = L.moe_block_forward_noalloc(ctypes.byref(blk.desc), _p(x), T, _p(out), None, _stream())
    torch.cuda.synchronize()
    assert st == moe.MOE_E_WORKSPACE
    assert b"static scratch" in L.moe_last_error()
    assert not out.view(torch.int16).any()
