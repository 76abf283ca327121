"""Whole-block parity (router -> top-k -> bucketing -> gate|up + SwiGLU -> down
-> combine, + shared expert) on the five benchmark configurations, against the
CPU checker on the same seeded inputs.

* routing: the HIP top-k indices and weights equal the checker's top-k on the
  HIP logits bit for bit; the HIP logits agree with the checker's within the
  fp32-accumulation bound (helpers.logits_bound); where a token's logits are
  identical, its indices are identical.
* bucketing: perm / inv_perm / offsets equal the checker's bit for bit.
* output: within |a-b| <= 2e-2 + 1e-2*|b| of the checker run on the HIP
  routing on all but 1e-4 of the elements, and every element within that bound
  plus one bf16 ulp of the bf16-rounded terms it sums (helpers.assert_close_block);
  on all tokens (small T) or a sample of tokens (large T, where the checker
  would take minutes); per-token outputs depend on that token only.
* full size: offsets[E] = T*k, perm is a permutation, and a second run is
  bit-identical (the combine uses no atomics).
"""
import gc

import numpy as np
import pytest

from helpers import assert_close, assert_close_block, assert_logits_close, load_pkg
from oracle import moe_oracle as O

torch = pytest.importorskip("torch")
moe = load_pkg()
from lemon_mlx_engine_amd import workloads as W  # noqa: E402

pytestmark = pytest.mark.gpu
DEV = "cuda:0"
SAMPLE = 48

CASES = [("tiny", 16), ("tiny", 1),
         ("qwen3_30b_a3b", 1), ("qwen3_30b_a3b", 8), ("qwen3_30b_a3b", 64), ("qwen3_30b_a3b", 8192),
         ("qwen3_next_80b", 1), ("qwen3_next_80b", 32), ("qwen3_next_80b", 4096),
         ("mixtral_8x7b", 1), ("mixtral_8x7b", 16), ("mixtral_8x7b", 8192),
         ("deepseek_v3", 1), ("deepseek_v3", 64), ("deepseek_v3", 4096)]

_cache = {}


def get_layer(name):
    if name not in _cache:
        _cache.clear()
        gc.collect()
        torch.cuda.empty_cache()
        host = W.make_layer(W.CONFIGS[name])
        _cache[name] = (host, moe.MoeBlock.from_host(host, DEV))
    return _cache[name]


def hbf(t):
    return t.view(torch.int16).cpu().numpy().view(np.uint16)


QR_CASES = [("tiny", 16), ("qwen3_30b_a3b", 1), ("qwen3_30b_a3b", 64), ("qwen3_next_80b", 32)]


@pytest.mark.timeout(600)
@pytest.mark.parametrize("name,T", QR_CASES, ids=[f"{n}-T{t}" for n, t in QR_CASES])
def test_block_quantized_router(name, T):
    """8-bit router weight (moe_block_desc.router_q): logits against the oracle's quantized matmul
    (one expert), routing and bucketing bit-exact on the device logits, outputs against the oracle."""
    _cache.clear()
    gc.collect()
    torch.cuda.empty_cache()
    cfg = W.CONFIGS[name]
    host = W.make_layer(cfg, router_bits=8)
    blk = moe.MoeBlock.from_host(host, DEV)
    E, k = cfg.num_experts, cfg.top_k
    x = W.make_tokens(cfg, T)
    xd = torch.from_numpy(x.view(np.int16)).to(DEV).view(torch.bfloat16)
    out, aux = blk.forward(xd, return_aux=True)
    torch.cuda.synchronize()
    logits = hbf(aux["logits"])
    inds = aux["inds"].cpu().numpy().astype(np.uint32)
    scores = aux["scores"].cpu().numpy()
    rlog = O.gather_qmm(x.reshape(T, 1, -1), host.router_q, None, np.zeros(T, np.uint32), 1).reshape(T, E)
    assert_close(logits, rlog, what="quantized router logits")
    params = O.make_router(cfg.variant, E, k, cfg.norm_topk_prob, cfg.n_group, cfg.topk_group,
                           cfg.routed_scaling_factor)
    ri, rs, _ = O.route(logits, params, host.score_bias)
    np.testing.assert_array_equal(inds, ri)
    np.testing.assert_array_equal(scores.view(np.uint32), rs.view(np.uint32))
    rp, rinv, _, ro = O.bucket(inds, E)
    np.testing.assert_array_equal(aux["offsets"].cpu().numpy(), ro)
    np.testing.assert_array_equal(aux["perm"].cpu().numpy(), rp)
    ref, terms = O.moe_experts(host, x, inds, scores, with_terms=True)
    assert_close_block(hbf(out), ref, terms, what=f"{name} T={T} (8-bit router)")
    del blk


@pytest.mark.timeout(600)
@pytest.mark.parametrize("name,T", CASES, ids=[f"{n}-T{t}" for n, t in CASES])
def test_block(name, T):
    host, blk = get_layer(name)
    cfg = host.cfg
    E, k = cfg.num_experts, cfg.top_k
    x = W.make_tokens(cfg, T)
    xd = torch.from_numpy(x.view(np.int16)).to(DEV).view(torch.bfloat16)
    out, aux = blk.forward(xd, return_aux=True)
    out2 = blk.forward(xd)
    torch.cuda.synchronize()
    out_h = hbf(out)
    assert (out_h == hbf(out2)).all(), "second run differs"

    logits = hbf(aux["logits"])
    inds = aux["inds"].cpu().numpy().astype(np.uint32)
    scores = aux["scores"].cpu().numpy()
    perm = aux["perm"].cpu().numpy()
    inv = aux["inv_perm"].cpu().numpy()
    offs = aux["offsets"].cpu().numpy()

    # routing on identical logits: bit-exact
    ri, rs, _ = O.route(logits, O.make_router(cfg.variant, E, k, cfg.norm_topk_prob, cfg.n_group,
                                              cfg.topk_group, cfg.routed_scaling_factor), host.score_bias)
    np.testing.assert_array_equal(inds, ri)
    np.testing.assert_array_equal(scores.view(np.uint32), rs.view(np.uint32))

    # bucketing: bit-exact, and the full-size invariants
    rp, rinv, _, ro = O.bucket(inds, E)
    np.testing.assert_array_equal(offs, ro)
    np.testing.assert_array_equal(perm, rp)
    np.testing.assert_array_equal(inv, rinv)
    assert offs[-1] == T * k and (np.sort(perm) == np.arange(T * k)).all()

    # sampled tokens: logits within one ulp, end-to-end routing, outputs
    S = np.arange(T) if T <= SAMPLE else np.unique(np.linspace(0, T - 1, SAMPLE).astype(np.int64))
    rlog = O.router_logits(x[S], host.router_weight)
    assert_logits_close(logits[S], rlog, x[S], host.router_weight)
    same = (rlog == logits[S]).all(1)
    if same.any():
        oi, _, _ = O.route(rlog[same], O.make_router(cfg.variant, E, k, cfg.norm_topk_prob, cfg.n_group,
                                                     cfg.topk_group, cfg.routed_scaling_factor),
                           host.score_bias)
        np.testing.assert_array_equal(oi, inds[S][same])
    ref, terms = O.moe_experts(host, x[S], inds[S], scores[S], with_terms=True)
    err, nbad = assert_close_block(out_h[S], ref, terms, what=f"{name} T={T}")
    print(f"{name} T={T}: max abs err {err:.3g}; {nbad} elements outside the strict tolerance; "
          f"logits differ in {(~same).sum()} of {len(S)} rows")


def test_block_from_checkpoint(tmp_path):
    """A checkpoint directory (MLX safetensors, 8-bit router by a per-prefix override) read by
    checkpoint.load_moe_layer runs through the device block bit-identically to the layer it holds."""
    import json
    from test_checkpoint import config_json, layer_tensors, write_safetensors
    from lemon_mlx_engine_amd import checkpoint as C

    cfg = W.CONFIGS["tiny"]
    layer = W.make_layer(cfg, router_bits=8)
    write_safetensors(tmp_path / "model.safetensors", layer_tensors(0, layer))
    q8 = {"model.layers.0.mlp.gate": {"group_size": 64, "bits": 8}}
    (tmp_path / "config.json").write_text(json.dumps(config_json(cfg, "qwen3_moe", q8)))
    got = C.load_moe_layer(str(tmp_path), 0)
    x = torch.from_numpy(W.make_tokens(cfg, 16).view(np.int16)).to(DEV).view(torch.bfloat16)
    a = moe.MoeBlock.from_host(layer, DEV).forward(x)
    b = moe.MoeBlock.from_host(got, DEV).forward(x)
    torch.cuda.synchronize()
    assert (hbf(a) == hbf(b)).all()


@pytest.mark.parametrize("name,T", [("qwen3_30b_a3b", 1), ("qwen3_30b_a3b", 8), ("tiny", 16)])
def test_block_graph_replays(name, T):
    """moe_block_graph: the captured block replayed over new token rows written in place, with eager
    forwards and synchronisations between the replays; every replay equals the eager result."""
    host, blk = get_layer(name)
    cfg = host.cfg
    x = torch.empty((T, cfg.hidden), dtype=torch.bfloat16, device=DEV)
    out = torch.empty_like(x)
    g = blk.graph(x, out)
    for i in range(4):
        xi = W.normal_bf16(100 + i, 100, T * cfg.hidden, 1.0).reshape(T, cfg.hidden)
        xd = torch.from_numpy(xi.view(np.int16)).to(DEV).view(torch.bfloat16)
        x.copy_(xd)
        g.launch()
        torch.cuda.synchronize()
        got = hbf(out).copy()
        ref = hbf(blk.forward(xd))
        torch.cuda.synchronize()
        assert (got == ref).all(), f"replay {i} differs from the eager forward"
    del g
