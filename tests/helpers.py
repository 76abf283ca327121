"""Shared test helpers: package loader and numeric comparisons."""
import importlib.util
import sys
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[1]
PKG_DIR = ROOT / "lemon-mlx-engine_amd"

# Output tolerance of the benchmark definition: max-abs 2e-2 / rel 1e-2 (bf16
# outputs, fp32 accumulation), applied elementwise as |a - b| <= ATOL + RTOL*|b|.
ATOL = 2e-2
RTOL = 1e-2


def load_pkg():
    """Import lemon-mlx-engine_amd/ as the package `lemon_mlx_engine_amd`."""
    name = "lemon_mlx_engine_amd"
    if name in sys.modules:
        return sys.modules[name]
    spec = importlib.util.spec_from_file_location(name, PKG_DIR / "__init__.py",
                                                  submodule_search_locations=[str(PKG_DIR)])
    mod = importlib.util.module_from_spec(spec)
    sys.modules[name] = mod
    spec.loader.exec_module(mod)
    return mod


def bf16(a):
    return (np.asarray(a, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def to_bf16(a):
    u = np.ascontiguousarray(a, dtype=np.float32).view(np.uint32).astype(np.uint64)
    return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)


def assert_close(got_bf16, ref_bf16, atol=ATOL, rtol=RTOL, what="output"):
    g = bf16(got_bf16).astype(np.float64)
    r = bf16(ref_bf16).astype(np.float64)
    assert g.shape == r.shape, (g.shape, r.shape)
    err = np.abs(g - r)
    bad = err > atol + rtol * np.abs(r)
    assert not bad.any(), (f"{what}: {bad.sum()} of {bad.size} outside tolerance; max abs err "
                           f"{err.max():.4g} at {np.unravel_index(err.argmax(), err.shape)}")
    return float(err.max())


def logits_bound(x_bf16, w_bf16, bias_bf16=None):
    """Allowed |a - b| between two bf16 roundings of fp32 dot products (plus a
    bias, added before the rounding) summed in different orders: one bf16 ulp of
    the result plus 8*sqrt(K)*2^-24 times the sum of |products| (fp32
    accumulation noise; matters where terms cancel)."""
    xf = bf16(x_bf16).astype(np.float64)
    wf = bf16(w_bf16).astype(np.float64)
    exact = xf @ wf.T
    mag = np.abs(xf) @ np.abs(wf).T
    if bias_bf16 is not None:
        b = bf16(bias_bf16).astype(np.float64)
        exact = exact + b
        mag = mag + np.abs(b)
    K = xf.shape[1]
    ulp = np.spacing(np.abs(exact).astype(np.float32)).astype(np.float64) * 65536.0
    return exact, ulp + 8.0 * np.sqrt(K) * 2.0**-24 * mag


def assert_logits_close(got_bf16, ref_bf16, x_bf16, w_bf16, bias_bf16=None):
    _, bound = logits_bound(x_bf16, w_bf16, bias_bf16)
    d = np.abs(bf16(got_bf16).astype(np.float64) - bf16(ref_bf16).astype(np.float64))
    assert (d <= bound).all(), f"logits differ by {d.max():.3g} (bound {bound[d.argmax() // d.shape[1]].min():.3g})"
    return int((d > 0).sum())


def assert_close_block(got_bf16, ref_bf16, term_mag, what="block output", strict_frac=1e-4, extra=None):
    """Block outputs: the benchmark tolerance |a-b| <= ATOL + RTOL*|b| must hold
    on all but a fraction `strict_frac` of elements, and every element must lie
    within that bound plus one bf16 ulp (2^-8 relative) of the magnitude of the
    bf16-rounded terms the output sums (expert outputs Y times their weights,
    the shared-expert output).  The reference rounds those intermediates to
    bf16 (each op's output dtype), so two correct implementations whose fp32
    sums straddle a rounding boundary differ by up to one such ulp; where the
    terms cancel, that exceeds the bound taken relative to the output.
    extra (optional, per element): a further allowance for rounding points
    inside the expert MLP (h_rounding_mag)."""
    g = bf16(got_bf16).astype(np.float64)
    r = bf16(ref_bf16).astype(np.float64)
    err = np.abs(g - r)
    strict = err <= ATOL + RTOL * np.abs(r)
    nbad = int((~strict).sum())
    bound = ATOL + RTOL * np.abs(r) + 2.0**-8 * np.asarray(term_mag, np.float64)
    if extra is not None:
        bound = bound + np.asarray(extra, np.float64)
    loose = err <= bound
    assert loose.all(), f"{what}: {int((~loose).sum())} elements outside the rounding-aware bound"
    assert nbad <= strict_frac * err.size, (f"{what}: {nbad} of {err.size} outside the strict tolerance "
                                            "(all within the rounding-aware bound)")
    return float(err.max()), nbad


def h_rounding_mag(O, layer, x_bf16, inds, scores):
    """How far the bf16 rounding points inside an expert MLP can move a block output, to first order:
    D[t, c] = sum_j |s_tj| sum_i |W_down[e_tj][c, i]| dh_tji with
        dh = |dh/dg| 2^-7 |g| + |dh/du| 2^-7 |u| + 2^-7 |h|,
    one bf16 ulp (at most 2^-7 relative) of the rounded gate, up and h values, carried through the
    activation's derivatives and the down projection.  Two correct fp32 summation orders can round g or
    u to neighbouring bf16 values; with GPT-OSS's clipped SwiGLU at |g|, |u| of a few units one such
    ulp moves h by up to 7 ulp(g).  Rounding h (GPT-OSS, relu^2: the reference keeps h in fp32, its
    scalar operands promoting it) is the last term.  g, u, h from fp64 gate/up products with the
    layer's biases and activation (cfg.activation); derivatives of the unclipped branch (an upper
    bound at the limits)."""
    cfg = layer.cfg
    xf = bf16(x_bf16).astype(np.float64)
    T, k = inds.shape
    D = np.zeros((T, cfg.hidden))
    cache = {}

    def deq(q, e):
        if (id(q), e) not in cache:
            cache[(id(q), e)] = O.dequant(q.w[e], q.scales[e], q.biases[e], q.N, q.K, q.group_size,
                                          q.bits).astype(np.float64)
        return cache[(id(q), e)]

    def lb(q, e):
        return 0.0 if q.linear_bias is None else bf16(q.linear_bias[e]).astype(np.float64)

    for e in np.unique(inds):
        rows = np.argwhere(inds == e)
        xe = xf[rows[:, 0]]
        g = xe @ deq(layer.gate, e).T + lb(layer.gate, e)
        u = xe @ deq(layer.up, e).T + lb(layer.up, e)
        act = getattr(cfg, "activation", 0)
        if act == 0:
            sg = 1.0 / (1.0 + np.exp(-g))
            h = g * sg * u
            dg, du = sg * (1.0 + g * (1.0 - sg)) * u, g * sg
        else:
            lin, glu = (g, u) if act == 1 else (u, g)
            xl, xg = np.clip(lin, -7.0, 7.0), np.minimum(glu, 7.0)
            s = 1.0 / (1.0 + np.exp(-1.702 * xg))
            h = xg * s * (xl + 1.0)
            d_lin, d_glu = xg * s, (s + 1.702 * xg * s * (1.0 - s)) * (xl + 1.0)
            dg, du = (d_lin, d_glu) if act == 1 else (d_glu, d_lin)
        dh = 2.0**-7 * (np.abs(dg) * np.abs(g) + np.abs(du) * np.abs(u) + np.abs(h))
        mag = dh @ np.abs(deq(layer.down, e)).T
        np.add.at(D, rows[:, 0], np.abs(scores[rows[:, 0], rows[:, 1]])[:, None] * mag)
    return D


def record_parity(key, fields):
    """Merge {key: fields} into parity_block.json in the run's output directory (per-config parity
    counts of a GPU run, returned with the run's other outputs)."""
    import json
    import os
    out = ROOT / "gpurun_out"
    out.mkdir(exist_ok=True)
    path = out / "parity_block.json"
    data = {}
    if path.exists():
        try:
            data = json.loads(path.read_text())
        except ValueError:
            data = {}
    data[key] = fields
    tmp = path.with_suffix(".tmp")
    tmp.write_text(json.dumps(data, indent=1, sort_keys=True))
    os.replace(tmp, path)


def _ranks(inds, E):
    """rank[t, e] = slot of expert e in row t, k where not selected."""
    T, k = inds.shape
    r = np.full((T, E), k, np.int64)
    r[np.arange(T)[:, None], inds.astype(np.int64)] = np.arange(k)[None, :]
    return r


def routing_near_ties(O, cfg, x, router_w, logits_gpu, inds_gpu, bias=None, router_bias=None):
    """End-to-end routing from x: the checker's routing on its own logits (O.router_logits, then
    O.route) against the device's routing.  A token may differ only where the device's logits differ
    from the checker's (two fp32 summation orders rounded to bf16) and every pair of experts whose
    order flips is a near tie: their selection values (in the variant's own units) lie within the sum
    of their perturbation bounds, each derived from logits_bound (the rounding-order bound of the
    logits) through the selection function (plus the bf16 rounding width where the selection value is
    a bf16 probability / sigmoid).  For group-limited routing a flip of the kept groups must be a near
    tie of the group scores in the same sense.  Returns (tokens whose routing differs, flipped pairs);
    raises on any flip that is not a near tie."""
    E, k = cfg.num_experts, cfg.top_k
    params = O.make_router(cfg.variant, E, k, cfg.norm_topk_prob, cfg.n_group, cfg.topk_group,
                           cfg.routed_scaling_factor)
    lo = O.router_logits(x, router_w, router_bias)
    io, _, _ = O.route(lo, params, bias)
    ig = np.asarray(inds_gpu, np.uint32)
    diff = (io != ig).any(1)
    if not diff.any():
        return 0, 0
    rows = np.nonzero(diff)[0]
    same_logits = (lo[rows] == np.asarray(logits_gpu)[rows]).all(1)
    assert not same_logits.any(), f"routing differs on tokens {rows[same_logits][:8]} with identical logits"
    _, bound = logits_bound(x[rows], router_w, router_bias)
    l = bf16(lo[rows]).astype(np.float64)
    V = cfg.variant
    grouped = V in (O.R_SIGMOID_GROUP, O.R_SIGMOID_GROUP_DROP_BEST)
    if V in (O.R_SIGMOID_GROUP, O.R_SIGMOID_GROUP_DROP_BEST, O.R_SIGMOID_CORRECTED, O.R_GLM4_SIGMOID):
        # unmasked corrected scores sigma(l) + bias, as the checker computes them (no group limit)
        p1 = O.make_router(V, E, k, cfg.norm_topk_prob, 1, 1, cfg.routed_scaling_factor)
        _, _, sv = O.route(lo[rows], p1, bias)
        sv = sv.astype(np.float64)
        sg = 1.0 / (1.0 + np.exp(-l))
        pb = sg * (1.0 - sg) * bound + 2.0**-21
    elif V in (O.R_GLM4_SOFTMAX, O.R_LFM2):
        # fp32 probabilities + bias: a logit move of d_i changes p_i by p_i (d_i - sum_j p_j d_j)
        p1 = O.make_router(V, E, k, cfg.norm_topk_prob, 1, 1, cfg.routed_scaling_factor)
        _, _, sv = O.route(lo[rows], p1, bias)
        sv = sv.astype(np.float64)
        pr = np.exp(l - l.max(1, keepdims=True))
        pr /= pr.sum(1, keepdims=True)
        pb = pr * (bound + bound.max(1, keepdims=True)) + 2.0**-21
    elif V == O.R_SIGMOID:
        sv = l
        sg = 1.0 / (1.0 + np.exp(-l))
        pb = bound + 2.0**-7 / np.maximum(1.0 - sg, 2.0**-7)
    elif V == O.R_TOPK_PROBS:
        sv, pb = l, bound + 2.0**-7  # bf16 probabilities: equal within a relative 2^-7 of p
    else:
        sv, pb = l, bound
    ro, rg = _ranks(io[rows], E), _ranks(ig[rows], E)
    excused = np.zeros((len(rows), E), bool)
    if grouped and cfg.n_group > 1:
        G, gsz = cfg.n_group, E // cfg.n_group
        sgrp = sv.reshape(len(rows), G, gsz)
        top2 = np.sort(sgrp, axis=2)[:, :, -2:].sum(2)
        pbg = np.sort(pb.reshape(len(rows), G, gsz), axis=2)[:, :, -2:].sum(2)
        for r in range(len(rows)):
            # the checker's kept groups in the canonical group order (value desc, index asc): the
            # topk_group best, or (as nemotron_h.cpp:425-447 writes it) all but the best G - topk_group
            order = sorted(range(G), key=lambda g: (-top2[r, g], g))
            kept_o = set(order[:cfg.topk_group] if V == O.R_SIGMOID_GROUP else order[G - cfg.topk_group:])
            used_g = set(np.unique(ig[rows[r]] // gsz).tolist())  # groups the device routed into
            used_o = set(np.unique(io[rows[r]] // gsz).tolist())
            assert len(used_g) <= cfg.topk_group, f"token {rows[r]}: routed into {len(used_g)} groups"

            def near(ga, gb):
                return abs(top2[r, ga] - top2[r, gb]) <= pbg[r, ga] + pbg[r, gb]
            # a group the checker drops but the device routes into must near-tie a kept group the
            # device does not use (the device kept it instead)
            for ga in used_g - kept_o:
                ok = [gb for gb in kept_o - used_g if near(ga, gb)]
                assert ok, (f"token {rows[r]}: routed into group {ga} (group score {top2[r, ga]:.6g}), "
                            f"not a near tie of any kept group the device dropped")
                for g in (ga, ok[0]):
                    excused[r, g * gsz:(g + 1) * gsz] = True
            # a kept group the checker routes into and the device does not may have been dropped by
            # the device for a near-tied group outside the checker's kept set
            for gb in used_o - used_g:
                ok = [ga for ga in set(range(G)) - kept_o if near(ga, gb)]
                if ok:
                    for g in (gb, ok[0]):
                        excused[r, g * gsz:(g + 1) * gsz] = True
    flips = 0
    for r in range(len(rows)):
        cand = np.nonzero((ro[r] < k) | (rg[r] < k))[0]
        for i, a in enumerate(cand):
            for b in cand[i + 1:]:
                if (ro[r, a] - ro[r, b]) * (rg[r, a] - rg[r, b]) >= 0 or (ro[r, a] == k and ro[r, b] == k):
                    continue
                if excused[r, a] or excused[r, b]:
                    continue
                flips += 1
                gap = abs(sv[r, a] - sv[r, b])
                assert gap <= pb[r, a] + pb[r, b], (
                    f"token {rows[r]}: experts {a}/{b} swap with selection gap {gap:.3g} "
                    f"> {pb[r, a] + pb[r, b]:.3g}")
    return len(rows), flips


def tile_sample(perm, offsets, k, T, n=1024, tile=128):
    """Tokens covering the first and last row of every token tile of the large-bucket GEMM (128 rows,
    then the one remainder tile of 32, 64, 96 or 128 rows of each expert's bucket), the first and last token of every
    128-token block (the one-expert shared-expert GEMM over the T rows), and evenly spaced tokens up to
    at least n."""
    pos = []
    offs = np.asarray(offsets, np.int64)
    for e in range(len(offs) - 1):
        a, b = offs[e], offs[e + 1]
        c = b - a
        if c == 0:
            continue
        starts = list(range(0, (c // tile) * tile, tile))
        rem = c % tile
        for s in starts:
            pos += [a + s, a + s + tile - 1]
        if rem:
            r0 = a + (c // tile) * tile
            pos += [r0, r0 + min(rem, 64) - 1, b - 1]  # the remainder tile (and its middle)
    toks = set((np.asarray(perm, np.int64)[np.asarray(pos, np.int64)] // k).tolist())
    for s in range(0, T, tile):
        toks.update((s, min(s + tile, T) - 1))
    if len(toks) < n:  # fill with evenly spaced tokens, then a fixed shuffle, until n are chosen
        for t in np.concatenate([np.linspace(0, T - 1, n).astype(np.int64),
                                 np.random.default_rng(0).permutation(T)]):
            if len(toks) >= min(n, T):
                break
            toks.add(int(t))
    return np.array(sorted(toks), np.int64)
