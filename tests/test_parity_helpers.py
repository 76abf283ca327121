"""The parity helpers the GPU tests rely on, exercised on the CPU with the checker standing in for
the device: routing_near_ties accepts routings that come from logits moved within the rounding-order
bound (one bf16 ulp, as a different fp32 summation order gives) and rejects a planted swap of
far-apart experts; tile_sample covers every token tile."""
import numpy as np
import pytest

from helpers import bf16, routing_near_ties, tile_sample, to_bf16
from oracle import moe_oracle as O


class Cfg:
    def __init__(self, variant, E, k, norm=True, n_group=1, topk_group=1, rsf=1.0):
        self.variant, self.num_experts, self.top_k = variant, E, k
        self.norm_topk_prob, self.n_group, self.topk_group, self.routed_scaling_factor = norm, n_group, topk_group, rsf


def _inputs(E, H, T, seed):
    rng = np.random.default_rng(seed)
    x = to_bf16(rng.standard_normal((T, H)).astype(np.float32))
    w = to_bf16((0.02 * rng.standard_normal((E, H))).astype(np.float32))
    return x, w


def _nudge(logits, rng, frac=0.3):
    """Move a fraction of the logits by one bf16 ulp up or down (bit pattern +-1, same sign)."""
    l = logits.copy()
    m = rng.random(l.shape) < frac
    step = np.where(rng.random(l.shape) < 0.5, 1, -1).astype(np.int32)
    nz = (l & 0x7FFF) > 1
    l[m & nz] = (l[m & nz].astype(np.int32) + step[m & nz]).astype(np.uint16)
    return l


CASES = [(O.R_TOPK_LOGITS, 128, 8, 1, 1), (O.R_TOPK_PROBS, 512, 10, 1, 1), (O.R_SOFTMAX_TOPK, 8, 2, 1, 1),
         (O.R_SIGMOID_GROUP, 256, 8, 8, 4), (O.R_SIGMOID_GROUP_DROP_BEST, 256, 8, 8, 3),
         (O.R_SIGMOID_CORRECTED, 256, 8, 8, 4), (O.R_GLM4_SIGMOID, 128, 8, 8, 4), (O.R_GLM4_SOFTMAX, 128, 8, 1, 1),
         (O.R_LFM2, 64, 4, 1, 1)]


@pytest.mark.parametrize("variant,E,k,ng,tg", CASES)
def test_near_ties_accepted_and_far_swaps_rejected(variant, E, k, ng, tg):
    H, T = 256, 2048
    cfg = Cfg(variant, E, k, True, ng, tg, 2.5 if ng > 1 else 1.0)
    x, w = _inputs(E, H, T, variant)
    rng = np.random.default_rng(7)
    bias = (0.01 * rng.standard_normal(E)).astype(np.float32) if variant >= O.R_SIGMOID_GROUP else None
    params = O.make_router(variant, E, k, True, ng, tg, cfg.routed_scaling_factor)
    lo = O.router_logits(x, w)
    lg = _nudge(lo, rng)
    ig, _, _ = O.route(lg, params, bias)
    ntok, nflip = routing_near_ties(O, cfg, x, w, lg, ig, bias)
    assert ntok >= 1 and nflip >= 1, "the nudge should flip at least one near tie"
    # plant a swap: a token's last selected expert replaced by its least preferred unselected one
    io, _, sel = O.route(lo, params, bias)
    t = int(np.nonzero((lg == lo).all(1) == False)[0][0])  # noqa: E712  (a token whose logits differ)
    bad = ig.copy()
    unsel = np.setdiff1d(np.arange(E), io[t])
    if ng > 1 and variant in (O.R_SIGMOID_GROUP, O.R_SIGMOID_GROUP_DROP_BEST):  # the least preferred expert of a dropped group
        # (upstream rule: the worst group; as written: the best group, which it zeroes)
        _, _, sv = O.route(lo, O.make_router(O.R_SIGMOID_GROUP, E, k, True, 1, 1, 2.5), bias)
        gsz = E // ng
        gsc = np.sort(sv[t].reshape(ng, gsz), axis=1)[:, -2:].sum(1)
        worst = int(np.argmin(gsc) if variant == O.R_SIGMOID_GROUP else np.argmax(gsc))
        unsel = np.arange(worst * gsz, (worst + 1) * gsz)
        sel = sv
    bad[t, k - 1] = unsel[np.argmin(sel[t, unsel])]
    with pytest.raises(AssertionError, match="swap|groups"):
        routing_near_ties(O, cfg, x, w, lg, bad, bias)
    # identical logits must route identically
    bad2 = io.copy()
    s = int(np.nonzero((lg == lo).all(1))[0][0]) if (lg == lo).all(1).any() else None
    if s is not None:
        bad2[s, [0, 1]] = bad2[s, [1, 0]]
        with pytest.raises(AssertionError, match="identical logits"):
            routing_near_ties(O, cfg, x, w, lo, bad2, bias)


def test_tile_sample_covers_every_tile():
    rng = np.random.default_rng(3)
    T, k, E = 4096, 8, 256
    inds = np.stack([rng.choice(E, k, replace=False) for _ in range(T)]).astype(np.uint32)
    perm, _, _, offs = O.bucket(inds, E)
    S = set(tile_sample(perm, offs, k, T, 1024).tolist())
    assert len(S) >= 1024
    for e in range(E):
        a, b = offs[e], offs[e + 1]
        for r in range(a, b, 32):  # every 32-row unit's first row belongs to a tile whose ends are sampled
            t0 = a + ((r - a) // 128) * 128
            assert perm[t0] // k in S
        if b > a:
            assert perm[b - 1] // k in S
