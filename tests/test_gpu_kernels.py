"""Parity of each HIP entry point against the CPU checker, on seeded inputs.

Integer / index work (top-k indices, sort permutation, offsets) is compared
bit-exact; router weights are compared bit-exact on identical logits (both
sides evaluate the same canonical arithmetic); floating-point products are
compared with the benchmark tolerance |a-b| <= 2e-2 + 1e-2*|b| (helpers.ATOL /
RTOL), bf16 outputs with fp32 accumulation.
"""
import dataclasses

import numpy as np
import pytest

from helpers import assert_close, assert_logits_close, bf16, load_pkg, to_bf16
from oracle import moe_oracle as O

torch = pytest.importorskip("torch")
moe = load_pkg()
from lemon_mlx_engine_amd import workloads as W  # noqa: E402

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def dbf(a):
    return torch.from_numpy(np.ascontiguousarray(a, np.uint16).view(np.int16)).to(DEV).view(torch.bfloat16)


def di32(a):
    return torch.from_numpy(np.ascontiguousarray(a).astype(np.int32)).to(DEV)


def hbf(t):
    return t.view(torch.int16).cpu().numpy().view(np.uint16)


def host(t):
    return t.cpu().numpy()


def dqw(h):
    return moe.QuantizedWeight.from_numpy(h.w, h.scales, h.biases, h.group_size, h.bits, DEV,
                                          getattr(h, "linear_bias", None))


def distinct_inds(T, k, E, seed):
    rng = np.random.default_rng(seed)
    return np.stack([rng.choice(E, k, replace=False) for _ in range(T)]).astype(np.uint32)


# ------------------------------------------------------------------ router projection
@pytest.mark.parametrize("T,H,E", [(1, 2048, 128), (16, 512, 8), (64, 2048, 512), (333, 7168, 256),
                                   (2048, 2048, 128), (8192, 4096, 8), (1000, 7168, 1), (513, 512, 40),
                                   (4096, 2048, 512)])
def test_router_logits(T, H, E):
    x = W.normal_bf16(1, 100, T * H, 1.0).reshape(T, H)
    wg = W.normal_bf16(1, 1, E * H, 0.02).reshape(E, H)
    got = hbf(moe.router_logits(dbf(x), dbf(wg)))
    ref = O.router_logits(x, wg)
    # fp32 sums in a different order may round to a neighbouring bf16 value
    ndiff = assert_logits_close(got, ref, x, wg)
    assert ndiff / got.size < 0.02


@pytest.mark.parametrize("T,H,E", [(1, 2048, 128), (16, 512, 8), (64, 2048, 512), (600, 2048, 128), (2048, 512, 40)])
def test_router_logits_bias(T, H, E):
    """linear_forward's addmm(bias, x, W^T) (quantized_linear.h:86-94; GPT-OSS's router, gptoss.cpp:130):
    the bias is added before the one rounding, on both router kernels."""
    x = W.normal_bf16(2, 100, T * H, 1.0).reshape(T, H)
    wg = W.normal_bf16(2, 1, E * H, 0.02).reshape(E, H)
    b = W.normal_bf16(2, 13, E, 0.1)
    got = hbf(moe.router_logits(dbf(x), dbf(wg), dbf(b)))
    ref = O.router_logits(x, wg, b)
    ndiff = assert_logits_close(got, ref, x, wg, b)
    assert ndiff / got.size < 0.02
    assert (got != hbf(moe.router_logits(dbf(x), dbf(wg)))).any()


# ------------------------------------------------------------------ routing
VARIANTS = [moe.ROUTE_TOPK_LOGITS, moe.ROUTE_TOPK_PROBS, moe.ROUTE_SOFTMAX_TOPK, moe.ROUTE_SIGMOID,
            moe.ROUTE_SIGMOID_GROUP, moe.ROUTE_SIGMOID_GROUP_DROP_BEST, moe.ROUTE_SIGMOID_CORRECTED,
            moe.ROUTE_GLM4_SIGMOID, moe.ROUTE_GLM4_SOFTMAX, moe.ROUTE_LFM2]
# (the variants that take n_group / topk_group; Bailing and GLM4 compute a group index and never apply it)
GROUPED = (moe.ROUTE_SIGMOID_GROUP, moe.ROUTE_SIGMOID_GROUP_DROP_BEST, moe.ROUTE_SIGMOID_CORRECTED,
           moe.ROUTE_GLM4_SIGMOID, moe.ROUTE_GLM4_SOFTMAX)


@pytest.mark.parametrize("variant", VARIANTS)
@pytest.mark.parametrize("T,E,k,norm", [(16, 8, 2, True), (64, 128, 8, True), (33, 512, 10, True),
                                        (64, 256, 8, True), (17, 64, 6, False), (5, 1024, 16, True),
                                        (3, 40, 1, True)])
def test_route_bit_exact(variant, T, E, k, norm):
    rng = np.random.default_rng(T * 1000 + E + variant)
    lg = to_bf16(rng.normal(0, 1.0, (T, E)))
    # sprinkle exact ties to exercise the canonical tie order
    lg[:, E // 2] = lg[:, 0]
    bias = rng.normal(0, 0.01, E).astype(np.float32)
    ng, tg = (8, 3) if (variant in GROUPED and E % 8 == 0 and E >= 64) else (1, 1)
    p = moe.ops.make_router_params(variant, E, k, norm, ng, tg, 2.5)
    gi, gs = moe.route(dbf(lg), p, torch.from_numpy(bias).to(DEV))
    ri, rs, _ = O.route(lg, O.make_router(variant, E, k, norm, ng, tg, 2.5), bias)
    np.testing.assert_array_equal(host(gi).astype(np.uint32), ri)
    np.testing.assert_array_equal(host(gs).view(np.uint32), rs.view(np.uint32))


@pytest.mark.parametrize("k,norm", [(4, True), (1, True), (2, False)])
def test_route_lfm2_without_expert_bias(k, norm):
    """LFM2-MoE with use_expert_bias off (lfm2_moe.cpp:222): no score bias, the plain fp32 probabilities
    select and weigh (renormalised with + 1e-20 for any k when norm_topk_prob, bf16 weights)."""
    T, E = 20, 32
    lg = to_bf16(np.random.default_rng(3 + k).normal(0, 1.0, (T, E)))
    p = moe.ops.make_router_params(moe.ROUTE_LFM2, E, k, norm, 1, 1, 1.0)
    gi, gs = moe.route(dbf(lg), p, None)
    ri, rs, _ = O.route(lg, O.make_router(O.R_LFM2, E, k, norm, 1, 1, 1.0), None)
    np.testing.assert_array_equal(host(gi).astype(np.uint32), ri)
    np.testing.assert_array_equal(host(gs).view(np.uint32), rs.view(np.uint32))


# ------------------------------------------------------------------ bucketing
@pytest.mark.parametrize("T,k,E", [(1, 8, 128), (8, 8, 128), (16, 2, 8), (64, 8, 128), (4096, 10, 512),
                                   (8192, 8, 128), (4096, 8, 256), (3000, 4, 1000), (1, 1, 1), (3001, 3, 64)])
def test_bucket_bit_exact(T, k, E):
    inds = distinct_inds(T, k, E, seed=T + E)
    perm, inv, se, offs = moe.bucket(di32(inds), E)
    rp, ri, rse, ro = O.bucket(inds, E)
    np.testing.assert_array_equal(host(offs), ro)
    np.testing.assert_array_equal(host(perm), rp)
    np.testing.assert_array_equal(host(inv), ri)
    np.testing.assert_array_equal(host(se).astype(np.uint32), rse)


def test_bucket_skewed_single_expert():
    # every token picks expert 3 first: one bucket holds all T pairs of slot 0
    T, k, E = 20000, 2, 16
    inds = np.stack([np.full(T, 3), np.random.default_rng(0).integers(4, 16, T)], 1).astype(np.uint32)
    perm, inv, _, offs = moe.bucket(di32(inds), E)
    rp, ri, _, ro = O.bucket(inds, E)
    np.testing.assert_array_equal(host(offs), ro)
    np.testing.assert_array_equal(host(perm), rp)
    np.testing.assert_array_equal(host(inv), ri)


# ------------------------------------------------------------------ gather_qmm
@pytest.mark.parametrize("bits", [2, 3, 4, 5, 6, 8])
@pytest.mark.parametrize("E,N,K,batch", [(8, 512, 2048, 16), (4, 128, 768, 40), (16, 256, 1024, 1), (4, 256, 1024, 600)])
def test_gather_qmm_group32(bits, E, N, K, batch):
    """Group size 32 (MLX's --group-size 32): the per-16-row kernel with one MFMA per group (each lane's
    K values of a block split into the two 32-wide groups), at every width; decode-sized buckets, a
    bucket of 40 rows, one pair, and ~150 rows an expert (large buckets stay on this kernel)."""
    q = W.make_qweight(bits + 30, 2, E, N, K, 0.02, 32, bits)
    x = W.normal_bf16(bits + 30, 100, batch * K, 1.0).reshape(batch, 1, K)
    rhs = np.random.default_rng(batch + bits).integers(0, E, batch).astype(np.uint32)
    if batch == 40:
        rhs[:] = 1
    got = moe.gather_qmm(dbf(x), dqw(q), None, di32(rhs), M=1)
    assert_close(hbf(got), O.gather_qmm(x, q, None, rhs, 1), what=f"gather_qmm gs32 {bits}-bit")


@pytest.mark.parametrize("bits", [2, 3, 4, 5, 6, 8])
@pytest.mark.parametrize("E,N,K,batch,M,use_lhs", [
    (8, 512, 2048, 16, 1, True),     # examples/test_qbits.cpp:44-66 shape
    (8, 512, 2048, 16, 1, False),
    (4, 128, 768, 40, 1, False),     # > 16 rows per expert: several token chunks
    (3, 64, 512, 7, 2, True),        # M = 2, explicit lhs
    (16, 256, 1024, 1, 1, False),    # a single pair
    (8, 256, 1280, 4, 1, True),      # K split over four waves in 5-block parts: stages start on whole stages
])
def test_gather_qmm(bits, E, N, K, batch, M, use_lhs):
    q = W.make_qweight(bits, 2, E, N, K, 0.02, 64, bits)
    nx = batch + 3
    x = W.normal_bf16(bits, 100, nx * M * K, 1.0).reshape(nx, M, K)
    rng = np.random.default_rng(batch)
    rhs = rng.integers(0, E, batch).astype(np.uint32)
    if batch == 40:
        rhs[:] = 2  # all rows on one expert
    lhs = rng.integers(0, nx, batch).astype(np.uint32) if use_lhs else None
    if not use_lhs:
        x = x[:batch]
    got = moe.gather_qmm(dbf(x), dqw(q), None if lhs is None else di32(lhs), di32(rhs), M=M)
    ref = O.gather_qmm(x, q, lhs, rhs, M)
    assert_close(hbf(got), ref, what="gather_qmm")


@pytest.mark.parametrize("E,N,K,batch,M,use_lhs,biased", [
    (8, 512, 2048, 16, 1, False, False),   # decode-sized buckets
    (8, 512, 2048, 16, 1, True, True),
    (4, 256, 1024, 1000, 1, False, True),  # ~250 rows per expert
    (3, 40, 512, 9, 2, True, False),       # M = 2, a partial last column tile
    (16, 64, 96, 1, 1, False, False),      # one pair, K = 3 steps
])
def test_gather_mm(E, N, K, batch, M, use_lhs, biased):
    """Dense gather_mm (SwitchLinear's non-quantized branch, switch_layers.cpp:103-115) against the
    checker, with and without SwitchLinear's bias."""
    rng = np.random.default_rng(E * 100 + batch)
    w = W.normal_bf16(E, 2, E * N * K, 0.05).reshape(E, N, K)
    nx = batch + 3
    x = W.normal_bf16(E, 100, nx * M * K, 1.0).reshape(nx, M, K)
    rhs = rng.integers(0, E, batch).astype(np.uint32)
    lhs = rng.integers(0, nx, batch).astype(np.uint32) if use_lhs else None
    if not use_lhs:
        x = x[:batch]
    b = W.normal_bf16(E, 10, E * N, 0.1).reshape(E, N) if biased else None
    got = moe.gather_mm(dbf(x), dbf(w), None if lhs is None else di32(lhs), di32(rhs), M=M,
                        linear_bias=None if b is None else dbf(b))
    assert_close(hbf(got), O.gather_mm(x, w, lhs, rhs, M, b), what="gather_mm")


@pytest.mark.parametrize("kind,batch", [("q4", 16), ("q4", 1000), ("q6", 40), ("dense", 16), ("dense", 1000)])
def test_gather_out_of_range_experts(kind, batch):
    """rhs entries >= E (outside the contract; the checker rejects them): those output rows are zeros,
    the other rows equal the checker's on the valid pairs (per-16-row kernel at 16 and 40 pairs,
    large-bucket GEMM / dense tiles at 1000)."""
    E, N, K = 4, 256, 1024
    rng = np.random.default_rng(batch + 7)
    rhs = rng.integers(0, E, batch).astype(np.uint32)
    bad = rng.permutation(batch)[: max(1, batch // 8)]
    rhs[bad[0::2]] = E
    rhs[bad[1::2]] = 0xFFFFFFFF
    ok = rhs < E
    x = W.normal_bf16(9, 100, batch * K, 1.0).reshape(batch, 1, K)
    out = torch.full((batch, 1, N), float("nan"), dtype=torch.bfloat16, device=DEV)
    if kind == "dense":
        w = W.normal_bf16(9, 2, E * N * K, 0.05).reshape(E, N, K)
        moe.gather_mm(dbf(x), dbf(w), None, di32(rhs.view(np.int32)), M=1, out=out)
        ref = O.gather_mm(x[ok], w, None, rhs[ok], 1)
    else:
        bits = int(kind[1])
        q = W.make_qweight(bits + 40, 2, E, N, K, 0.02, 64, bits)
        moe.gather_qmm(dbf(x), dqw(q), None, di32(rhs.view(np.int32)), M=1, out=out)
        ref = O.gather_qmm(x[ok], q, None, rhs[ok], 1)
    got = hbf(out)
    assert not got[~ok].any(), "rows of out-of-range experts are not zero"
    assert_close(got[ok], ref, what=f"gather {kind} with out-of-range experts")


@pytest.mark.parametrize("bits", [2, 3, 4, 5, 6, 8])
@pytest.mark.parametrize("E,N,K,batch", [(8, 512, 2048, 16), (4, 256, 1024, 1000), (3, 40, 512, 9)])
def test_gather_qmm_linear_bias(bits, E, N, K, batch):
    """SwitchLinear with a bias (switch_layers.cpp:111-114): bf16(bf16(x.W^T) + bias[rhs]) from the
    epilogue of the per-16-row kernel (16 and 9 pairs; N = 40: a partial last tile) and of the
    large-bucket GEMM (1000 pairs)."""
    q = W.make_qweight(bits + 20, 2, E, N, K, 0.02, 64, bits)
    q.linear_bias = W.normal_bf16(bits, 10, E * N, 0.1).reshape(E, N)
    x = W.normal_bf16(bits, 100, batch * K, 1.0).reshape(batch, 1, K)
    rhs = np.random.default_rng(batch).integers(0, E, batch).astype(np.uint32)
    got = hbf(moe.gather_qmm(dbf(x), dqw(q), None, di32(rhs), M=1))
    assert_close(got, O.gather_qmm(x, q, None, rhs, 1), what="gather_qmm + linear bias")


@pytest.mark.parametrize("bits", [2, 3, 4, 5, 6, 8])
@pytest.mark.parametrize("E,N,K,batch,skew,gs", [
    (4, 256, 512, 1000, False, 64),     # ~250 rows per expert: 256-row token tiles
    (8, 512, 768, 700, True, 64),       # one expert holds half the rows, others ragged
    (2, 512, 1024, 130, False, 64),     # 64-row token tiles, partial last tile
    (3, 256, 256, 5000, True, 64),      # many token tiles per expert
    (2, 256, 1024, 600, False, 128),    # group size 128: two K steps per scale
])
def test_gather_qmm_large_buckets(bits, E, N, K, batch, skew, gs):
    """Large per-expert buckets take the LDS-staged GEMM path (prefill; 6-bit: the per-16-row
    kernel over many token chunks)."""
    q = W.make_qweight(bits + 10, 2, E, N, K, 0.02, gs, bits)
    x = W.normal_bf16(bits, 100, batch * K, 1.0).reshape(batch, 1, K)
    rng = np.random.default_rng(batch)
    rhs = rng.integers(0, E, batch).astype(np.uint32)
    if skew:
        rhs[: batch // 2] = 1
        rng.shuffle(rhs)
    lhs = rng.permutation(batch).astype(np.uint32)
    got = moe.gather_qmm(dbf(x), dqw(q), di32(lhs), di32(rhs), M=1)
    ref = O.gather_qmm(x, q, lhs, rhs, 1)
    assert_close(hbf(got), ref, what="gather_qmm (large buckets)")


@pytest.mark.parametrize("bits", [4, 8])
def test_gather_qmm_tile_classes(bits):
    """Bucket remainders (mod 128 rows) of 0, 1, 32, 33, 64, 65, 96, 97 and 127
    rows: every token-tile class of the large-bucket GEMM (128-row tiles, and
    remainder tiles of 32, 64, 96 and a partial 128 rows, each at both ends of
    its range)."""
    counts = [128, 129, 160, 161, 192, 193, 224, 225, 255]
    E, N, K = len(counts), 256, 512
    q = W.make_qweight(bits + 30, 2, E, N, K, 0.02, 64, bits)
    rhs = np.repeat(np.arange(E, dtype=np.uint32), counts)
    batch = rhs.size
    rng = np.random.default_rng(11)
    rng.shuffle(rhs)
    x = W.normal_bf16(bits + 1, 100, batch * K, 1.0).reshape(batch, 1, K)
    lhs = rng.permutation(batch).astype(np.uint32)
    got = moe.gather_qmm(dbf(x), dqw(q), di32(lhs), di32(rhs), M=1)
    assert_close(hbf(got), O.gather_qmm(x, q, lhs, rhs, 1), what="gather_qmm (tile classes)")


@pytest.mark.parametrize("bits", [4, 8])
def test_gather_qmm_large_buckets_degenerate_scales(bits):
    """Zero and extreme scales on the LDS-staged GEMM path: the workgroups that
    meet them take the exact per-group fold instead of the rescaled
    accumulator."""
    E, N, K, batch = 3, 256, 512, 900
    q = W.make_qweight(bits + 20, 2, E, N, K, 0.02, 64, bits)
    s = q.scales.copy()
    s[0, 5, 3] = 0                     # zero scale (dequantized weights = bias)
    s[1, 200, 0] = 0x0080              # smallest normal bf16 (~1.2e-38)
    s[2, 17, 7] = 0x7000               # ~1.6e29
    q = dataclasses.replace(q, scales=s)
    x = W.normal_bf16(bits, 100, batch * K, 1.0).reshape(batch, 1, K)
    rng = np.random.default_rng(7)
    rhs = rng.integers(0, E, batch).astype(np.uint32)
    lhs = rng.permutation(batch).astype(np.uint32)
    got = hbf(moe.gather_qmm(dbf(x), dqw(q), di32(lhs), di32(rhs), M=1))
    ref = O.gather_qmm(x, q, lhs, rhs, 1)
    assert np.isfinite(bf16(ref)).all()
    assert_close(got, ref, what="gather_qmm (degenerate scales)")


@pytest.mark.parametrize("bits,N", [(4, 8), (8, 40), (4, 72), (6, 24)])
def test_gather_qmm_partial_tile(bits, N):
    """N not a multiple of 16 (a router projection of 8 experts): the last 16-row tile reads row
    N-1 for its missing rows and stores only the columns below N."""
    q = W.make_qweight(5, 3, 2, N, 512, 0.02, 64, bits)
    x = W.normal_bf16(5, 100, 7 * 512, 1.0).reshape(7, 1, 512)
    rhs = np.array([0, 1, 1, 0, 1, 0, 0], np.uint32)
    got = moe.gather_qmm(dbf(x), dqw(q), None, di32(rhs))
    assert_close(hbf(got), O.gather_qmm(x, q, None, rhs, 1))


@pytest.mark.parametrize("bits,K", [(4, 512), (8, 512), (4, 1280), (8, 1280), (6, 512), (6, 1280)])
def test_gather_qmm_group128(bits, K):
    q = W.make_qweight(3, 2, 4, 64, K, 0.02, 128, bits)
    x = W.normal_bf16(3, 100, 6 * K, 1.0).reshape(6, 1, K)
    rhs = np.array([0, 3, 3, 1, 2, 0], np.uint32)
    got = moe.gather_qmm(dbf(x), dqw(q), None, di32(rhs))
    assert_close(hbf(got), O.gather_qmm(x, q, None, rhs, 1))


# ------------------------------------------------------------------ residual add + RMSNorm
@pytest.mark.parametrize("T,H", [(1, 2048), (5, 512), (300, 4096), (17, 7168), (64, 8)])
def test_add_rms_norm(T, H):
    """The step before the block (add_rms_norm, gated_delta.cpp:313-345): the sum bit-exact (fp32 add,
    round to nearest even), the normalised row within an ulp (2^-7 relative: the sum of squares is
    accumulated in another order)."""
    rng = np.random.default_rng(T + H)
    a, b = to_bf16(rng.normal(0, 1, (T, H))), to_bf16(rng.normal(0, 0.3, (T, H)))
    w = to_bf16(rng.normal(1, 0.1, H))
    s, n = moe.add_rms_norm(dbf(a), dbf(b), dbf(w), 1e-6)
    rs, rn = O.add_rms_norm(a, b, w, 1e-6)
    np.testing.assert_array_equal(hbf(s), rs)
    assert_close(hbf(n), rn, atol=1e-6, rtol=2.0**-7, what="normed")


# ------------------------------------------------------------------ swiglu / combine
def test_swiglu():
    rng = np.random.default_rng(4)
    g, u = to_bf16(rng.normal(0, 2, 10001)), to_bf16(rng.normal(0, 2, 10001))
    assert_close(hbf(moe.swiglu(dbf(g), dbf(u))), O.swiglu(g, u), atol=1e-3, rtol=8e-3)


@pytest.mark.parametrize("T,k,H,sorted_rows", [(16, 2, 512, True), (64, 8, 2048, True), (5, 10, 2048, False)])
def test_combine(T, k, H, sorted_rows):
    rng = np.random.default_rng(T)
    Y = to_bf16(rng.normal(0, 1, (T * k, H)))
    sc = rng.uniform(0, 1, (T, k)).astype(np.float32)
    if sorted_rows:
        inds = distinct_inds(T, k, 4 * k, seed=1)
        perm, inv, _, _ = O.bucket(inds, 4 * k)
        Ys = Y[perm]  # rows in sorted order
        got = moe.combine(dbf(Ys), torch.from_numpy(sc).to(DEV), di32(inv))
    else:
        got = moe.combine(dbf(Y), torch.from_numpy(sc).to(DEV))
    assert_close(hbf(got), O.combine(Y, sc), atol=1e-3, rtol=8e-3)


# ------------------------------------------------------------------ row gather / expert bias / SwitchGLU
@pytest.mark.parametrize("n_src,H,k", [(16, 2048, 8), (5, 7, 2), (300, 512, 1)])
def test_take_rows(n_src, H, k):
    """dst[i] = src[rows[i] // k]; rows outside the source give zero rows (7-element rows take
    the 2-byte path, the others the 16-byte path)."""
    rng = np.random.default_rng(n_src)
    src = to_bf16(rng.normal(0, 1, (n_src, H)))
    rows = rng.integers(0, n_src * k, n_src * k + 3).astype(np.int32)
    rows[-1] = n_src * k + 5
    rows[-2] = -1
    got = hbf(moe.take_rows(dbf(src), di32(rows), k))
    ref = np.zeros((rows.size, H), np.uint16)
    ok = (rows >= 0) & (rows // k < n_src)
    ref[ok] = src[rows[ok] // k]
    np.testing.assert_array_equal(got, ref)


@pytest.mark.parametrize("T,k,E", [(16, 2, 8), (64, 8, 128), (1000, 4, 32)])
def test_gather_sort_scatter_unsort(T, k, E):
    """gather_sort = bucket + take(x, perm // k); scatter_unsort = take(y, inv_perm)
    (switch_layers.cpp:17-46): sorted rows follow the checker's stable order and the
    round trip restores the pair order bit for bit."""
    H = 256
    x = W.normal_bf16(5, 100, T * H, 1.0).reshape(T, H)
    inds = distinct_inds(T, k, E, seed=T)
    perm, inv, se, _ = moe.bucket(di32(inds), E)
    rp, ri, rse, _ = O.bucket(inds, E)
    np.testing.assert_array_equal(host(perm), rp)
    sorted_x = moe.take_rows(dbf(x), perm, k)
    np.testing.assert_array_equal(hbf(sorted_x), x[rp // k])
    np.testing.assert_array_equal(host(se).astype(np.uint32), inds.reshape(-1)[rp])
    back = hbf(moe.take_rows(sorted_x, inv, 1))
    np.testing.assert_array_equal(back, np.repeat(x, k, axis=0))


def test_add_expert_bias():
    rng = np.random.default_rng(9)
    batch, M, N, E = 37, 2, 300, 5
    out = to_bf16(rng.normal(0, 1, (batch, M, N)))
    bias = to_bf16(rng.normal(0, 1, (E, N)))
    rhs = rng.integers(0, E, batch).astype(np.int32)
    rhs[3] = E + 2  # no such expert: the row is left as it is
    got = hbf(moe.add_expert_bias(dbf(out), dbf(bias), di32(rhs)))
    ref = out.copy()
    ok = rhs < E
    ref[ok] = to_bf16(bf16(out[ok]) + bf16(bias[rhs[ok]])[:, None, :])
    np.testing.assert_array_equal(got, ref)


@pytest.mark.parametrize("T,k,E,H,I,bits", [(5, 2, 8, 512, 1024, 4), (512, 4, 8, 512, 1024, 4), (64, 6, 16, 256, 512, 8)])
def test_switch_mlp_relu2(T, k, E, H, I, bits):
    """Nemotron-H SwitchMLP (nemotron_h.cpp:484-511) against the checker's composition: gather_qmm(fc1),
    relu_squared (bf16(max(v, 0)^2), activations.h:45-55), gather_qmm(fc2), unsorted.  The second case
    runs both projections on the large-bucket GEMM."""
    up = W.make_qweight(T + 7, 3, E, I, H, 0.02, 64, bits)
    dn = W.make_qweight(T + 7, 4, E, H, I, 0.02, 64, bits)
    x = W.normal_bf16(T, 100, T * H, 1.0).reshape(T, H)
    inds = distinct_inds(T, k, E, seed=T + k + 1)
    got = hbf(moe.switch_mlp_relu2(dbf(x), di32(inds), dqw(up), dqw(dn)))
    flat = inds.reshape(-1)
    lhs = np.repeat(np.arange(T, dtype=np.uint32), k)
    hh = bf16(O.gather_qmm(x.reshape(T, 1, H), up, lhs, flat, 1)).astype(np.float32)
    h2 = to_bf16(np.maximum(hh, 0.0) * np.maximum(hh, 0.0))
    ref = O.gather_qmm(h2, dn, None, flat, 1).reshape(T, k, H)
    assert got.shape == (T, k, H)
    assert_close(got, ref, what="switch_mlp_relu2")


@pytest.mark.parametrize("T,k,E,H,I,bits,gs", [
    (16, 2, 8, 512, 1024, 4, 64),     # tiny config
    (3, 8, 128, 2048, 768, 4, 64),    # Qwen3-30B-A3B shape, decode
    (40, 4, 6, 256, 512, 8, 64),      # 8-bit
    (600, 2, 4, 512, 256, 4, 64),     # ~300 pairs per expert: the GEMM path (h group sums from gate|up)
    (700, 2, 4, 512, 512, 4, 128),    # GEMM path, group size 128 (zero-padded group-sum chunk)
    (500, 2, 2, 256, 768, 8, 64),     # GEMM path, 8-bit (zero code offset)
    (16, 2, 8, 512, 1024, 6, 64),     # 6-bit
    (600, 2, 4, 512, 256, 6, 64),     # 6-bit, ~300 pairs per expert (per-16-row kernel, many chunks)
    (40, 4, 6, 256, 512, 6, 128),     # 6-bit, group size 128
])
def test_switch_glu(T, k, E, H, I, bits, gs):
    """SwitchGLU (switch_layers.cpp:200-245) against the checker's composition of the
    reference ops: gather_qmm(gate), gather_qmm(up), swiglu, gather_qmm(down), unsorted."""
    _switch_glu_case(T, k, E, H, I, bits, gs, False)


@pytest.mark.parametrize("T,k,E,H,I,bits", [(16, 2, 8, 512, 1024, 4), (600, 2, 4, 512, 256, 4), (40, 4, 6, 256, 512, 8)])
def test_switch_glu_linear_bias(T, k, E, H, I, bits):
    """SwitchGLU(bias=true) (switch_layers.cpp:101-115): each projection's bias added to its bf16 output
    before the SwiGLU (gate, up) or as the result (down), on the per-16-row kernels and on the GEMMs."""
    _switch_glu_case(T, k, E, H, I, bits, 64, True)


@pytest.mark.parametrize("T,k,E,H,I,bits", [(16, 2, 8, 512, 1024, 4), (600, 2, 4, 512, 256, 4), (40, 4, 6, 256, 512, 8),
                                            (500, 2, 2, 256, 768, 8)])
@pytest.mark.parametrize("act", [moe.ACT_GPTOSS, moe.ACT_GPTOSS_UPSTREAM])
def test_switch_glu_gptoss(T, k, E, H, I, bits, act):
    """SwitchGLU with GPT-OSS's clipped SwiGLU between gate|up and down (gptoss.cpp:50-58, called as
    swiglu(x_gate, x_up) at :158; or the upstream roles), linear biases ~ N(0, 4) on gate and up so the
    clip limits are crossed: the fused epilogues of the per-16-row kernels and of the GEMMs against the
    checker's composition gather_qmm, gather_qmm, gptoss_swiglu, gather_qmm."""
    _switch_glu_case(T, k, E, H, I, bits, 64, True, act)


def test_gptoss_swiglu():
    """moe_gptoss_swiglu against the checker, inputs straddling -7 and +7."""
    rng = np.random.default_rng(5)
    a, b = to_bf16(rng.normal(0, 6, 10001)), to_bf16(rng.normal(0, 6, 10001))
    h, _ = O.gptoss_swiglu(a, b)
    assert_close(hbf(moe.gptoss_swiglu(dbf(a), dbf(b))), h, atol=1e-3, rtol=8e-3)


def _switch_glu_case(T, k, E, H, I, bits, gs, biased, act=0):
    g = W.make_qweight(T + 1, 2, E, I, H, 0.02, gs, bits)
    u = W.make_qweight(T + 1, 3, E, I, H, 0.02, gs, bits)
    d = W.make_qweight(T + 1, 4, E, H, I, 0.02, gs, bits)
    if biased:
        std = 4.0 if act else 0.1
        for q, tid, sd in ((g, 10, std), (u, 11, std), (d, 12, 0.1)):
            q.linear_bias = W.normal_bf16(T, tid, q.experts * q.N, sd).reshape(q.experts, q.N)
    x = W.normal_bf16(T, 100, T * H, 1.0).reshape(T, H)
    inds = distinct_inds(T, k, E, seed=T + k)
    got = hbf(moe.switch_glu(dbf(x), di32(inds), dqw(g), dqw(u), dqw(d), act))
    flat = inds.reshape(-1)
    lhs = np.repeat(np.arange(T, dtype=np.uint32), k)
    gg = O.gather_qmm(x.reshape(T, 1, H), g, lhs, flat, 1)
    uu = O.gather_qmm(x.reshape(T, 1, H), u, lhs, flat, 1)
    if act == moe.ACT_GPTOSS:
        h = O.gptoss_swiglu(gg, uu)[0]
    elif act == moe.ACT_GPTOSS_UPSTREAM:
        h = O.gptoss_swiglu(uu, gg)[0]
    else:
        h = O.swiglu(gg, uu)
    ref = O.gather_qmm(h, d, None, flat, 1).reshape(T, k, H)
    assert got.shape == (T, k, H)
    assert_close(got, ref, what="switch_glu")
