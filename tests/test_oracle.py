"""Pins the CPU checker (oracle/) before it is trusted.

Each oracle function is checked against what the reference itself fixes (the
dequant known-answer test of examples/diagnose.cpp:297-311, the gather_qmm
construction of examples/test_qbits.cpp:51-58) and, where the reference holds
no vector, against an independent numpy fp64 restatement, brute force, closed
forms and invariants.  No GPU needed.
"""
import numpy as np
import pytest

from helpers import ATOL, RTOL, assert_close, assert_close_block, bf16, h_rounding_mag, load_pkg, to_bf16
from oracle import moe_oracle as O

moe = load_pkg()
from lemon_mlx_engine_amd import workloads as W  # noqa: E402


# ---------------------------------------------------------------- numpy restatements
def np_codes(w, K, bits):
    """Codes of packed rows: the rows' bytes in little-endian order as one LSB-first bit stream,
    `bits` bits per code (numpy's unpackbits, independent of the per-word shifts in the checker)."""
    w = np.ascontiguousarray(np.asarray(w, np.uint32).reshape(-1, K * bits // 32))
    stream = np.unpackbits(w.astype("<u4").view(np.uint8), axis=1, bitorder="little")
    fields = stream.reshape(w.shape[0], K, bits).astype(np.uint64)
    return (fields << np.arange(bits, dtype=np.uint64)).sum(-1)


def np_dequant(w, s, b, K, gs, bits):
    """LSB-first unpack, w = s*q + b per group (debug_numerical_trace.py:67-98 form)."""
    q = np_codes(w, K, bits).astype(np.float64)
    s = bf16(s).reshape(q.shape[0], -1).astype(np.float64)
    b = np.zeros_like(s) if b is None else bf16(b).reshape(q.shape[0], -1).astype(np.float64)
    return q * np.repeat(s, gs, axis=1) + np.repeat(b, gs, axis=1)


def np_sigmoid(v):
    return 1.0 / (1.0 + np.exp(-v))


def np_softmax(v):
    e = np.exp(v - v.max(-1, keepdims=True))
    return e / e.sum(-1, keepdims=True)


def np_topk(sel, k):
    """Canonical order: value descending, index ascending (lexsort brute force)."""
    T, E = sel.shape
    out = np.empty((T, k), np.int64)
    for t in range(T):
        order = np.lexsort((np.arange(E), -sel[t].astype(np.float64)))
        out[t] = order[:k]
    return out


def np_silu(g):
    return g / (1.0 + np.exp(-g))


def np_gptoss(x_linear, x_glu):
    """GPT-OSS's swiglu (gptoss.cpp:50-58, alpha 1.702, limit 7) in fp64: the linear input clipped to
    [-7, 7], the gated input clipped from above only."""
    xl = np.clip(x_linear, -7.0, 7.0)
    xg = np.minimum(x_glu, 7.0)
    return xg * np_sigmoid(1.702 * xg) * (xl + 1.0)


def np_act(act, g, u):
    if act == O.ACT_GPTOSS:
        return np_gptoss(g, u)  # swiglu(x_gate, x_up), gptoss.cpp:158
    if act == O.ACT_GPTOSS_UPSTREAM:
        return np_gptoss(u, g)
    return np_silu(g) * u


def np_block(layer, x, inds, scores):
    """fp64 restatement of SwitchGLU + combine (+ shared) with given routing (the routed experts'
    activation is layer.cfg.activation)."""
    cfg = layer.cfg
    H, I = cfg.hidden, cfg.intermediate
    xf = bf16(x).astype(np.float64)
    T, k = inds.shape
    out = np.zeros((T, H))
    cache = {}

    def deq(q, e):
        key = (id(q), e)
        if key not in cache:
            cache[key] = np_dequant(q.w[e], q.scales[e], q.biases[e], q.K, q.group_size, q.bits)
        return cache[key]

    def lb(q, e):  # SwitchLinear's bias (0 without one)
        return 0.0 if q.linear_bias is None else bf16(q.linear_bias[e]).astype(np.float64)

    for t in range(T):
        for j in range(k):
            e = int(inds[t, j])
            g = deq(layer.gate, e) @ xf[t] + lb(layer.gate, e)
            u = deq(layer.up, e) @ xf[t] + lb(layer.up, e)
            h = np_act(cfg.activation, g, u)
            out[t] += scores[t, j] * (deq(layer.down, e) @ h + lb(layer.down, e))
    if layer.shared is not None:
        sg, su, sd, sgw = layer.shared
        g = xf @ deq(sg, 0).T
        u = xf @ deq(su, 0).T
        ys = (np_silu(g) * u) @ deq(sd, 0).T
        if sgw is None:
            gate = 1.0
        elif isinstance(sgw, np.ndarray):
            gate = np_sigmoid(xf @ bf16(sgw).astype(np.float64).T)
        else:  # a quantized gate [1][1, H]
            gate = np_sigmoid(xf @ deq(sgw, 0).T)
        out += gate * ys
    return out


# ---------------------------------------------------------------- dequant
def test_dequant_kat_4bit():
    # reference examples/diagnose.cpp:297-311: 0x76543210, s=1, b=0, gs=8 -> 0..7
    w = np.array([0x76543210], np.uint32)
    out = O.dequant(w, to_bf16([1.0]), to_bf16([0.0]), 1, 8, 8, 4)
    assert out.tolist() == [[0, 1, 2, 3, 4, 5, 6, 7]]


def test_dequant_kat_8bit():
    w = np.array([0x03020100], np.uint32)
    out = O.dequant(w, to_bf16([1.0]), to_bf16([0.0]), 1, 4, 4, 8)
    assert out.tolist() == [[0, 1, 2, 3]]


def test_dequant_6bit_three_byte_packs():
    """6 bits: four codes per three bytes, least significant first.  Codes (q0, q1, q2, q3) of a
    pack are byte0 = q0 | q1 << 6, byte1 = q1 >> 2 | q2 << 4, byte2 = q2 >> 4 | q3 << 2 (the
    24-bit little-endian value q0 + 64 q1 + 4096 q2 + 262144 q3).  A wrong bit or byte order,
    or packing each code into its own byte, fails this."""
    rng = np.random.default_rng(11)
    K = 64
    q = rng.integers(0, 64, K)
    by = np.zeros(K * 6 // 8, np.uint8)
    for p in range(K // 4):
        q0, q1, q2, q3 = (int(v) for v in q[4 * p:4 * p + 4])
        by[3 * p] = (q0 | (q1 << 6)) & 0xFF
        by[3 * p + 1] = ((q1 >> 2) | (q2 << 4)) & 0xFF
        by[3 * p + 2] = ((q2 >> 4) | (q3 << 2)) & 0xFF
    w = by.view("<u4")
    out = O.dequant(w, to_bf16([1.0]), to_bf16([0.0]), 1, K, K, 6)
    assert out[0].tolist() == q.astype(np.float32).tolist()
    assert np_codes(w, K, 6)[0].tolist() == q.tolist()


@pytest.mark.parametrize("bits", [3, 5])
def test_dequant_odd_width_packs(bits):
    """3 and 5 bits: eight codes per `bits` bytes, least significant first -- a pack is the
    little-endian integer sum(q_i << bits*i) (MLX's packing of these widths; the 6-bit rule above is
    the same with four codes).  Built byte by byte from Python integers: a wrong bit or byte order,
    or per-word packing that does not cross word boundaries, fails this."""
    rng = np.random.default_rng(12 + bits)
    K = 128
    q = rng.integers(0, 1 << bits, K)
    by = bytearray()
    for p in range(K // 8):
        v = sum(int(c) << (bits * i) for i, c in enumerate(q[8 * p:8 * p + 8]))
        by += v.to_bytes(bits, "little")
    w = np.frombuffer(bytes(by), dtype="<u4")
    out = O.dequant(w, to_bf16([1.0] * (K // 64)), to_bf16([0.0] * (K // 64)), 1, K, 64, bits)
    assert out[0].tolist() == q.astype(np.float32).tolist()
    assert np_codes(w, K, bits)[0].tolist() == q.tolist()


@pytest.mark.parametrize("gs", [32, 64, 128])
@pytest.mark.parametrize("bits", [2, 3, 4, 5, 6, 8])
def test_dequant_closed_form(bits, gs):
    rng = np.random.default_rng(1)
    rows, K = 5, 256
    w = rng.integers(0, 2**32, size=(rows, K * bits // 32), dtype=np.uint64).astype(np.uint32)
    s = to_bf16(rng.normal(0, 0.01, (rows, K // gs)))
    b = to_bf16(rng.normal(0, 0.1, (rows, K // gs)))
    got = O.dequant(w, s, b, rows, K, gs, bits)
    ref = np_dequant(w, s, b, K, gs, bits)
    np.testing.assert_allclose(got, ref, rtol=1e-6, atol=1e-7)


@pytest.mark.parametrize("gs", [32, 64])
@pytest.mark.parametrize("bits", [2, 3, 4, 5, 6, 8])
def test_quantizer_roundtrip(bits, gs):
    """moe_quantize_affine + dequant reproduces each weight within half a step."""
    rng = np.random.default_rng(2)
    rows, K = 16, 512
    wd = to_bf16(rng.normal(0, 0.02, (rows, K)))
    wq, s, b = W.quantize(wd, rows, K, gs, bits)
    deq = O.dequant(wq, s, b, rows, K, gs, bits).astype(np.float64)
    step = np.abs(np.repeat(bf16(s).reshape(rows, -1), gs, axis=1)).astype(np.float64)
    err = np.abs(deq - bf16(wd))
    q = np_codes(wq, K, bits).astype(np.float64)
    nb = (1 << bits) - 1
    # Interior codes: half a step, plus the scale's bf16 rounding (2^-9
    # relative) carried q times.  Edge codes may also be clipped by up to one
    # step, because the scale is re-derived as edge/round(edge/scale) so that
    # the anchored edge is exact.
    bound = 0.5 * step + q * step * 2.0**-8 + 1e-9
    edge = (q == 0) | (q == nb)
    bound[edge] += 0.5 * step[edge]
    assert (err <= bound).all()
    # the anchored edge of every group is the group's min or max, reproduced exactly
    g = q.reshape(rows, K // gs, gs)
    assert ((g.min(-1) == 0)).all()


def test_generator_is_counter_based():
    a = W.normal_bf16(7, 3, 1000, 1.0)
    b = W.normal_bf16(7, 3, 600, 1.0, first=400)
    assert (a[400:] == b).all()
    big = bf16(W.normal_bf16(0, 1, 200000, 0.02)).astype(np.float64)
    assert abs(big.mean()) < 2e-4 and abs(big.std() - 0.02) < 2e-4


# ---------------------------------------------------------------- canonical exp
def test_canon_expf_accuracy():
    xs = np.concatenate([np.linspace(-86.9, 88.0, 20011), np.linspace(-2, 2, 4001)]).astype(np.float32)
    got = np.array([O.canon_expf(float(v)) for v in xs], np.float32)
    ref = np.exp(xs.astype(np.float64))
    ulp = np.spacing(ref.astype(np.float32)).astype(np.float64)
    assert (np.abs(got - ref) <= 2 * ulp).all()
    assert O.canon_expf(-100.0) == 0.0 and O.canon_expf(0.0) == 1.0


# ---------------------------------------------------------------- router
def test_router_logits_bias():
    """addmm(bias, x, W^T) (quantized_linear.h:86-94, GPT-OSS's router gptoss.cpp:130): x = 0 gives the
    bias exactly; otherwise within one bf16 ulp of the exact x.W^T + b."""
    rng = np.random.default_rng(4)
    E, H = 24, 512
    wg = to_bf16(rng.normal(0, 0.02, (E, H)))
    b = to_bf16(rng.normal(0, 0.1, E))
    np.testing.assert_array_equal(O.router_logits(np.zeros((3, H), np.uint16), wg, b), np.tile(b, (3, 1)))
    x = to_bf16(rng.normal(0, 1, (9, H)))
    got = O.router_logits(x, wg, b)
    ref = bf16(x).astype(np.float64) @ bf16(wg).astype(np.float64).T + bf16(b).astype(np.float64)
    ulp = np.spacing(np.abs(bf16(to_bf16(ref))).astype(np.float32), dtype=np.float32) * 65536
    assert (np.abs(bf16(got) - ref) <= ulp).all()
    assert (got != O.router_logits(x, wg)).any()


def test_router_logits_vs_numpy():
    rng = np.random.default_rng(3)
    x = to_bf16(rng.normal(0, 1, (9, 512)))
    wg = to_bf16(rng.normal(0, 0.02, (24, 512)))
    got = O.router_logits(x, wg)
    ref = bf16(x).astype(np.float64) @ bf16(wg).astype(np.float64).T
    ulp = np.spacing(np.abs(bf16(to_bf16(ref))).astype(np.float32) * 1.0, dtype=np.float32) * 65536
    assert (np.abs(bf16(got) - ref) <= ulp).all()  # within one bf16 ulp of the exact product


def _logits(T, E, seed, scale=1.0):
    rng = np.random.default_rng(seed)
    return to_bf16(rng.normal(0, scale, (T, E)))


GROUPED = (O.R_SIGMOID_GROUP, O.R_SIGMOID_GROUP_DROP_BEST, O.R_SIGMOID_CORRECTED, O.R_GLM4_SIGMOID,
           O.R_GLM4_SOFTMAX)
ALL_VARIANTS = [O.R_TOPK_LOGITS, O.R_TOPK_PROBS, O.R_SOFTMAX_TOPK, O.R_SIGMOID, O.R_SIGMOID_GROUP,
                O.R_SIGMOID_GROUP_DROP_BEST, O.R_SIGMOID_CORRECTED, O.R_GLM4_SIGMOID, O.R_GLM4_SOFTMAX,
                O.R_LFM2]


@pytest.mark.parametrize("variant", ALL_VARIANTS)
@pytest.mark.parametrize("E,k", [(8, 2), (128, 8), (512, 10), (256, 8)])
def test_route_selection_bruteforce(variant, E, k):
    T = 33
    lg = _logits(T, E, seed=E + variant)
    ng, tg = (8, 3) if (variant in GROUPED and E % 8 == 0 and E >= 64) else (1, 1)
    bias = np.random.default_rng(5).normal(0, 0.01, E).astype(np.float32)
    p = O.make_router(variant, E, k, True, ng, tg, 2.5)
    inds, scores, sel = O.route(lg, p, bias)
    np.testing.assert_array_equal(inds, np_topk(sel, k))
    # the selection values are what each reference router compares
    lf = bf16(lg).astype(np.float64)
    if variant in (O.R_TOPK_LOGITS, O.R_SOFTMAX_TOPK):
        assert (sel == bf16(lg)).all()
    elif variant == O.R_TOPK_PROBS:
        assert_close(to_bf16(sel), to_bf16(np_softmax(lf)), atol=1e-6, rtol=8e-3, what="probs")
    elif variant == O.R_SIGMOID:
        assert_close(to_bf16(sel), to_bf16(np_sigmoid(lf)), atol=1e-6, rtol=8e-3, what="sigmoid")
    elif variant in (O.R_GLM4_SOFTMAX, O.R_LFM2):  # fp32 softmax + bias; GLM4 never applies its group index
        np.testing.assert_allclose(sel, np_softmax(lf) + bias, rtol=1e-5, atol=1e-7)
    else:
        corr = np_sigmoid(lf) + bias
        # Bailing and GLM4 compute the groups but never apply them
        if ng > 1 and variant in (O.R_SIGMOID_GROUP, O.R_SIGMOID_GROUP_DROP_BEST):
            gsz = E // ng
            gsc = np.sort(corr.reshape(T, ng, gsz), -1)[..., -2:].sum(-1)
            keep = np.zeros((T, ng), bool)
            for t in range(T):
                order = np.lexsort((np.arange(ng), -gsc[t]))  # best group first
                if variant == O.R_SIGMOID_GROUP:
                    keep[t, order[:tg]] = True  # upstream noaux_tc: keep the topk_group best
                else:
                    keep[t, order[ng - tg:]] = True  # as written: the n_group - topk_group best are zeroed
            corr = corr * np.repeat(keep, gsz, axis=1)
        np.testing.assert_allclose(sel, corr, rtol=1e-6, atol=1e-6)


@pytest.mark.parametrize("variant", ALL_VARIANTS)
@pytest.mark.parametrize("norm", [True, False])
def test_route_weights_closed_form(variant, norm):
    T, E, k, rsf = 40, 64, 6, 2.5
    lg = _logits(T, E, seed=11)
    bias = np.random.default_rng(6).normal(0, 0.01, E).astype(np.float32)
    p = O.make_router(variant, E, k, norm, 1, 1, rsf)
    inds, scores, _ = O.route(lg, p, bias)
    lf = bf16(lg).astype(np.float64)
    rows = np.arange(T)[:, None]
    if variant in (O.R_TOPK_LOGITS, O.R_TOPK_PROBS):
        w = np_softmax(lf)[rows, inds]
        if norm:
            w = w / w.sum(-1, keepdims=True)
    elif variant == O.R_SOFTMAX_TOPK:
        w = np_softmax(lf[rows, inds])
    elif variant == O.R_SIGMOID:
        w = np_sigmoid(lf)[rows, inds]
        if norm:
            w = w / w.sum(-1, keepdims=True) * rsf
    elif variant == O.R_SIGMOID_CORRECTED:  # Bailing: the corrected scores are the weights, cast to bf16
        w = (np_sigmoid(lf) + bias)[rows, inds]
        if norm:
            w = w / w.sum(-1, keepdims=True)
        w = w * rsf
        assert (bf16(to_bf16(scores)) == scores).all()
    elif variant == O.R_LFM2:  # the biased probabilities, renormalised with + 1e-20, in bf16; no scaling
        w = (np_softmax(lf) + bias)[rows, inds]
        if norm:
            w = w / (w.sum(-1, keepdims=True) + 1e-20)
        assert (bf16(to_bf16(scores)) == scores).all()
    elif variant in (O.R_GLM4_SIGMOID, O.R_GLM4_SOFTMAX):  # fp32 weights: uncorrected scores, no epsilon
        w = (np_sigmoid(lf) if variant == O.R_GLM4_SIGMOID else np_softmax(lf))[rows, inds]
        if norm:
            w = w / w.sum(-1, keepdims=True)
        np.testing.assert_allclose(scores, w * rsf, rtol=2e-6, atol=1e-9)
        w = w * rsf
    else:
        w = np_sigmoid(lf)[rows, inds]
        if norm:
            w = w / w.sum(-1, keepdims=True)
        w = w * rsf
    np.testing.assert_allclose(scores, w, rtol=1.2e-2, atol=1e-6)
    if variant in (O.R_TOPK_LOGITS, O.R_TOPK_PROBS, O.R_SOFTMAX_TOPK):
        assert (to_bf16(scores) == to_bf16(scores.astype(np.float32))).all()
        assert (bf16(to_bf16(scores)) == scores).all(), "bf16 variants return bf16-exact weights"


def test_glm4_gate_has_no_epsilon_and_no_group_limit():
    """glm4_moe.cpp:158-191 against R6: with every logit near -42 the sigmoid scores are ~1e-18, where
    R6's renorm epsilon (1e-20) moves the weights by ~1e-3 and GLM4's (none) keeps their sum at
    routed_scaling_factor; and GLM4 routes on the corrected scores over all groups where R6 confines the
    top-k to the topk_group best groups."""
    E, k, rsf = 16, 4, 2.5
    lg = to_bf16(np.full((1, E), -44.0) + np.arange(E) * 0.25)
    glm = O.route(lg, O.make_router(O.R_GLM4_SIGMOID, E, k, True, 1, 1, rsf))[1]
    r6 = O.route(lg, O.make_router(O.R_SIGMOID_GROUP, E, k, True, 1, 1, rsf), np.zeros(E, np.float32))[1]
    assert abs(float(glm.astype(np.float64).sum()) - rsf) < 1e-5
    assert abs(float(r6.astype(np.float64).sum()) - rsf) > 1e-4
    # group limit: the 4 best corrected scores all lie in group 0 of 4, yet GLM4 picks them
    bias = np.zeros(E, np.float32)
    bias[:4] = 1.0
    lg2 = to_bf16(np.zeros((1, E)))
    gi = O.route(lg2, O.make_router(O.R_GLM4_SOFTMAX, E, k, True, 4, 1, 1.0), bias)[0]
    assert sorted(gi[0].tolist()) == [0, 1, 2, 3]
    ri = O.route(lg2, O.make_router(O.R_SIGMOID_GROUP, E, k, True, 4, 2, 1.0), bias)[0]
    assert sorted(ri[0].tolist()) == [0, 1, 2, 3]
    bias[[0, 4, 8, 12]] = 2.0  # one strong expert per group: a limit to 1 group would keep only one
    gi = O.route(lg2, O.make_router(O.R_GLM4_SIGMOID, E, k, True, 4, 1, 1.0), bias)[0]
    assert sorted(gi[0].tolist()) == [0, 4, 8, 12]


def test_route_ties_go_to_lower_index():
    lg = to_bf16(np.array([[0.5, 1.0, 1.0, 0.25, 1.0, -1.0, 0.5, 0.0]]))
    inds, _, _ = O.route(lg, O.make_router(O.R_TOPK_LOGITS, 8, 4), None)
    assert inds.tolist() == [[1, 2, 4, 0]]


def test_r3_equals_r1_renorm():
    # softmax over the top-k logits == renormalised full softmax restricted to top-k
    lg = _logits(64, 128, seed=21)
    i1, s1, _ = O.route(lg, O.make_router(O.R_TOPK_LOGITS, 128, 8, True), None)
    i3, s3, _ = O.route(lg, O.make_router(O.R_SOFTMAX_TOPK, 128, 8, True), None)
    np.testing.assert_array_equal(i1, i3)
    np.testing.assert_allclose(s1, s3, rtol=1.6e-2, atol=1e-6)


def test_group_limit_as_written_drops_best_groups():
    """nemotron_h.cpp:425-447 negates the group scores before argpartition, so the groups it zeroes are
    the n_group - topk_group BEST: with one strong group among 4 (topk_group 3) the upstream rule
    routes into it and the as-written rule never does."""
    E, G, k = 16, 4, 2
    lg = np.full((1, E), to_bf16(np.array([-2.0]))[0], np.uint16)
    lg[0, 4:8] = to_bf16(np.array([3.0, 2.5, 2.0, 1.5]))  # group 1 is the best by far
    bias = np.zeros(E, np.float32)
    up, _, _ = O.route(lg, O.make_router(O.R_SIGMOID_GROUP, E, k, True, G, 3, 1.0), bias)
    aw, _, sel = O.route(lg, O.make_router(O.R_SIGMOID_GROUP_DROP_BEST, E, k, True, G, 3, 1.0), bias)
    assert set(up[0].tolist()) == {4, 5}
    assert not (set(aw[0].tolist()) & {4, 5, 6, 7}) and (sel[0, 4:8] == 0).all()


def test_group_limit_drops_lowest_groups():
    # experts of group 0 have the best single score but group 0 has the worst
    # top-2 sum: it must be dropped, so no expert of group 0 is selected.
    E, ng, tg = 16, 4, 2
    lf = np.full((1, E), -4.0)
    lf[0, 0] = 3.0                          # group 0: one strong expert, others weak
    lf[0, 4:8] = [1.0, 1.0, 0.9, 0.9]      # group 1 strong pair
    lf[0, 8:12] = [0.8, 0.8, 0.7, 0.7]     # group 2
    lf[0, 12:16] = [-2.0, -2.0, -2.0, -2.0]
    p = O.make_router(O.R_SIGMOID_GROUP, E, 4, True, ng, tg, 1.0)
    inds, _, sel = O.route(to_bf16(lf), p, np.zeros(E, np.float32))
    assert set(inds[0].tolist()) == {4, 5, 6, 7}
    assert (sel[0, 0:4] == 0).all() and (sel[0, 12:16] == 0).all()


# ---------------------------------------------------------------- bucketing
@pytest.mark.parametrize("T,k,E", [(1, 8, 128), (16, 2, 8), (64, 8, 128), (333, 10, 512), (4096, 8, 256)])
def test_bucket_vs_stable_argsort(T, k, E):
    rng = np.random.default_rng(T + E)
    inds = np.stack([rng.choice(E, k, replace=False) for _ in range(T)]).astype(np.uint32)
    perm, inv, se, offs = O.bucket(inds, E)
    flat = inds.reshape(-1)
    ref = np.argsort(flat, kind="stable")
    np.testing.assert_array_equal(perm, ref)
    np.testing.assert_array_equal(inv, np.argsort(ref, kind="stable"))
    np.testing.assert_array_equal(se, flat[ref])
    np.testing.assert_array_equal(offs, np.concatenate([[0], np.cumsum(np.bincount(flat, minlength=E))]))
    assert offs[-1] == T * k and (inv[perm] == np.arange(T * k)).all()


def test_bucket_rejects_out_of_range():
    with pytest.raises(ValueError):
        O.bucket(np.array([[0, 9]], np.uint32), 8)


# ---------------------------------------------------------------- gather_qmm
def _qw(E, N, K, bits, seed, gs=64):
    return W.make_qweight(seed, 2, E, N, K, 0.02, gs, bits)


@pytest.mark.parametrize("bits", [2, 3, 4, 5, 6, 8])
def test_gather_qmm_test_qbits_construction(bits):
    # reference examples/test_qbits.cpp:44-66: E=8, N=512, K=2048, B=16, M=1,
    # rhs = arange(B) % E, lhs = identity; reference = take(dequantize) + matmul
    E, N, K, B = 8, 512, 2048, 16
    q = _qw(E, N, K, bits, seed=bits)
    x = W.normal_bf16(9, 100, B * K, 1.0).reshape(B, 1, K)
    rhs = (np.arange(B) % E).astype(np.uint32)
    got = O.gather_qmm(x, q, np.arange(B, dtype=np.uint32), rhs, 1)
    ref = np.stack([np_dequant(q.w[e], q.scales[e], q.biases[e], K, 64, bits) @ bf16(x[b, 0]).astype(np.float64)
                    for b, e in enumerate(rhs)])[:, None, :]
    assert_close(got, to_bf16(ref), what="gather_qmm")
    rel = np.abs(bf16(got) - ref).mean() / np.abs(ref).mean()
    assert rel < 0.01  # test_qbits flags > 0.05 as garbage


def test_gather_qmm_linear_bias():
    """SwitchLinear's bias (switch_layers.cpp:111-114): out = bf16(bf16(x.W^T) + bias[rhs]).  Zero input
    gives the gathered bias exactly; a zero bias changes nothing; otherwise bf16(gather_qmm) + bias
    rounded once more."""
    E, N, K, B = 4, 64, 256, 10
    q = _qw(E, N, K, 4, seed=11)
    rng = np.random.default_rng(12)
    q.linear_bias = to_bf16(rng.normal(0, 0.1, (E, N)))
    rhs = (np.arange(B) * 3 % E).astype(np.uint32)
    got0 = O.gather_qmm(np.zeros((B, 1, K), np.uint16), q, None, rhs, 1)
    np.testing.assert_array_equal(got0[:, 0], q.linear_bias[rhs])
    x = W.normal_bf16(13, 100, B * K, 1.0).reshape(B, 1, K)
    got = O.gather_qmm(x, q, None, rhs, 1)
    lb = q.linear_bias
    q.linear_bias = None
    plain = O.gather_qmm(x, q, None, rhs, 1)
    np.testing.assert_array_equal(got[:, 0], to_bf16(bf16(plain[:, 0]) + bf16(lb[rhs])))
    q.linear_bias = np.zeros_like(lb)
    np.testing.assert_array_equal(O.gather_qmm(x, q, None, rhs, 1), plain)


def test_gather_mm_vs_numpy():
    """Dense gather_mm (SwitchLinear's non-quantized branch, switch_layers.cpp:103-115): take the expert's
    weight, matmul (fp64 numpy), within the tolerance; a one-hot x selects a weight column exactly; with
    a bias, x = 0 gives the bias exactly."""
    E, N, K, B, M = 5, 48, 256, 9, 2
    rng = np.random.default_rng(21)
    w = to_bf16(rng.normal(0, 0.05, (E, N, K)))
    x = to_bf16(rng.normal(0, 1, (B + 2, M, K)))
    rhs = rng.integers(0, E, B).astype(np.uint32)
    lhs = rng.integers(0, B + 2, B).astype(np.uint32)
    got = O.gather_mm(x, w, lhs, rhs, M)
    ref = np.einsum("bmk,bnk->bmn", bf16(x[lhs]).astype(np.float64), bf16(w[rhs]).astype(np.float64))
    assert_close(got, to_bf16(ref), what="gather_mm")
    oh = np.zeros((1, 1, K), np.uint16)
    oh[0, 0, 17] = to_bf16(np.array([1.0]))[0]
    np.testing.assert_array_equal(O.gather_mm(oh, w, None, np.array([3], np.uint32))[0, 0], w[3, :, 17])
    b = to_bf16(rng.normal(0, 0.1, (E, N)))
    z = O.gather_mm(np.zeros((B, 1, K), np.uint16), w, None, rhs, 1, b)
    np.testing.assert_array_equal(z[:, 0], b[rhs])


def test_gather_qmm_one_hot_selects_column():
    q = _qw(3, 32, 128, 4, seed=5)
    x = np.zeros((1, 1, 128), np.uint16)
    x[0, 0, 77] = to_bf16([1.0])[0]
    got = O.gather_qmm(x, q, None, np.array([2], np.uint32), 1)
    col = np_dequant(q.w[2], q.scales[2], q.biases[2], 128, 64, 4)[:, 77]
    np.testing.assert_array_equal(got[0, 0], to_bf16(col))


def test_gather_qmm_integer_exact():
    # s = 1, b = 0: an integer matmul, exact in fp32 at this size
    rng = np.random.default_rng(8)
    E, N, K = 2, 16, 128
    w = rng.integers(0, 2**32, size=(E, N, K // 8), dtype=np.uint64).astype(np.uint32)
    s = np.full((E, N, K // 64), to_bf16([1.0])[0], np.uint16)
    b = np.zeros_like(s)
    q = W.HostQWeight(w, s, b, E, N, K, 64, 4)
    xi = rng.integers(-3, 4, size=(3, 1, K))
    got = O.gather_qmm(to_bf16(xi.astype(np.float32)), q, None, np.array([1, 0, 1], np.uint32), 1)
    ref = np.stack([np_dequant(w[e], s[e], b[e], K, 64, 4) @ xi[i, 0] for i, e in enumerate([1, 0, 1])])
    np.testing.assert_array_equal(bf16(got[:, 0]), bf16(to_bf16(ref)))


def test_gather_qmm_lhs_and_m():
    q = _qw(4, 64, 256, 4, seed=9)
    x = W.normal_bf16(3, 100, 5 * 2 * 256, 1.0).reshape(5, 2, 256)
    lhs = np.array([4, 0, 0, 2], np.uint32)
    rhs = np.array([1, 3, 1, 0], np.uint32)
    got = O.gather_qmm(x, q, lhs, rhs, 2)
    for b in range(4):
        d = np_dequant(q.w[rhs[b]], q.scales[rhs[b]], q.biases[rhs[b]], 256, 64, 4)
        for m in range(2):
            assert_close(got[b, m], to_bf16(d @ bf16(x[lhs[b], m]).astype(np.float64)))


def test_gather_qmm_sorted_equals_unsorted():
    q = _qw(8, 64, 256, 4, seed=10)
    x = W.normal_bf16(4, 100, 12 * 256, 1.0).reshape(12, 1, 256)
    rhs = np.random.default_rng(1).integers(0, 8, 12).astype(np.uint32)
    order = np.argsort(rhs, kind="stable")
    a = O.gather_qmm(x, q, None, rhs, 1)
    b = O.gather_qmm(x[order], q, None, rhs[order], 1)
    np.testing.assert_array_equal(a[order], b)


# ---------------------------------------------------------------- swiglu / combine
def test_swiglu_closed_form():
    rng = np.random.default_rng(12)
    g, u = to_bf16(rng.normal(0, 2, 4096)), to_bf16(rng.normal(0, 2, 4096))
    h = O.swiglu(g, u)
    gf, uf = bf16(g).astype(np.float64), bf16(u).astype(np.float64)
    assert_close(h, to_bf16(np_silu(gf) * uf), atol=1e-6, rtol=8e-3)


def test_gptoss_swiglu_closed_form():
    """GPT-OSS's clipped SwiGLU (gptoss.cpp:50-58) against the fp64 closed form, on inputs on both sides
    of -7 and +7 and far beyond, in asymmetric pairs: a swapped argument order, a missing + 1, a clip of
    the gated input from below or a wrong alpha each fail here."""
    edges = np.array([-40.0, -10.0, -7.5, -7.0, -6.9375, -1.0, 0.0, 0.5, 3.0, 6.9375, 7.0, 7.5, 10.0, 40.0])
    xl, xg = np.meshgrid(edges, edges, indexing="ij")
    rng = np.random.default_rng(21)
    xl = np.concatenate([xl.ravel(), rng.normal(0, 6, 4096)])
    xg = np.concatenate([xg.ravel(), rng.normal(0, 6, 4096)])
    a, b = to_bf16(xl), to_bf16(xg)
    h, hf = O.gptoss_swiglu(a, b)
    exact = np_gptoss(bf16(a).astype(np.float64), bf16(b).astype(np.float64))
    # fp32 arithmetic: a few ulp of the result, plus the rounding of exp's argument near the limits
    np.testing.assert_allclose(hf.astype(np.float64), exact, rtol=4e-6, atol=1e-30)
    np.testing.assert_array_equal(h, to_bf16(hf.astype(np.float64)))
    # the roles are not symmetric, so the upstream order gives other values
    swapped = np_gptoss(bf16(b).astype(np.float64), bf16(a).astype(np.float64))
    assert np.abs(swapped - exact).max() > 1.0
    # values the clips fix exactly: x_glu at or above 7 gives 7 sigmoid(11.914) (xl + 1)
    big = O.gptoss_swiglu(to_bf16(np.array([7.0, 100.0, -100.0])), to_bf16(np.array([100.0, 7.0, 9.0])))[1]
    s7 = 7.0 / (1.0 + np.exp(-1.702 * 7.0))
    np.testing.assert_allclose(big, [s7 * 8.0, s7 * 8.0, s7 * -6.0], rtol=4e-6)


def test_gather_qmm_f32x_vs_numpy():
    """gather_qmm on fp32 activations (the reference's promoted relu^2 / GPT-OSS hidden values) against
    the fp64 product, with and without a linear bias; equal to the bf16 path on bf16-exact inputs
    before its output rounding."""
    E, N, K = 4, 64, 256
    q = _qw(E, N, K, 4, 31)
    rng = np.random.default_rng(31)
    x = rng.normal(0, 1, (10, 1, K)).astype(np.float32)
    rhs = rng.integers(0, E, 10).astype(np.uint32)
    y = O.gather_qmm_f32x(x, q, None, rhs)
    for b in range(10):
        wd = np_dequant(q.w[rhs[b]], q.scales[rhs[b]], q.biases[rhs[b]], K, 64, 4)
        ref = wd @ x[b, 0].astype(np.float64)
        mag = np.abs(wd) @ np.abs(x[b, 0]).astype(np.float64)
        assert (np.abs(y[b, 0] - ref) <= 1e-6 * mag + 1e-30).all()
    xb = to_bf16(x)
    np.testing.assert_array_equal(O.gather_qmm(xb, q, None, rhs),
                                  to_bf16(O.gather_qmm_f32x(bf16(xb), q, None, rhs).astype(np.float64)))
    q.linear_bias = to_bf16(rng.normal(0, 1, (E, N)))
    yb = O.gather_qmm_f32x(x, q, None, rhs)
    np.testing.assert_array_equal(yb, y + bf16(q.linear_bias)[rhs][:, None, :])


def test_combine_linear_in_scores():
    rng = np.random.default_rng(13)
    T, k, H = 7, 4, 256
    Y = to_bf16(rng.normal(0, 1, (T * k, H)))
    s1 = rng.uniform(0, 1, (T, k)).astype(np.float32)
    ref = np.einsum("tk,tkh->th", s1.astype(np.float64), bf16(Y).reshape(T, k, H).astype(np.float64))
    assert_close(O.combine(Y, s1), to_bf16(ref), atol=1e-6, rtol=8e-3)
    # order invariance over the k slots
    perm = rng.permutation(k)
    Yp = Y.reshape(T, k, H)[:, perm].reshape(T * k, H)
    assert_close(O.combine(Yp, s1[:, perm]), O.combine(Y, s1), atol=1e-6, rtol=8e-3)


# ---------------------------------------------------------------- whole block
@pytest.fixture(scope="module")
def tiny():
    return W.make_layer(W.CONFIGS["tiny"])


def test_block_tiny_vs_numpy(tiny):
    x = W.make_tokens(tiny.cfg, 16)
    out, logits, inds, scores = O.block_forward(tiny, x)
    ref = np_block(tiny, x, inds.astype(np.int64), scores.astype(np.float64))
    assert_close(out, to_bf16(ref), what="tiny block")
    # routing from the numpy logits agrees (no near-ties at this seed)
    lf = bf16(x).astype(np.float64) @ bf16(tiny.router_weight).astype(np.float64).T
    np.testing.assert_array_equal(np.sort(inds, 1), np.sort(np_topk(bf16(to_bf16(lf)), 2), 1))


@pytest.mark.parametrize("name", ["qwen3_next_80b"])
def test_block_shared_expert_vs_numpy(name):
    cfg = W.CONFIGS[name]
    small = W.MoeConfig(**{**cfg.__dict__, "num_experts": 16, "top_k": 4, "hidden": 256,
                           "intermediate": 128, "shared_intermediate": 128})
    layer = W.make_layer(small)
    x = W.make_tokens(small, 5)
    out, _, inds, scores = O.block_forward(layer, x)
    ref = np_block(layer, x, inds.astype(np.int64), scores.astype(np.float64))
    assert_close(out, to_bf16(ref), what="shared expert block")


def test_block_quantized_shared_gate_vs_numpy():
    """Qwen3-Next's sigmoid gate quantized (8-bit, as MLX conversions store it): linear_forward's
    quantized branch (qwen3_next.cpp:488) against the fp64 restatement with the dequantized gate."""
    cfg = W.CONFIGS["qwen3_next_80b"]
    small = W.MoeConfig(**{**cfg.__dict__, "num_experts": 16, "top_k": 4, "hidden": 256,
                           "intermediate": 128, "shared_intermediate": 128})
    layer = W.make_layer(small, shared_gate_bits=8)
    x = W.make_tokens(small, 6)
    out, _, inds, scores = O.block_forward(layer, x)
    ref = np_block(layer, x, inds.astype(np.int64), scores.astype(np.float64))
    assert_close(out, to_bf16(ref), what="quantized shared gate block")
    dense = W.make_layer(small)
    assert (O.moe_experts(dense, x, inds, scores) != out).any()  # the quantized gate is the one applied


def test_block_deepseek_style_small_vs_numpy():
    cfg = W.CONFIGS["deepseek_v3"]
    small = W.MoeConfig(**{**cfg.__dict__, "num_experts": 32, "hidden": 256, "intermediate": 128,
                           "shared_intermediate": 128})
    layer = W.make_layer(small)
    x = W.make_tokens(small, 6)
    out, _, inds, scores = O.block_forward(layer, x)
    ref = np_block(layer, x, inds.astype(np.int64), scores.astype(np.float64))
    assert_close(out, to_bf16(ref), what="deepseek-style block")


def test_block_biased_vs_numpy():
    """A GPT-OSS-style block (gptoss.cpp:129-168): router with a bias, top-k of the logits with softmax
    over the k, gate/up/down SwitchLinears with biases, weighted combine -- against the fp64
    restatement."""
    cfg = W.MoeConfig("gptoss_small", 50, 256, 256, 16, 4, O.R_SOFTMAX_TOPK, False, 4)
    layer = W.make_layer(cfg, linear_bias=True)
    x = W.make_tokens(cfg, 8)
    out, logits, inds, scores = O.block_forward(layer, x)
    np.testing.assert_array_equal(logits, O.router_logits(x, layer.router_weight, layer.router_bias))
    ref = np_block(layer, x, inds.astype(np.int64), scores.astype(np.float64))
    assert_close(out, to_bf16(ref), what="biased block")
    lb = layer.gate.linear_bias
    layer.gate.linear_bias = None
    assert (O.moe_experts(layer, x, inds, scores) != out).any()  # the biases are applied
    layer.gate.linear_bias = lb


def test_block_gptoss_activation_vs_numpy():
    """GPT-OSS's expert MLP (gptoss.cpp:141-167): SwitchLinear biases, and the clipped SwiGLU called as
    swiglu(x_gate, x_up) (:158).  Gate and up biases ~ N(0, 4) put a good share of the activation's
    inputs past its limits.  Both oracle modes -- h kept in fp32 (the reference's promotion) and h
    rounded to bf16 (the device's storage) -- agree with the fp64 restatement; the standard SwiGLU and
    the upstream argument order each give a different block."""
    base = W.MoeConfig("gptoss_small", 50, 256, 256, 16, 4, O.R_SOFTMAX_TOPK, False, 4)
    cfg = W.MoeConfig(**{**base.__dict__, "activation": O.ACT_GPTOSS})
    layer = W.make_layer(cfg, linear_bias=True, glu_bias_std=4.0)
    x = W.make_tokens(cfg, 8)
    out, _, inds, scores = O.block_forward(layer, x, hidden_f32=True)
    ref = np_block(layer, x, inds.astype(np.int64), scores.astype(np.float64))
    assert_close(out, to_bf16(ref), what="gpt-oss block (fp32 h)")
    # the bf16 rounding points of g, u and h move an output by at most h_rounding_mag (first order)
    out_b, terms = O.moe_experts(layer, x, inds, scores, with_terms=True)
    D = h_rounding_mag(O, layer, x, inds, scores)
    assert_close_block(out_b, to_bf16(ref), terms, what="gpt-oss block (bf16 h)", strict_frac=0.01, extra=D)
    # the clip limits are exercised
    xf = bf16(x).astype(np.float64)
    g = np.array([np_dequant(layer.gate.w[e], layer.gate.scales[e], layer.gate.biases[e], 256, 64, 4) @ xf[t]
                  + bf16(layer.gate.linear_bias[e]) for t in range(8) for e in inds[t]])
    u = np.array([np_dequant(layer.up.w[e], layer.up.scales[e], layer.up.biases[e], 256, 64, 4) @ xf[t]
                  + bf16(layer.up.linear_bias[e]) for t in range(8) for e in inds[t]])
    assert ((np.abs(g) > 7) | (u > 7)).mean() > 0.05
    assert ((np.abs(g) < 7) & (u < 7)).mean() > 0.5
    for other in (O.ACT_SWIGLU, O.ACT_GPTOSS_UPSTREAM):
        layer.cfg = W.MoeConfig(**{**base.__dict__, "activation": other})
        alt = bf16(O.moe_experts(layer, x, inds, scores)).astype(np.float64)
        assert (np.abs(alt - bf16(out)) > 2e-2 + 1e-2 * np.abs(bf16(out))).mean() > 0.1
        if other == O.ACT_GPTOSS_UPSTREAM:
            assert_close(to_bf16(alt), to_bf16(np_block(layer, x, inds.astype(np.int64),
                                                        scores.astype(np.float64))), what="upstream roles")


def test_block_linear_in_scores(tiny):
    x = W.make_tokens(tiny.cfg, 4)
    _, _, inds, scores = O.block_forward(tiny, x)
    a = bf16(O.moe_experts(tiny, x, inds, scores)).astype(np.float64)
    b = bf16(O.moe_experts(tiny, x, inds, scores * 0.5)).astype(np.float64)
    np.testing.assert_allclose(b, 0.5 * a, rtol=1e-2, atol=1e-3)


def test_block_quantized_router_vs_numpy():
    """The quantized router branch (linear_forward's quantized_matmul, quantized_linear.h:73-96, taken
    for an 8-bit mlp.gate, examples/convert.cpp:56-60): logits = bf16(x . dequant(Wq)^T) against a
    float64 product of the unpacked codes; routing and experts then follow those logits."""
    cfg = W.CONFIGS["tiny"]
    layer = W.make_layer(cfg, router_bits=8)
    T, K, E, k = 16, cfg.hidden, cfg.num_experts, cfg.top_k
    x = W.make_tokens(cfg, T)
    out, logits, inds, scores = O.block_forward(layer, x)
    rq = layer.router_q
    wd = np_dequant(rq.w, rq.scales, rq.biases, K, 64, 8)
    xf = bf16(x).astype(np.float64)
    exact, mag = xf @ wd.T, np.abs(xf) @ np.abs(wd).T
    ulp = np.spacing(np.abs(exact).astype(np.float32)).astype(np.float64) * 65536.0
    d = np.abs(bf16(logits).astype(np.float64) - exact)
    assert (d <= ulp + 8.0 * np.sqrt(K) * 2.0**-24 * mag).all(), d.max()
    assert (logits != O.router_logits(x, layer.router_weight)).any()  # not the bf16 router's logits
    ri, rs, _ = O.route(logits, O.make_router(cfg.variant, E, k, cfg.norm_topk_prob))
    np.testing.assert_array_equal(inds, ri)
    np.testing.assert_array_equal(scores.view(np.uint32), rs.view(np.uint32))
    np.testing.assert_array_equal(out, O.moe_experts(layer, x, inds, scores))


def test_add_rms_norm_vs_numpy():
    """add_rms_norm (gated_delta.cpp:313-345): the sum is the fp32 add rounded to bf16 exactly; the
    normalised row is within an ulp of the float64 formula on the rounded sums."""
    rng = np.random.default_rng(11)
    T, H, eps = 6, 2048, 1e-6
    a, b = to_bf16(rng.normal(0, 1, (T, H))), to_bf16(rng.normal(0, 0.5, (T, H)))
    w = to_bf16(rng.normal(1, 0.1, H))
    s, n = O.add_rms_norm(a, b, w, eps)
    sf = bf16(a).astype(np.float64) + bf16(b).astype(np.float64)  # exact
    np.testing.assert_array_equal(s, to_bf16(sf))
    ref = bf16(s).astype(np.float64) / np.sqrt((sf ** 2).mean(1, keepdims=True) + eps) * bf16(w)
    assert_close(n, to_bf16(ref), atol=1e-6, rtol=2.0**-7, what="normed")


def test_add_rms_norm_closed_forms():
    """Constant rows c (a power of two) normalise to sign(c) w exactly with eps = 0 (pins the mean over
    H, the square root and the weight); eps = 3 c^2 halves them (pins eps); scaling a row by 2^k
    changes nothing (the norm uses the same sums it divides)."""
    H = 8
    w = to_bf16(np.linspace(0.5, 2.0, H))
    for c in (2.0, -0.25):
        a = to_bf16(np.full((1, H), c))
        z = to_bf16(np.zeros((1, H)))
        _, n = O.add_rms_norm(a, z, w, 0.0)
        np.testing.assert_array_equal(bf16(n)[0], np.sign(c) * bf16(w))
        _, n = O.add_rms_norm(a, z, w, 3 * c * c)
        np.testing.assert_array_equal(bf16(n)[0], np.sign(c) * bf16(w) / 2)
    rng = np.random.default_rng(3)
    a, b = to_bf16(rng.normal(0, 1, (4, 64))), to_bf16(rng.normal(0, 1, (4, 64)))
    w64 = to_bf16(rng.normal(1, 0.2, 64))
    _, n1 = O.add_rms_norm(a, b, w64, 0.0)
    _, n2 = O.add_rms_norm(to_bf16(bf16(a) * 8.0), to_bf16(bf16(b) * 8.0), w64, 0.0)
    np.testing.assert_array_equal(n1, n2)
