"""The C ABI library on the host: it loads, exports every symbol the header
declares, and rejects bad arguments with the documented status codes before
touching the device.  No GPU needed (no call here launches a kernel)."""
import ctypes
import re

import numpy as np
import pytest

from helpers import ROOT, load_pkg

moe = load_pkg()
L = moe.lib()
HEADER = (ROOT / "include" / "moe_mi355x.h").read_text()
FAKE = 0x10000  # an aligned non-null address; never dereferenced by the host checks


def declared_functions():
    body = re.sub(r"/\*.*?\*/", "", HEADER, flags=re.S)
    return sorted(set(re.findall(r"\b(moe_\w+)\s*\(", body)))


def test_exports_every_declared_symbol():
    names = declared_functions()
    assert len(names) >= 15
    for n in names:
        assert hasattr(L, n), n
        assert n in moe.SIGNATURES, f"{n} missing from the ctypes signature table"
    assert set(moe.SIGNATURES) == set(names)


def test_status_strings():
    assert L.moe_version() >= 1
    for st in (0, -1, -2, -3, -4, -6):
        assert L.moe_status_string(st).decode() not in ("", "unknown status")


def _qw(bits=4, gs=64, E=8, N=64, K=256):
    return moe.QWeightC(FAKE, FAKE, FAKE, E, N, K, gs, bits)


def test_router_logits_validation():
    assert L.moe_router_logits(None, FAKE, None, 4, 256, 8, FAKE, None) == moe.MOE_E_INVALID_ARG
    assert L.moe_router_logits(FAKE, FAKE, None, 4, 250, 8, FAKE, None) == moe.MOE_E_UNSUPPORTED
    assert L.moe_router_logits(FAKE, FAKE, FAKE, 0, 256, 8, FAKE, None) == moe.MOE_OK  # empty: no launch


@pytest.mark.parametrize("params,bias,status", [
    ((1, 8, 9, 1, 1, 1, 1.0), None, moe.MOE_E_INVALID_ARG),     # k > E
    ((1, 8, 0, 1, 1, 1, 1.0), None, moe.MOE_E_INVALID_ARG),     # k = 0
    ((1, 2048, 8, 1, 1, 1, 1.0), None, moe.MOE_E_UNSUPPORTED),  # E > 1024
    ((1, 64, 17, 1, 1, 1, 1.0), None, moe.MOE_E_UNSUPPORTED),   # k > 16
    ((99, 8, 2, 1, 1, 1, 1.0), None, moe.MOE_E_INVALID_ARG),    # unknown variant
    ((6, 256, 8, 1, 8, 4, 2.5), None, moe.MOE_E_INVALID_ARG),   # R6 without bias
    ((6, 250, 8, 1, 8, 4, 2.5), FAKE, moe.MOE_E_UNSUPPORTED),   # E % n_group
    ((6, 256, 8, 1, 8, 9, 2.5), FAKE, moe.MOE_E_INVALID_ARG),   # topk_group > n_group
])
def test_route_validation(params, bias, status):
    p = moe.RouterParams(*params)
    assert L.moe_route(FAKE, bias, 4, ctypes.byref(p), FAKE, FAKE, None) == status


def test_route_empty_is_ok():
    p = moe.RouterParams(1, 8, 2, 1, 1, 1, 1.0)
    assert L.moe_route(FAKE, None, 0, ctypes.byref(p), FAKE, FAKE, None) == moe.MOE_OK


def test_bucket_validation():
    assert L.moe_bucket(FAKE, 4, 2, 2048, FAKE, FAKE, FAKE, FAKE, None, 0, None) == moe.MOE_E_UNSUPPORTED
    assert L.moe_bucket(FAKE, 4, 2, 8, FAKE, FAKE, FAKE, None, None, 0, None) == moe.MOE_E_INVALID_ARG
    assert L.moe_bucket(FAKE, 4, 0, 8, FAKE, FAKE, FAKE, FAKE, None, 0, None) == moe.MOE_E_INVALID_ARG
    # large P needs a workspace
    need = L.moe_bucket_workspace_size(8192, 8, 128)
    assert need > 0
    assert L.moe_bucket(FAKE, 8192, 8, 128, FAKE, FAKE, FAKE, FAKE, FAKE, need - 1, None) == moe.MOE_E_WORKSPACE
    assert L.moe_bucket_workspace_size(1, 8, 128) == 0  # decode sizes need none


@pytest.mark.parametrize("kw,status", [
    (dict(bits=1), moe.MOE_E_UNSUPPORTED),
    (dict(bits=7), moe.MOE_E_UNSUPPORTED),
    (dict(bits=3, K=192), moe.MOE_E_UNSUPPORTED),  # 3 / 5 bits: K a multiple of 128 (whole 16-byte row units)
    (dict(bits=5, K=320), moe.MOE_E_UNSUPPORTED),
    (dict(gs=16), moe.MOE_E_UNSUPPORTED),
    (dict(gs=256), moe.MOE_E_UNSUPPORTED),
    (dict(K=200), moe.MOE_E_UNSUPPORTED),
    (dict(E=0), moe.MOE_E_INVALID_ARG),
])
def test_gather_qmm_validation(kw, status):
    q = _qw(**kw)
    assert L.moe_gather_qmm(FAKE, ctypes.byref(q), None, FAKE, 4, 1, 0, FAKE, FAKE, 1 << 20, None) == status


def test_gather_qmm_workspace_checked():
    q = _qw()
    need = L.moe_gather_qmm_workspace_size(16, 1, 8)
    assert need > 0
    assert L.moe_gather_qmm(FAKE, ctypes.byref(q), None, FAKE, 16, 1, 0, FAKE, FAKE, need - 1,
                            None) == moe.MOE_E_WORKSPACE
    assert L.moe_gather_qmm(FAKE, ctypes.byref(q), None, FAKE, 16, 1, 0, FAKE, None, need,
                            None) == moe.MOE_E_WORKSPACE
    assert L.moe_gather_qmm(FAKE, ctypes.byref(q), None, FAKE, 0, 1, 0, FAKE, None, 0, None) == moe.MOE_OK


def _desc(**over):
    d = moe.BlockDesc()
    H, I, E = 512, 1024, 8
    d.hidden, d.intermediate, d.num_experts = H, I, E
    d.router = moe.RouterParams(1, E, 2, 1, 1, 1, 1.0)
    d.router_weight = FAKE
    d.gate = moe.QWeightC(FAKE, FAKE, FAKE, E, I, H, 64, 4)
    d.up = moe.QWeightC(FAKE, FAKE, FAKE, E, I, H, 64, 4)
    d.down = moe.QWeightC(FAKE, FAKE, FAKE, E, H, I, 64, 4)
    for k, v in over.items():
        setattr(d, k, v)
    return d


def test_block_validation():
    d = _desc()
    need = L.moe_block_workspace_size(ctypes.byref(d), 16)
    assert need > 0
    assert L.moe_block_forward(ctypes.byref(d), FAKE, 16, FAKE, None, FAKE, need - 1, None) == moe.MOE_E_WORKSPACE
    assert L.moe_block_forward(ctypes.byref(d), FAKE, 0, FAKE, None, None, 0, None) == moe.MOE_OK
    bad = _desc(down=moe.QWeightC(FAKE, FAKE, FAKE, 8, 512, 512, 64, 4))  # down K != I
    assert L.moe_block_workspace_size(ctypes.byref(bad), 16) == 0
    assert L.moe_block_forward(ctypes.byref(bad), FAKE, 16, FAKE, None, FAKE, need, None) == moe.MOE_E_INVALID_ARG
    bad = _desc(router=moe.RouterParams(1, 16, 2, 1, 1, 1, 1.0))  # router E != num_experts
    assert L.moe_block_forward(ctypes.byref(bad), FAKE, 16, FAKE, None, FAKE, need, None) == moe.MOE_E_INVALID_ARG
    bad = _desc(shared_intermediate=128)  # shared expert without weights
    assert L.moe_block_forward(ctypes.byref(bad), FAKE, 16, FAKE, None, FAKE, need, None) == moe.MOE_E_INVALID_ARG
    for act in (moe.ACT_GPTOSS, moe.ACT_GPTOSS_UPSTREAM):
        assert L.moe_block_workspace_size(ctypes.byref(_desc(activation=act)), 16) == need
    bad = _desc(activation=7)  # not a moe_activation
    assert L.moe_block_workspace_size(ctypes.byref(bad), 16) == 0
    assert L.moe_block_forward(ctypes.byref(bad), FAKE, 16, FAKE, None, FAKE, need, None) == moe.MOE_E_INVALID_ARG


def test_block_add_norm_validation():
    """moe_block_forward_add_norm: its own arguments (a, b, norm weight, sum and normed outputs, eps) are
    checked first, then everything moe_block_forward checks, all before any launch."""
    d = _desc()
    need = L.moe_block_workspace_size(ctypes.byref(d), 16)
    args = [FAKE, FAKE, FAKE, 1e-6, 16, FAKE, FAKE, FAKE, None, FAKE, need, None]

    def call(desc, a):
        return L.moe_block_forward_add_norm(ctypes.byref(desc) if desc is not None else None, *a)
    for i in (0, 1, 2, 5, 6):  # a, b, norm_weight, sum_out, normed_out
        a = list(args)
        a[i] = None
        assert call(d, a) == moe.MOE_E_INVALID_ARG
    for eps in (-1e-6, float("nan")):
        a = list(args)
        a[3] = eps
        assert call(d, a) == moe.MOE_E_INVALID_ARG
    a = list(args)
    a[10] = need - 1
    assert call(d, a) == moe.MOE_E_WORKSPACE
    assert call(_desc(activation=7), args) == moe.MOE_E_INVALID_ARG
    assert call(None, args) == moe.MOE_E_INVALID_ARG
    a = list(args)
    a[4] = 0
    assert call(d, a) == moe.MOE_OK  # T = 0: nothing to do


def test_quantize_validation():
    w = np.zeros(128, np.uint16)
    out = np.zeros(64, np.uint32)
    s = np.zeros(8, np.uint16)
    vp = lambda a: ctypes.c_void_p(a.ctypes.data)  # noqa: E731
    assert L.moe_quantize_affine(vp(w), 1, 128, 64, 7, vp(out), vp(s), vp(s)) == moe.MOE_E_UNSUPPORTED
    assert L.moe_quantize_affine(vp(w), 1, 128, 64, 3, vp(out), vp(s), vp(s)) == moe.MOE_OK  # 2, 3, 5 bits too
    assert L.moe_quantize_affine(vp(w), 1, 100, 64, 4, vp(out), vp(s), vp(s)) == moe.MOE_E_UNSUPPORTED
    assert L.moe_quantize_affine(None, 1, 128, 64, 4, vp(out), vp(s), vp(s)) == moe.MOE_E_INVALID_ARG
    assert L.moe_synth_normal_bf16(0, 0, 0.0, 1.0, 0, -1, None) == moe.MOE_E_INVALID_ARG


def test_python_wrappers_raise_typed_errors():
    with pytest.raises(moe.MoeArgumentError):
        moe.check(moe.MOE_E_UNSUPPORTED, "x")
    with pytest.raises(moe.MoeError):
        moe.check(moe.MOE_E_WORKSPACE, "x")


def test_take_rows_validation():
    assert L.moe_take_rows(FAKE, 4, FAKE, 3, 0, 16, FAKE, None) == moe.MOE_E_INVALID_ARG  # divisor 0
    assert L.moe_take_rows(FAKE, 4, FAKE, 3, 1, 15, FAKE, None) == moe.MOE_E_INVALID_ARG  # odd row bytes
    assert L.moe_take_rows(None, 4, FAKE, 3, 1, 16, FAKE, None) == moe.MOE_E_INVALID_ARG
    assert L.moe_take_rows(None, 0, None, 0, 1, 16, None, None) == moe.MOE_OK  # empty: no launch


def test_add_expert_bias_validation():
    assert L.moe_add_expert_bias(FAKE, FAKE, FAKE, 4, 0, 8, 2, None) == moe.MOE_E_INVALID_ARG
    assert L.moe_add_expert_bias(None, FAKE, FAKE, 4, 1, 8, 2, None) == moe.MOE_E_INVALID_ARG
    assert L.moe_add_expert_bias(None, None, None, 0, 1, 8, 2, None) == moe.MOE_OK


def test_switch_glu_validation():
    g, u, d = _qw(E=8, N=128, K=256), _qw(E=8, N=128, K=256), _qw(E=8, N=256, K=128)
    R = ctypes.byref
    assert L.moe_switch_glu_workspace_size(R(g), R(d), 16, 2) > 0
    need = L.moe_switch_glu_workspace_size(R(g), R(d), 16, 2)
    assert L.moe_switch_glu(R(g), R(u), R(d), FAKE, FAKE, 16, 2, 0, FAKE, FAKE, need - 1, None) == \
        moe.MOE_E_WORKSPACE
    bad_d = _qw(E=8, N=128, K=128)  # down must map I -> H
    assert L.moe_switch_glu(R(g), R(u), R(bad_d), FAKE, FAKE, 16, 2, 0, FAKE, FAKE, need, None) == \
        moe.MOE_E_INVALID_ARG
    assert L.moe_switch_glu(R(g), R(u), R(d), FAKE, FAKE, 16, 9, 0, FAKE, FAKE, need, None) == moe.MOE_E_INVALID_ARG
    for act in (-1, 3):  # not a moe_activation
        assert L.moe_switch_glu(R(g), R(u), R(d), FAKE, FAKE, 16, 2, act, FAKE, FAKE, need, None) == \
            moe.MOE_E_INVALID_ARG
    assert L.moe_switch_glu(R(g), R(u), R(d), FAKE, FAKE, 0, 2, 0, None, None, 0, None) == moe.MOE_OK


def test_gptoss_swiglu_validation():
    assert L.moe_gptoss_swiglu(None, FAKE, 4, FAKE, None) == moe.MOE_E_INVALID_ARG
    assert L.moe_gptoss_swiglu(FAKE, FAKE, -1, FAKE, None) == moe.MOE_E_INVALID_ARG
    assert L.moe_gptoss_swiglu(None, None, 0, None, None) == moe.MOE_OK


def test_abi_version():
    """The library reports the MOE_ABI_VERSION of the header the binding follows."""
    import re
    hdr = (ROOT / "include" / "moe_mi355x.h").read_text()
    ver = int(re.search(r"#define MOE_ABI_VERSION (\d+)", hdr).group(1))
    assert L.moe_version() == ver == moe.ABI_VERSION


def test_add_rms_norm_validation():
    assert L.moe_add_rms_norm(FAKE, FAKE, FAKE, ctypes.c_float(1e-6), 4, 12, FAKE, FAKE, None) == moe.MOE_E_UNSUPPORTED
    assert L.moe_add_rms_norm(FAKE, FAKE, FAKE, ctypes.c_float(1e-6), 4, 16384, FAKE, FAKE, None) == \
        moe.MOE_E_UNSUPPORTED
    assert L.moe_add_rms_norm(None, FAKE, FAKE, ctypes.c_float(1e-6), 4, 64, FAKE, FAKE, None) == moe.MOE_E_INVALID_ARG
    assert L.moe_add_rms_norm(FAKE, FAKE, FAKE, ctypes.c_float(-1.0), 4, 64, FAKE, FAKE, None) == \
        moe.MOE_E_INVALID_ARG
    assert L.moe_add_rms_norm(FAKE, FAKE, FAKE, ctypes.c_float(1e-6), 0, 64, FAKE, FAKE, None) == moe.MOE_OK


def test_block_graph_validation():
    h = ctypes.c_void_p()
    assert L.moe_block_graph_create(None, FAKE, 1, FAKE, FAKE, 1 << 20, ctypes.byref(h)) == moe.MOE_E_INVALID_ARG
    assert L.moe_block_graph_launch(None, None) == moe.MOE_E_INVALID_ARG
    assert L.moe_block_graph_destroy(None) == moe.MOE_OK


def test_gather_mm_validation():
    ws = moe.lib().moe_gather_mm_workspace_size(4, 1, 8)
    assert ws > 0
    args = dict(x=FAKE, w=FAKE, b=None, E=8, N=64, K=256, lhs=None, rhs=FAKE, batch=4, M=1)

    def call(**kw):
        a = {**args, **kw}
        return L.moe_gather_mm(a["x"], a["w"], a["b"], a["E"], a["N"], a["K"], a["lhs"], a["rhs"], a["batch"], a["M"],
                               0, FAKE, FAKE, ws, None)
    assert call(K=100) == moe.MOE_E_UNSUPPORTED     # K not a multiple of 32
    assert call(w=None) == moe.MOE_E_INVALID_ARG
    assert call(E=0) == moe.MOE_E_INVALID_ARG
    assert call(batch=0) == moe.MOE_OK              # empty: no launch
    assert L.moe_gather_mm(FAKE, FAKE, None, 8, 64, 256, None, FAKE, 4, 1, 0, FAKE, FAKE, 0, None) == \
        moe.MOE_E_WORKSPACE


def test_block_forward_shape_checks_before_launch():
    """MoeBlock.forward / BlockGraph reject an x that is not [T, hidden] and an out whose shape
    differs from x's before any device call (the ABI cannot see buffer sizes); CPU tensors are
    refused as well.  Runs without a GPU: every case raises before the library is called."""
    torch = pytest.importorskip("torch")
    from lemon_mlx_engine_amd import ops
    from lemon_mlx_engine_amd import workloads as W

    cfg = W.CONFIGS["tiny"]
    blk = ops.MoeBlock.from_host(W.make_layer(cfg), "cpu")
    H = cfg.hidden
    bad = [
        (torch.zeros(4, H + 8, dtype=torch.bfloat16), None, "must be \\[T, 512\\]"),
        (torch.zeros(4, 2, H // 2, dtype=torch.bfloat16), None, "must be \\[T, 512\\]"),
        (torch.zeros(4, H, dtype=torch.bfloat16), torch.zeros(3, H, dtype=torch.bfloat16), "out must be"),
        (torch.zeros(4, H, dtype=torch.bfloat16), torch.zeros(4 * H, dtype=torch.bfloat16), "out must be"),
        (torch.zeros(4, H, dtype=torch.bfloat16), None, "device tensor"),
        (torch.zeros(4, H, dtype=torch.float32), None, "device tensor"),
    ]
    for x, out, msg in bad:
        with pytest.raises(ValueError, match=msg):
            blk.forward(x, out)
        with pytest.raises(ValueError, match=msg):
            ops.BlockGraph(blk, x, out if out is not None else torch.zeros_like(x))
