"""Committed end-to-end goldens of the tiny configurations (tests/golden/*.npz, written by
tests/golden/make_golden.py from the CPU checker).

CPU: the seeded generator reproduces the fixture's inputs (SHA-256 of weights and tokens) and
the checker reproduces every stored output bit for bit -- a change to either shows up here
instead of moving the checker and the checked together.
GPU: the device block on the fixture's inputs -- logits within the rounding-order bound; routing,
perm, inv_perm and offsets equal to the fixture (bit-exact; a token whose logits differ may
differ only at a near tie); outputs within the benchmark tolerance of the fixture."""
from pathlib import Path

import numpy as np
import pytest

from helpers import assert_close_block, assert_logits_close, load_pkg, routing_near_ties

moe = load_pkg()
from lemon_mlx_engine_amd import workloads as W  # noqa: E402
from oracle import moe_oracle as O  # noqa: E402

GOLDEN = Path(__file__).resolve().parent / "golden"
import sys  # noqa: E402

sys.path.insert(0, str(GOLDEN))
import make_golden as MG  # noqa: E402

NAMES = sorted(MG.GOLDENS)


def load(name):
    with np.load(GOLDEN / f"{name}.npz", allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


@pytest.mark.parametrize("name", NAMES)
def test_generator_reproduces_inputs(name):
    g = load(name)
    cfg, T = MG.GOLDENS[name]
    layer, x = W.make_layer(cfg), W.make_tokens(cfg, T)
    assert int(g["T"]) == T
    np.testing.assert_array_equal(x, g["x"])
    assert MG.layer_hash(layer, x) == str(g["sha256"]), f"{name}: generated weights changed"


@pytest.mark.parametrize("name", NAMES)
def test_checker_reproduces_golden(name):
    g = load(name)
    cfg, T = MG.GOLDENS[name]
    got = MG.make(name)
    for key in ("logits", "inds", "perm", "inv_perm", "offsets", "out"):
        np.testing.assert_array_equal(got[key], g[key], err_msg=f"{name}: {key}")
    np.testing.assert_array_equal(got["scores"].view(np.uint32), g["scores"].view(np.uint32))
    np.testing.assert_array_equal(got["term_mag"].view(np.uint32), g["term_mag"].view(np.uint32))
    assert g["offsets"][-1] == T * cfg.top_k


@pytest.mark.gpu
@pytest.mark.parametrize("name", NAMES)
def test_device_matches_golden(name):
    torch = pytest.importorskip("torch")
    g = load(name)
    cfg, T = MG.GOLDENS[name]
    layer = W.make_layer(cfg)
    blk = moe.MoeBlock.from_host(layer, "cuda:0")
    xd = torch.from_numpy(g["x"].view(np.int16)).to("cuda:0").view(torch.bfloat16)
    out, aux = blk.forward(xd, return_aux=True)
    torch.cuda.synchronize()

    def h(t):
        return t.view(torch.int16).cpu().numpy().view(np.uint16)

    logits, inds = h(aux["logits"]), aux["inds"].cpu().numpy().astype(np.uint32)
    scores = aux["scores"].cpu().numpy()
    assert_logits_close(logits, g["logits"], g["x"], layer.router_weight)
    same = (inds == g["inds"]).all(1)
    nroute, _ = routing_near_ties(O, cfg, g["x"], layer.router_weight, logits, inds, layer.score_bias)
    assert nroute == int((~same).sum())
    np.testing.assert_array_equal(scores[same].view(np.uint32), g["scores"][same].view(np.uint32))
    if same.all():
        np.testing.assert_array_equal(aux["perm"].cpu().numpy(), g["perm"])
        np.testing.assert_array_equal(aux["inv_perm"].cpu().numpy(), g["inv_perm"])
        np.testing.assert_array_equal(aux["offsets"].cpu().numpy(), g["offsets"])
    assert_close_block(h(out)[same], g["out"][same], g["term_mag"][same], what=f"golden {name}")
    print(f"golden {name}: routing identical on {same.sum()} of {T} tokens")
