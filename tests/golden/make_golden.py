"""Writes the committed end-to-end golden fixtures of the tiny configurations.

Each fixture holds, for one small MoE block from the seeded generator: a SHA-256 of
the generated weights and tokens (so a change to the generator or the quantizer shows
up as a hash mismatch), and the CPU checker's outputs on them -- router logits,
top-k indices and weights, the stable expert sort (perm, inv_perm, offsets), the
block output and the magnitude of the bf16-rounded terms each output sums.  The
checker (oracle/) is the only source of these values: the reference's own
arithmetic lives in an MLX fork that is absent here.

    python tests/golden/make_golden.py        # rewrites tests/golden/*.npz

Fixtures are plain .npz (no pickled objects).
"""
import hashlib
import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
ROOT = HERE.parents[1]
sys.path.insert(0, str(ROOT))
sys.path.insert(0, str(ROOT / "tests"))

from helpers import load_pkg  # noqa: E402

load_pkg()
from lemon_mlx_engine_amd import ROUTE_SIGMOID_GROUP, ROUTE_SOFTMAX_TOPK, ROUTE_TOPK_PROBS  # noqa: E402
from lemon_mlx_engine_amd import workloads as W  # noqa: E402
from oracle import moe_oracle as O  # noqa: E402

# name -> (config, T).  "tiny" is the benchmark definition's configs[0] exactly; the others are
# small layers of the Qwen3-Next (probabilities, gated shared expert), Mixtral (softmax over the k,
# 8-bit) and DeepSeek-V3 (sigmoid + bias, group limit, ungated shared expert, scaling) kinds.
GOLDENS = {
    "tiny": (W.CONFIGS["tiny"], 16),
    "tiny_next": (W.MoeConfig("tiny_next", 20, 256, 128, 16, 4, ROUTE_TOPK_PROBS, True, 4,
                              shared_intermediate=128, shared_gated=True), 24),
    "tiny_mixtral": (W.MoeConfig("tiny_mixtral", 30, 256, 512, 8, 2, ROUTE_SOFTMAX_TOPK, False, 8), 12),
    "tiny_deepseek": (W.MoeConfig("tiny_deepseek", 40, 256, 128, 32, 4, ROUTE_SIGMOID_GROUP, True, 4,
                                  n_group=4, topk_group=2, routed_scaling_factor=2.5,
                                  shared_intermediate=128), 20),
}


def layer_hash(layer, x) -> str:
    """SHA-256 over the generated tensors in a fixed order (absent tensors hash as a marker)."""
    h = hashlib.sha256()

    def add(a):
        h.update(b"-" if a is None else np.ascontiguousarray(a).tobytes())

    add(layer.router_weight)
    add(layer.score_bias)
    for q in (layer.gate, layer.up, layer.down):
        add(q.w), add(q.scales), add(q.biases)
    if layer.shared is not None:
        for q in layer.shared[:3]:
            add(q.w), add(q.scales), add(q.biases)
        add(layer.shared[3])
    add(x)
    return h.hexdigest()


def make(name):
    cfg, T = GOLDENS[name]
    layer = W.make_layer(cfg)
    x = W.make_tokens(cfg, T)
    out, logits, inds, scores = O.block_forward(layer, x)
    perm, inv, _, offs = O.bucket(inds, cfg.num_experts)
    _, terms = O.moe_experts(layer, x, inds, scores, with_terms=True)
    return dict(sha256=np.array(layer_hash(layer, x)), T=np.int64(T), x=x, logits=logits, inds=inds,
                scores=scores, perm=perm, inv_perm=inv, offsets=offs, out=out, term_mag=terms)


def main():
    for name in GOLDENS:
        np.savez_compressed(HERE / f"{name}.npz", **make(name))
        print("wrote", HERE / f"{name}.npz")


if __name__ == "__main__":
    main()
