"""The C++ host classes (lemon-mlx-engine_amd/host/switch_layers.hpp: SwitchLinear,
SwitchGLU, gather_sort, scatter_unsort, moe_route, QuantizedWeightRegistry) through
their C++ test program tests/cpp/test_switch_layers.cpp (built by
__graft_entry__.build() / `make -C tests/cpp`).

`cpu`: interface checks that touch no device.  `gpu`: forward passes of the
reference's two call patterns (Qwen3-MoE's SwitchGLU, GPT-OSS's SwitchLinear with
linear biases and gather_sort / scatter_unsort) against the CPU checker.

The checkpoint reader behind the host classes (host/safetensors.hpp,
host/quantize_utils.hpp): its tensors (name, dtype, shape, CRC-32 of the bytes)
against the `safetensors` package's numpy loader on files that package wrote; its
MoE sanitize against numpy stacks of the per-expert arrays; and, on the GPU, a
checkpoint directory loaded into the C++ SwitchGLU (read, sanitize, upload,
register_quantized_weights, load_weights) run against the CPU checker on the
weights that were written.

The CPU cases run twice: with the regular build and with
build/test_switch_layers_asan (`make -C tests/cpp asan`), in which the host
classes, the readers, the host data formats and the C ABI's host side are
compiled with AddressSanitizer and UndefinedBehaviorSanitizer; a sanitizer
report fails the test."""
import json
import os
import subprocess
import zlib

import numpy as np
import pytest

from helpers import ROOT, load_pkg
from oracle import moe_oracle as O

BIN = ROOT / "tests" / "cpp" / "build" / "test_switch_layers"
ASAN_BIN = ROOT / "tests" / "cpp" / "build" / "test_switch_layers_asan"
# leak checking is off: the HIP runtime keeps process-lifetime allocations
_SAN_ENV = {"ASAN_OPTIONS": "detect_leaks=0:abort_on_error=0", "UBSAN_OPTIONS": "halt_on_error=1:print_stacktrace=1"}


def _run(group: str, timeout: int, *args, binary=BIN) -> str:
    if not binary.exists():
        pytest.fail(f"{binary} is missing: build it with __graft_entry__.build() (make -C tests/cpp all asan)")
    env = dict(os.environ, **_SAN_ENV) if binary == ASAN_BIN else None
    r = subprocess.run([str(binary), group, *map(str, args)], stdout=subprocess.PIPE, stderr=subprocess.STDOUT,
                       text=True, timeout=timeout, env=env)
    print(r.stdout[-4000:])
    assert r.returncode == 0, r.stdout[-4000:]
    assert "AddressSanitizer" not in r.stdout and "runtime error:" not in r.stdout, r.stdout[-4000:]
    return r.stdout


def _dump(directory, sanitize=False, binary=BIN) -> dict:
    out = _run("dump", 60, directory, *(["sanitize"] if sanitize else []), binary=binary)
    rows = {}
    for line in out.splitlines():
        name, dt, shape, crc = line.split("\t")
        rows[name] = (dt, tuple(int(v) for v in shape.split(",")) if shape else (), int(crc, 16))
    return rows


def test_host_classes_cpu():
    _run("cpu", 60)


def test_host_classes_cpu_sanitized():
    """The CPU cases under AddressSanitizer + UndefinedBehaviorSanitizer; the binary is instrumented."""
    syms = subprocess.run(["nm", str(ASAN_BIN)], stdout=subprocess.PIPE, text=True).stdout if ASAN_BIN.exists() else ""
    assert "__asan_report_load" in syms and "__ubsan_handle_" in syms, "sanitized test binary is not instrumented"
    _run("cpu", 120, binary=ASAN_BIN)


@pytest.mark.gpu
def test_host_classes_gpu():
    _run("gpu", 110)


_NP_TO_ST = {np.dtype(np.float32): "F32", np.dtype(np.float16): "F16", np.dtype(np.float64): "F64",
             np.dtype(np.uint8): "U8", np.dtype(np.int8): "I8", np.dtype(np.uint16): "U16",
             np.dtype(np.int16): "I16", np.dtype(np.uint32): "U32", np.dtype(np.int32): "I32",
             np.dtype(np.uint64): "U64", np.dtype(np.int64): "I64", np.dtype(np.bool_): "BOOL"}


@pytest.mark.parametrize("binary", [BIN, ASAN_BIN], ids=["plain", "sanitized"])
def test_reader_matches_safetensors_package(tmp_path, binary):
    """Files written by the safetensors package (two shards behind an index, every numpy dtype it
    writes, a 0-d and an empty tensor, metadata) read by the C++ reader: the same names, dtypes,
    shapes and bytes as safetensors.numpy.load_file gives."""
    st = pytest.importorskip("safetensors.numpy")
    rng = np.random.default_rng(5)
    shard1 = {f"t_{np.dtype(d).name}": (rng.standard_normal((3, 5, 7)) * 100).astype(d)
              for d in _NP_TO_ST if d != np.dtype(np.bool_)}
    shard1["t_bool"] = rng.standard_normal((4, 9)) > 0
    shard2 = {"scalar": np.array(3.5, np.float32), "empty": np.zeros((0, 4), np.int32),
              "model.layers.0.mlp.switch_mlp.up_proj.weight": rng.integers(0, 2**32, (4, 16, 8), np.uint32)}
    st.save_file(shard1, str(tmp_path / "a.safetensors"), metadata={"format": "mlx"})
    st.save_file(shard2, str(tmp_path / "b.safetensors"))
    wm = {n: "a.safetensors" for n in shard1}
    wm.update({n: "b.safetensors" for n in shard2})
    (tmp_path / "model.safetensors.index.json").write_text(json.dumps({"weight_map": wm}))
    want = {}
    for f in ("a.safetensors", "b.safetensors"):
        for n, a in st.load_file(str(tmp_path / f)).items():
            want[n] = (_NP_TO_ST[a.dtype], tuple(a.shape), zlib.crc32(np.ascontiguousarray(a).tobytes()))
    assert _dump(tmp_path, binary=binary) == want


@pytest.mark.parametrize("binary", [BIN, ASAN_BIN], ids=["plain", "sanitized"])
def test_sanitize_matches_numpy_stack(tmp_path, binary):
    """The C++ MoE sanitize (DeepSeek-V3 per-expert naming) against numpy stacks of the arrays written."""
    load_pkg()
    from lemon_mlx_engine_amd import workloads as W
    from test_checkpoint import DS_SMALL, deepseek_config, deepseek_tensors, small, write_safetensors

    cfg = small("deepseek_v3", **DS_SMALL)
    layer = W.make_layer(cfg)
    write_safetensors(tmp_path / "model.safetensors", deepseek_tensors(1, layer))
    (tmp_path / "config.json").write_text(json.dumps(deepseek_config(cfg)))
    rows = _dump(tmp_path, sanitize=True, binary=binary)
    p = "model.layers.1.mlp.switch_mlp"
    for proj, q in (("gate_proj", layer.gate), ("up_proj", layer.up), ("down_proj", layer.down)):
        for suffix, dt, a in (("weight", "U32", q.w), ("scales", "BF16", q.scales), ("biases", "BF16", q.biases)):
            assert rows[f"{p}.{proj}.{suffix}"] == (dt, a.shape, zlib.crc32(np.ascontiguousarray(a).tobytes()))
    assert not any(".experts." in n for n in rows)
    assert rows["model.layers.1.mlp.gate.e_score_correction_bias"][:2] == ("F32", (cfg.num_experts,))


def _glu_case(tmp_path, cfg, layer, tensors, config, li, T, seed):
    from test_checkpoint import write_safetensors
    from lemon_mlx_engine_amd import workloads as W

    names = sorted(tensors)
    half = len(names) // 2
    write_safetensors(tmp_path / "s1.safetensors", {n: tensors[n] for n in names[:half]})
    write_safetensors(tmp_path / "s2.safetensors", {n: tensors[n] for n in names[half:]})
    wm = {n: ("s1" if i < half else "s2") + ".safetensors" for i, n in enumerate(names)}
    (tmp_path / "model.safetensors.index.json").write_text(json.dumps({"weight_map": wm}))
    (tmp_path / "model.safetensors").write_bytes(b"\x02\0\0\0\0\0\0\0{}")  # a stub the index overrides
    (tmp_path / "config.json").write_text(json.dumps(config))
    k, E = cfg.top_k, cfg.num_experts
    x = W.make_tokens(cfg, T)
    rng = np.random.default_rng(seed)
    inds = np.stack([rng.permutation(E)[:k] for _ in range(T)]).astype(np.uint32)
    (tmp_path / "in.bin").write_bytes(np.array([T, k], np.int32).tobytes() + x.tobytes() + inds.tobytes())
    _run("load-glu", 110, tmp_path, li, tmp_path / "in.bin", tmp_path / "out.bin")
    y = np.fromfile(tmp_path / "out.bin", np.uint16).reshape(T, k, cfg.hidden)
    lhs = np.repeat(np.arange(T, dtype=np.uint32), k)
    g = O.gather_qmm(x, layer.gate, lhs, inds.ravel())  # (with the layer's SwitchLinear biases, if any)
    u = O.gather_qmm(x, layer.up, lhs, inds.ravel())
    h = O.gptoss_swiglu(g, u)[0] if cfg.activation == O.ACT_GPTOSS else O.swiglu(g, u)
    ref = O.gather_qmm(h.reshape(T * k, -1), layer.down, None, inds.ravel()).reshape(T, k, -1)
    a, b = O.bf16_to_f32(y), O.bf16_to_f32(ref)
    bad = np.abs(a - b) > 2e-2 + 1e-2 * np.abs(b)
    assert not bad.any(), f"{int(bad.sum())} of {bad.size} outside |a-b| <= 2e-2 + 1e-2|b|"


@pytest.mark.gpu
@pytest.mark.parametrize("T", [4, 96])
def test_load_glu_deepseek_checkpoint(tmp_path, T):
    """A DeepSeek-V3-named checkpoint (per-expert tensors over two shards, an 8-bit down_proj by the
    override of its stacked name) loaded by the C++ reader into SwitchGLU; outputs against the CPU
    checker on the weights written, within |a-b| <= 2e-2 + 1e-2|b|."""
    load_pkg()
    from lemon_mlx_engine_amd import workloads as W
    from test_checkpoint import DS_SMALL, deepseek_config, deepseek_tensors, small

    cfg = small("deepseek_v3", **{**DS_SMALL, "hidden": 512})
    base = W.make_layer(cfg)
    down8 = W.make_qweight(cfg.seed, 99, cfg.num_experts, cfg.hidden, cfg.intermediate, 0.02, 64, 8)
    layer = W.HostLayer(cfg, base.router_weight, base.gate, base.up, down8, base.score_bias, base.shared)
    q = {"group_size": 64, "bits": 4, "model.layers.1.mlp.switch_mlp.down_proj": {"group_size": 64, "bits": 8}}
    _glu_case(tmp_path, cfg, layer, deepseek_tensors(1, layer), deepseek_config(cfg, quantization=q), 1, T, T)


@pytest.mark.gpu
def test_load_glu_6bit_checkpoint(tmp_path):
    """6-bit experts (examples/convert.cpp:10 --bits 6), DeepSeek-V3 naming, through the C++ reader,
    sanitize and register_quantized_weights into SwitchGLU; outputs against the CPU checker."""
    load_pkg()
    from lemon_mlx_engine_amd import workloads as W
    from test_checkpoint import DS_SMALL, deepseek_config, deepseek_tensors, small

    cfg = small("deepseek_v3", **{**DS_SMALL, "hidden": 512, "bits": 6})
    layer = W.make_layer(cfg)
    _glu_case(tmp_path, cfg, layer, deepseek_tensors(1, layer), deepseek_config(cfg), 1, 40, 6)


@pytest.mark.gpu
def test_load_glu_phimoe_checkpoint(tmp_path):
    """PhiMoE naming (block_sparse_moe, w1/w3/w2), 8-bit experts, through the C++ reader into SwitchGLU."""
    load_pkg()
    from lemon_mlx_engine_amd import workloads as W
    from test_checkpoint import phimoe_tensors, small

    cfg = small("mixtral_8x7b", hidden=256, intermediate=512, num_experts=8, top_k=2)
    layer = W.make_layer(cfg)
    c = {"model_type": "phimoe", "hidden_size": cfg.hidden, "intermediate_size": cfg.intermediate,
         "num_local_experts": cfg.num_experts, "num_experts_per_tok": cfg.top_k,
         "quantization": {"group_size": 64, "bits": 8}}
    _glu_case(tmp_path, cfg, layer, phimoe_tensors(0, layer), c, 0, 24, 3)


@pytest.mark.gpu
@pytest.mark.parametrize("fused", [False, True])
def test_load_glu_qwen35_checkpoint(tmp_path, fused):
    """Qwen3.5-MoE naming (VLM 'language_model.' / 'model.language_model.' names, config under text_config;
    stacked switch_mlp experts or a fused experts.gate_up_proj split at the middle row, qwen35_moe.cpp:
    1046-1160) through the C++ reader, sanitize and register_quantized_weights into SwitchGLU; outputs
    against the CPU checker on the weights written."""
    load_pkg()
    from lemon_mlx_engine_amd import workloads as W
    from test_checkpoint import QN_SMALL, qwen35_config, qwen35_tensors, small

    cfg = small("qwen3_next_80b", **{**QN_SMALL, "hidden": 512})
    layer = W.make_layer(cfg)
    head = "model.language_model" if fused else "language_model.model"
    _glu_case(tmp_path, cfg, layer, qwen35_tensors(4, layer, fused, head), qwen35_config(cfg), 4, 48, 11)


@pytest.mark.gpu
@pytest.mark.parametrize("fused", [False, True])
def test_load_glu_gptoss_checkpoint(tmp_path, fused):
    """GPT-OSS naming (stacked mlp.experts with SwitchLinear biases, or the fused gate_up_proj split
    even/odd with its bias, gptoss.cpp:305-350) through the C++ reader into SwitchGLU(bias=true) with the
    clipped SwiGLU (the per-projection path); outputs against the CPU checker."""
    load_pkg()
    from lemon_mlx_engine_amd import workloads as W
    from test_checkpoint import GPTOSS_SMALL, gptoss_config, gptoss_tensors

    layer = W.make_layer(GPTOSS_SMALL, linear_bias=True, glu_bias_std=4.0)
    _glu_case(tmp_path, GPTOSS_SMALL, layer, gptoss_tensors(0, layer, fused), gptoss_config(GPTOSS_SMALL), 0, 100,
              12)
