"""The C++ host classes (lemon-mlx-engine_amd/host/switch_layers.hpp: SwitchLinear,
SwitchGLU, gather_sort, scatter_unsort, moe_route, QuantizedWeightRegistry) through
their C++ test program tests/cpp/test_switch_layers.cpp (built by
__graft_entry__.build() / `make -C tests/cpp`).

`cpu`: interface checks that touch no device.  `gpu`: forward passes of the
reference's two call patterns (Qwen3-MoE's SwitchGLU, GPT-OSS's SwitchLinear with
linear biases and gather_sort / scatter_unsort) against the CPU checker."""
import subprocess

import pytest

from helpers import ROOT

BIN = ROOT / "tests" / "cpp" / "build" / "test_switch_layers"


def _run(group: str, timeout: int) -> None:
    if not BIN.exists():
        pytest.fail(f"{BIN} is missing: build it with __graft_entry__.build() (make -C tests/cpp)")
    r = subprocess.run([str(BIN), group], stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True,
                       timeout=timeout)
    print(r.stdout)
    assert r.returncode == 0, r.stdout[-4000:]


def test_host_classes_cpu():
    _run("cpu", 60)


@pytest.mark.gpu
def test_host_classes_gpu():
    _run("gpu", 110)
