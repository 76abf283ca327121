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


def logits_bound(x_bf16, w_bf16):
    """Allowed |a - b| between two bf16 roundings of fp32 dot products summed in
    different orders: one bf16 ulp of the result plus 8*sqrt(K)*2^-24 times the
    sum of |products| (fp32 accumulation noise; matters where terms cancel)."""
    xf = bf16(x_bf16).astype(np.float64)
    wf = bf16(w_bf16).astype(np.float64)
    exact = xf @ wf.T
    mag = np.abs(xf) @ np.abs(wf).T
    K = xf.shape[1]
    ulp = np.spacing(np.abs(exact).astype(np.float32)).astype(np.float64) * 65536.0
    return exact, ulp + 8.0 * np.sqrt(K) * 2.0**-24 * mag


def assert_logits_close(got_bf16, ref_bf16, x_bf16, w_bf16):
    _, bound = logits_bound(x_bf16, w_bf16)
    d = np.abs(bf16(got_bf16).astype(np.float64) - bf16(ref_bf16).astype(np.float64))
    assert (d <= bound).all(), f"logits differ by {d.max():.3g} (bound {bound[d.argmax() // d.shape[1]].min():.3g})"
    return int((d > 0).sum())


def assert_close_block(got_bf16, ref_bf16, term_mag, what="block output", strict_frac=1e-4):
    """Block outputs: the benchmark tolerance |a-b| <= ATOL + RTOL*|b| must hold
    on all but a fraction `strict_frac` of elements, and every element must lie
    within that bound plus one bf16 ulp (2^-8 relative) of the magnitude of the
    bf16-rounded terms the output sums (expert outputs Y times their weights,
    the shared-expert output).  The reference rounds those intermediates to
    bf16 (each op's output dtype), so two correct implementations whose fp32
    sums straddle a rounding boundary differ by up to one such ulp; where the
    terms cancel, that exceeds the bound taken relative to the output."""
    g = bf16(got_bf16).astype(np.float64)
    r = bf16(ref_bf16).astype(np.float64)
    err = np.abs(g - r)
    strict = err <= ATOL + RTOL * np.abs(r)
    nbad = int((~strict).sum())
    assert nbad <= strict_frac * err.size, f"{what}: {nbad} of {err.size} outside the strict tolerance"
    loose = err <= ATOL + RTOL * np.abs(r) + 2.0**-8 * np.asarray(term_mag, np.float64)
    assert loose.all(), f"{what}: {int((~loose).sum())} elements outside the rounding-aware bound"
    return float(err.max()), nbad
