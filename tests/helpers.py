"""Shared helpers of the GPU parity tests: model/scene construction on both
sides (device for libnerf.so, host arrays for the oracle) and the tolerance
rules stated by the parity contract."""
from __future__ import annotations

import ctypes as C

import numpy as np

from nerf_amd import _lib as L, ext
from nerf_amd.device import DeviceArray, synchronize
from oracle import oracle as orc

# MLP outputs and RGB: within 1e-3 relative.  Relative error is measured
# against max(|want|, floor) with floor = 10% of the RMS of the compared array
# (at least 1e-6): an output that crosses zero has no meaningful relative
# error, and the fp16 rounding of hidden activations perturbs every output by
# an amount proportional to the output scale, not to the output itself.
RTOL = 1e-3
FLOOR_FRAC = 0.1


def assert_rel(got, want, rtol=RTOL, floor=None, what=""):
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    assert got.shape == want.shape, (got.shape, want.shape)
    assert np.isfinite(got).all(), f"{what}: non-finite GPU output"
    if floor is None:
        floor = max(FLOOR_FRAC * float(np.sqrt(np.mean(want ** 2))), 1e-6)
    err = np.abs(got - want) / np.maximum(np.abs(want), floor)
    worst = np.unravel_index(np.argmax(err), err.shape)
    assert err.max() <= rtol, f"{what}: max rel err {err.max():.3e} at {worst}: got {got[worst]!r} want {want[worst]!r}"
    return float(err.max())


def oracle_grid(desc: L.NerfExtGridDesc) -> orc.OrcGrid:
    return orc.make_grid(desc.n_levels, desc.log2_table_size, desc.table_dtype, base=desc.base_resolution, scale=desc.per_level_scale, finest=desc.finest_resolution)


def host_table(model: ext.Model) -> np.ndarray:
    """The table as the oracle reads it: f32 values or f16 bit patterns."""
    t = model.table.numpy()
    return t if t.dtype == np.float32 else t.view(np.uint16)


def host_params(model: ext.Model):
    return model.density.numpy().view(np.uint16), model.color.numpy().view(np.uint16)


def points(n: int, seed: int = 0) -> np.ndarray:
    """n points uniform in [0,1]^3 from the splitmix64 stream (0x9017, seed)."""
    return orc.uniform_fill(0x9017, seed, 3 * n, 0.0, 1.0).reshape(n, 3)


def unit_dirs(n: int, seed: int = 0) -> np.ndarray:
    rng = np.random.default_rng(seed)
    d = rng.normal(size=(n, 3))
    return (d / np.linalg.norm(d, axis=1, keepdims=True)).astype(np.float32)


def byref(x):
    return C.byref(x)


__all__ = ["L", "ext", "orc", "DeviceArray", "synchronize", "assert_rel", "oracle_grid", "host_table", "host_params", "points", "unit_dirs", "byref"]
