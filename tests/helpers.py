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
# against max(|want|, floor) with floor = 10 % of the RMS of the compared
# channel (the last axis of a 2-D or larger array; the whole array when 1-D;
# at least 1e-6): an output that crosses zero has no meaningful relative
# error.  Taking the floor per channel keeps a large channel (the exp
# density, ~1) from loosening the bar on small ones (raw geometry features).
#
# fp16-MLP outputs (mlp=True) take a two-part bar.  Both sides round hidden
# activations to fp16 at the same points, but the GPU accumulates each
# pre-activation in fp32 in MFMA order, so an activation within an fp32
# rounding error of an fp16 tie may round the other way; one such flip moves
# every output of that sample by |W| x ulp_fp16(activation), an error in
# proportion to the channel's scale rather than to the output (with a
# U(-1e-4, 1e-4) table the hidden activations are fp16 subnormals and a
# flip is 6e-8 absolute).  So: every output within 1e-3 relative to
# max(|want|, RMS of the channel), and 99.9 % of outputs within 1e-4 at the
# strict floor above (the bulk, where no flip occurred).
RTOL = 1e-3
FLOOR_FRAC = 0.1


def channel_floor(want: np.ndarray, frac: float = FLOOR_FRAC) -> np.ndarray | float:
    want = np.asarray(want, np.float64)
    if want.ndim <= 1:
        return max(frac * float(np.sqrt(np.mean(want ** 2))) if want.size else 0.0, 1e-6)
    axes = tuple(range(want.ndim - 1))
    return np.maximum(frac * np.sqrt(np.mean(want ** 2, axis=axes)), 1e-6)


MLP_BULK_RTOL = 1e-4


def assert_rel(got, want, rtol=RTOL, floor=None, what="", mlp=False, bulk_rtol=MLP_BULK_RTOL):
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    assert got.shape == want.shape, (got.shape, want.shape)
    assert np.isfinite(got).all(), f"{what}: non-finite GPU output"
    strict = channel_floor(want) if floor is None else floor
    err = np.abs(got - want) / np.maximum(np.abs(want), strict)
    bulk = float(np.quantile(err, 0.999)) if err.size else 0.0
    if mlp:
        assert bulk <= bulk_rtol, f"{what}: 99.9th percentile rel err {bulk:.3e} > {bulk_rtol}"
        err = np.abs(got - want) / np.maximum(np.abs(want), channel_floor(want, 1.0))
    worst = np.unravel_index(np.argmax(err), err.shape)
    print(f"[rel] {what}: max {err.max():.3e} p99.9 {bulk:.3e}", flush=True)
    assert err.max() <= rtol, f"{what}: max rel err {err.max():.3e} at {worst}: got {got[worst]!r} want {want[worst]!r}"
    return float(err.max())


def assert_adam_step(got_w, w0, want_w, what=""):
    """An Adam update against the oracle's: within 1e-5 of the update plus 2
    ulp of the weight (lr decay's powf may differ by an ulp between the
    device and the host's libm, which moves a weight by at most an ulp)."""
    got_w, w0, want_w = (np.asarray(a, np.float32) for a in (got_w, w0, want_w))
    bound = 1e-5 * np.abs(want_w.astype(np.float64) - w0) + 2.0 * np.spacing(np.abs(want_w)).astype(np.float64)
    err = np.abs(got_w.astype(np.float64) - want_w)
    bad = err > bound
    assert not bad.any(), f"{what}: {int(bad.sum())} of {bad.size} weights off, worst {err.max():.3e} (update {np.abs(want_w.astype(np.float64) - w0)[np.argmax(err)]:.3e})"


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
