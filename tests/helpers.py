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
        # At most 0.1 % of outputs beyond the strict bar (implied by the bulk
        # bar when bulk_rtol <= rtol; stated so that the count is explicit).
        beyond = float(np.mean(err > rtol))
        assert beyond <= 1e-3, f"{what}: {beyond:.3e} of outputs beyond {rtol} at the strict floor"
        err = np.abs(got - want) / np.maximum(np.abs(want), channel_floor(want, 1.0))
    worst = np.unravel_index(np.argmax(err), err.shape)
    print(f"[rel] {what}: max {err.max():.3e} p99.9 {bulk:.3e}", flush=True)
    assert err.max() <= rtol, f"{what}: max rel err {err.max():.3e} at {worst}: got {got[worst]!r} want {want[worst]!r}"
    return float(err.max())


def assert_rel_rows(got, want, what="", rtol=RTOL, bulk_rtol=MLP_BULK_RTOL, max_row_frac=3e-3):
    """Per-sample rows [n][k] of a backward intermediate whose samples can
    flip a ReLU mask (a hidden activation within an fp32 rounding error of
    zero is masked on one side only, which changes that sample's whole row):
    99.9 % of values within bulk_rtol and at most max_row_frac of the rows
    with any value beyond rtol, both relative to max(|want|, 10 % of the
    column's RMS).  Returns the fraction of such rows."""
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    assert got.shape == want.shape and got.ndim == 2, (got.shape, want.shape)
    assert np.isfinite(got).all(), f"{what}: non-finite GPU output"
    err = np.abs(got - want) / np.maximum(np.abs(want), channel_floor(want))
    bulk = float(np.quantile(err, 0.999))
    bad_rows = float(np.mean(err.max(axis=1) > rtol))
    print(f"[rel] {what}: p99.9 {bulk:.3e}, rows beyond {rtol}: {bad_rows:.2e} (max {err.max():.3e})", flush=True)
    assert bulk <= bulk_rtol, f"{what}: 99.9th percentile rel err {bulk:.3e} > {bulk_rtol}"
    assert bad_rows <= max_row_frac, f"{what}: {bad_rows:.3e} of rows have a value beyond {rtol}"
    return bad_rows


def assert_adam_step(got_w, w0, want_w, what=""):
    """An Adam update against the oracle's: within 1e-5 of the update plus 2
    ulp of the weight (lr decay's powf may differ by an ulp between the
    device and the host's libm, which moves a weight by at most an ulp)."""
    got_w, w0, want_w = (np.asarray(a, np.float32) for a in (got_w, w0, want_w))
    bound = 1e-5 * np.abs(want_w.astype(np.float64) - w0) + 2.0 * np.spacing(np.abs(want_w)).astype(np.float64)
    err = np.abs(got_w.astype(np.float64) - want_w)
    bad = err > bound
    assert not bad.any(), f"{what}: {int(bad.sum())} of {bad.size} weights off, worst {err.max():.3e} (update {np.abs(want_w.astype(np.float64) - w0)[np.argmax(err)]:.3e})"


def fixed_point_floor(dfeat: np.ndarray) -> np.ndarray:
    """Per level, the size below which a gradient entry may round to zero in
    the GPU's fixed-point sums: the coarse levels' int32 slabs round each
    value to 2^-31 S with S the sum over a chunk's samples of max(|d0|, |d1|)
    (the binned levels' int64 sums to 2^-40 of a bin's largest record, far
    finer); 2^-28 S over all samples bounds eight such roundings."""
    d = np.abs(np.asarray(dfeat, np.float64)).reshape(dfeat.shape[0], -1, 2)
    return np.ldexp(d.max(axis=2).sum(axis=0), -28)


def assert_table_grad(got, want, n_levels: int, what: str, frob_tol: float, entry_tol: float = 1e-2, floor=None, entry_frac: float = 0.0):
    """A hash-table gradient [L][T][2] level by level: relative Frobenius
    error <= frob_tol; every entry (all but a fraction entry_frac of a
    level's touched entries) within entry_tol relative to max(|want|, 10 % of
    the level's RMS); the support (entries with a nonzero gradient)
    identical, except that an entry the GPU leaves at zero may be nonzero in
    the oracle below floor[l] (fixed_point_floor: the rounding of the GPU's
    fixed-point sums).  Returns the worst level's Frobenius error."""
    got = np.asarray(got, np.float64).reshape(n_levels, -1)
    want = np.asarray(want, np.float64).reshape(n_levels, -1)
    worst = 0.0
    below = 0
    for l in range(n_levels):
        g, w = got[l], want[l]
        extra = (g != 0) & (w == 0)
        assert not extra.any(), f"{what}: level {l}: {int(extra.sum())} entries nonzero on the GPU where the oracle has no contribution"
        missing = (g == 0) & (w != 0)
        if missing.any():
            lim = 0.0 if floor is None else float(floor[l])
            assert np.abs(w[missing]).max() <= lim, f"{what}: level {l}: {int(missing.sum())} entries zero on the GPU, largest oracle value {np.abs(w[missing]).max():.3e} > {lim:.3e}"
            below += int(missing.sum())
        nw = np.linalg.norm(w)
        frob = float(np.linalg.norm(g - w) / max(nw, 1e-30))
        rms_floor = max(0.1 * float(np.sqrt(np.mean(w ** 2))), 1e-30)
        ent = np.abs(g - w) / np.maximum(np.abs(w), rms_floor)
        k = int(np.argmax(ent))
        assert frob <= frob_tol, f"{what}: level {l}: relative Frobenius error {frob:.3e} > {frob_tol}"
        n_bad = int(np.count_nonzero(ent > entry_tol))
        assert n_bad <= entry_frac * np.count_nonzero(w), f"{what}: level {l}: {n_bad} entries beyond {entry_tol}, worst entry {k} off by {ent[k]:.3e} (got {g[k]!r} want {w[k]!r}, floor {rms_floor:.3e})"
        worst = max(worst, frob)
    print(f"[grad] {what}: worst level relative Frobenius {worst:.3e}; {below} entries below the fixed-point floor", flush=True)
    return worst


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


__all__ = ["L", "ext", "orc", "DeviceArray", "synchronize", "assert_rel", "assert_rel_rows", "assert_table_grad", "fixed_point_floor", "oracle_grid", "host_table", "host_params", "points", "unit_dirs", "byref"]
