"""The occupancy cell rule's box-relative coordinates on the GPU, bit for bit
against IEEE fp32 subtraction and division (numpy float32, round to nearest,
subnormals kept): the march kernels replace the three divisions by the box
size with its refined reciprocal and two FMA corrections and fall back to the
division where that could differ, so every input must match — ordinary
points, points on and one ulp beside the faces, zero, signed tiny and
subnormal offsets, quotients at the fallback's bounds (2^-80, 2^80),
infinities, NaN, and boxes whose size is outside [2^-20, 2^20], zero or
negative (backend-cuda.cu:338-351 divides inline)."""
import ctypes as C

import numpy as np
import pytest

from conftest import announce
from helpers import L, DeviceArray, synchronize

pytestmark = pytest.mark.gpu


def _gpu(points: np.ndarray, lo, hi) -> np.ndarray:
    pts = np.ascontiguousarray(points, np.float32).reshape(-1, 3)
    d_p = DeviceArray.from_numpy(pts)
    d_o = DeviceArray(pts.shape, np.float32)
    clo = (C.c_float * 3)(*lo)
    chi = (C.c_float * 3)(*hi)
    L.call("nerf_ext_box_relative", d_p.ptr, pts.shape[0], clo, chi, d_o.ptr, None)
    synchronize()
    return d_o.numpy()


def _want(points: np.ndarray, lo, hi) -> np.ndarray:
    pts = np.asarray(points, np.float32).reshape(-1, 3)
    lo32, hi32 = np.asarray(lo, np.float32), np.asarray(hi, np.float32)
    with np.errstate(all="ignore"):
        return (pts - lo32) / (hi32 - lo32)


def _assert_same_bits(got: np.ndarray, want: np.ndarray, what: str) -> None:
    nan_g, nan_w = np.isnan(got), np.isnan(want)
    assert np.array_equal(nan_g, nan_w), f"{what}: NaN positions differ"
    gb, wb = got.view(np.uint32)[~nan_g], want.view(np.uint32)[~nan_w]
    bad = np.flatnonzero(gb != wb)
    assert bad.size == 0, f"{what}: {bad.size} of {gb.size} coordinates differ, first got {got[~nan_g][bad[0]]!r} want {want[~nan_w][bad[0]]!r}"


def _adversarial(lo, hi, rng) -> np.ndarray:
    lo32, hi32 = np.asarray(lo, np.float32), np.asarray(hi, np.float32)
    size = hi32 - lo32
    cols = []
    # Uniform over the box and a margin around it.
    cols.append(lo32 + (rng.random((20000, 3)) * 1.4 - 0.2).astype(np.float32) * size)
    # On the faces, one ulp either side, and the centre.
    for base in (lo32, hi32, (lo32 + hi32) * np.float32(0.5)):
        for k in (-2, -1, 0, 1, 2):
            v = base.copy()
            for _ in range(abs(k)):
                v = np.nextafter(v, np.float32(np.inf) if k > 0 else np.float32(-np.inf)).astype(np.float32)
            cols.append(np.tile(v, (1, 1)))
    # Offsets from lo across the exponent range, both signs, including
    # subnormals and the fallback's bounds (offset = q * size).
    exps = np.arange(-149, 128, 1, dtype=np.float64)
    for sgn in (1.0, -1.0):
        mags = np.float32(2.0) ** exps.astype(np.float32)
        for q in (mags, mags * np.float32(1.5), np.float32(2.0 ** -80) * size[0] * np.ones(1, np.float32), np.float32(2.0 ** 80) * size[0] * np.ones(1, np.float32)):
            with np.errstate(all="ignore"):
                off = (np.float32(sgn) * np.asarray(q, np.float32)).astype(np.float32)
                cols.append(np.stack([lo32[0] + off, np.full_like(off, lo32[1] + size[1] * np.float32(0.5)), lo32[2] + off], axis=1))
    # Values just below and above the fallback's bounds on every axis.
    for bound in (2.0 ** -80, 2.0 ** 80):
        b = np.float32(bound)
        for f in (np.nextafter(b, np.float32(0)), b, np.nextafter(b, np.float32(np.inf))):
            with np.errstate(all="ignore"):
                cols.append((lo32 + np.float32(f) * size).reshape(1, 3).astype(np.float32))
                cols.append((lo32 - np.float32(f) * size).reshape(1, 3).astype(np.float32))
    # Non-finite coordinates and exact zeros of the offset.
    special = np.array([[np.inf, 0.5, 0.5], [-np.inf, 0.5, 0.5], [np.nan, 0.5, 0.5], [0.5, np.inf, np.nan], [np.finfo(np.float32).max, 0, 0], [-np.finfo(np.float32).max, 0, 0]], np.float32)
    cols.append(lo32 + special * np.float32(1.0))
    cols.append(np.tile(lo32, (4, 1)))
    return np.concatenate([c.reshape(-1, 3) for c in cols]).astype(np.float32)


BOXES = [
    ((-1.5, -1.5, -1.5), (1.5, 1.5, 1.5)),
    ((0.0, 0.0, 0.0), (1.0, 1.0, 1.0)),
    ((-0.3, 2.7, -1e-3), (0.9, 3.1, 5.0)),
    ((1e-30, -1e-30, 0.0), (1e-30 + 3.0, 2.0, 0.7)),
    ((-1e6, -2e6, 123.0), (1e6, 3e6, 124.0)),  # sizes above 2^20 on two axes
    ((0.0, 0.0, 0.0), (1e-7, 2e-6, 0.5)),  # sizes below 2^-20
    ((0.25, 0.25, 0.25), (0.25, 0.75, 0.75)),  # zero size on x
    ((1.0, 1.0, 1.0), (-1.0, 2.0, 2.0)),  # negative size on x
]


@pytest.mark.parametrize("box", range(len(BOXES)))
def test_box_relative_bit_exact(box):
    lo, hi = BOXES[box]
    announce(f"box_relative box={lo}..{hi}")
    rng = np.random.default_rng(100 + box)
    pts = _adversarial(lo, hi, rng)
    _assert_same_bits(_gpu(pts, lo, hi), _want(pts, lo, hi), f"box {box}")


def test_box_relative_random_bits():
    """Random float32 bit patterns as points (every class: normal,
    subnormal, zero, infinite, NaN) against two boxes."""
    announce("box_relative random bit patterns")
    rng = np.random.default_rng(7)
    pts = rng.integers(0, 2**32, (200000, 3), dtype=np.uint64).astype(np.uint32).view(np.float32)
    for lo, hi in BOXES[:2]:
        _assert_same_bits(_gpu(pts, lo, hi), _want(pts, lo, hi), f"random bits {lo}")
