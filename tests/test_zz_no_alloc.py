"""The allocation-free march count (nerf_ext_march_count_noalloc) against
nerf_ext_march_count, through the C ABI: bit-identical per-ray counts on two
calls in a row, the second with a smaller image (the scratch keeps the first
call's ray records: nothing there may leak into the second), and a clear
error past the scratch maximum of 2^20 rays."""
import ctypes as C

import numpy as np
import pytest

from conftest import announce
from helpers import L, ext, orc, DeviceArray, synchronize

pytestmark = pytest.mark.gpu

RES = 64


@pytest.fixture(scope="module")
def occupancy():
    g = ext.scene_gaussians(32, seed=5)
    bits = DeviceArray.from_numpy(orc.occupancy_from_scene(g, RES, threshold=0.01))
    return bits, ext.occupancy_struct(bits, RES)


def _counts(fn, cam, occ, max_steps):
    n = cam.width * cam.height
    out = DeviceArray((n,), np.uint32)
    L.call(fn, C.byref(cam), C.byref(occ), max_steps, out.ptr, None)
    synchronize()
    return out.numpy()


def test_noalloc_march_matches_allocating_entry_point(occupancy):
    _, occ = occupancy
    for w, h, steps in ((1024, 1024, 1024), (320, 200, 256)):
        announce(f"march count noalloc {w}x{h} steps={steps}")
        cam = ext.camera_orbit(3, 0, 1.32, (0.5, 0.5, 0.5), w, h, 1111.0 * w / 800.0)
        want = _counts("nerf_ext_march_count", cam, occ, steps)
        got = _counts("nerf_ext_march_count_noalloc", cam, occ, steps)
        assert (want > 0).mean() > 0.05, "too few rays hit occupied cells"
        assert np.array_equal(got, want), f"{w}x{h}: counts differ from nerf_ext_march_count"


def test_noalloc_march_rejects_more_than_2p20_rays(occupancy):
    announce("march count noalloc: size limit")
    _, occ = occupancy
    cam = ext.camera_orbit(3, 0, 1.32, (0.5, 0.5, 0.5), 1025, 1024, 1111.0)
    out = DeviceArray((1,), np.uint32)
    lib = L.load()
    status = lib.nerf_ext_march_count_noalloc(C.byref(cam), C.byref(occ), 64, out.ptr, None)
    assert status == L.NERF_STATUS_INVALID_USAGE
    assert b"2^20" in lib.nerf_ext_last_error()
