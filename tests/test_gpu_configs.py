"""Parity of the large configurations on the GPU.

C4: hash grid T = 2^22 (16 levels, fp16, finest resolution 4096), 256
Gaussians, 256^3 occupancy, <= 2048 march steps, a 1920x1080 camera's field
of view (focal 1111 * 1920 / 800) rendered at reduced size.
C5: unbounded scene of 512 Gaussians over radius 16 plus a uniform shell,
5 nested 128^3 occupancy cascades (cascade 0 = [-1, 1]^3, doubling), hash
grid T = 2^21, several views of a 1280x720 camera's field of view rendered in
one launch with one compacted sample stream, <= 4096 march steps.

Occupancy bits: bit-exact against the oracle in full at reduced resolution
and on sampled cells at the configured resolution; per-ray sample counts
bit-exact; RGB within 1e-3 relative; RGBA8 within 1 LSB.
"""
import numpy as np
import pytest

from conftest import announce
from helpers import L, ext, orc, DeviceArray, synchronize, byref, oracle_grid, host_table, host_params, assert_rel

pytestmark = pytest.mark.gpu

C5_BOX = (-1.0, -1.0, -1.0, 1.0, 1.0, 1.0)
C5_CASCADES = 5
C5_SHELL = ((0.0, 0.0, 0.0), 12.0, 15.5)


def c5_scene():
    return ext.scene_gaussians(512, seed=5, centre=(-16.0, 16.0), sigma=(0.3, 1.5), amplitude=(5.0, 50.0))


def c4_scene():
    return ext.scene_gaussians(256, seed=4)


def cell_centres(res, lo, hi, idx):
    """fp32 cell centres lo + (i + 0.5) * ((hi - lo) / res), the oracle's operations."""
    f = np.float32
    x, y, z = idx % res, (idx // res) % res, idx // (res * res)
    out = np.empty((idx.size, 3), np.float32)
    for a, i in enumerate((x, y, z)):
        step = f(f(hi[a]) - f(lo[a])) / f(res)
        out[:, a] = f(lo[a]) + (i.astype(np.float32) + f(0.5)) * step
    return out


def cascade_box(box, c):
    f = np.float32
    lo, hi = [f(v) for v in box[:3]], [f(v) for v in box[3:]]
    if c == 0:
        return lo, hi
    centre = [f(0.5) * (lo[a] + hi[a]) for a in range(3)]
    half = [f(0.5) * (hi[a] - lo[a]) for a in range(3)]
    s = f(2.0 ** c)
    return [centre[a] - half[a] * s for a in range(3)], [centre[a] + half[a] * s for a in range(3)]


def check_sampled_bits(bits, gaussians, res, box, cascades, shell=None, n=20000, seed=0):
    """Bits of sampled cells against the oracle's density at their centres
    (cells within 1e-5 relative of the threshold or the shell radii skipped)."""
    rng = np.random.default_rng(seed)
    words = (res ** 3 + 31) // 32
    checked = 0
    for c in range(cascades):
        lo, hi = cascade_box(box, c)
        idx = rng.integers(0, res ** 3, size=n // cascades)
        q = cell_centres(res, lo, hi, idx)
        dens = orc.scene_density(gaussians, q)
        want = dens > np.float32(0.01)
        keep = np.abs(dens - 0.01) > 1e-5 * 0.01
        if shell is not None:
            r2 = np.sum((q.astype(np.float64) - np.array(shell[0])) ** 2, axis=1)
            in_shell = (r2 >= shell[1] ** 2) & (r2 <= shell[2] ** 2)
            want |= in_shell
            keep &= (np.abs(r2 - shell[1] ** 2) > 1e-3) & (np.abs(r2 - shell[2] ** 2) > 1e-3)
        got = (bits[c * words + (idx >> 5)] >> (idx & 31).astype(np.uint32)) & 1
        assert np.array_equal(got[keep].astype(bool), want[keep]), f"cascade {c}: {np.count_nonzero(got[keep].astype(bool) != want[keep])} cells differ"
        checked += int(keep.sum())
    assert checked > n // 2


def render_and_check(model, desc, bits_dev, res, box, cascades, cams, max_steps, threads=16):
    occ = ext.occupancy_struct(bits_dev, res, box[:3], box[3:], cascades)
    views, w, h = len(cams), cams[0].width, cams[0].height
    rgb = DeviceArray((views, h, w, 3), np.float32)
    counts = DeviceArray((views, h, w), np.uint32)
    rgba, stats = ext.Renderer().render(model, occ, cams, max_steps, rgb=rgb, counts=counts, timed=True)
    synchronize()
    dp, cp = host_params(model)
    table = host_table(model)
    bits = bits_dev.numpy()
    got_rgb, got_rgba, got_counts = rgb.numpy().reshape(views, -1, 3), rgba.numpy().reshape(views, -1), counts.numpy().reshape(views, -1)
    assert stats.samples == int(got_counts.sum())
    rays = np.arange(w * h, dtype=np.uint32)
    for v in range(views):
        ocam = orc.camera_from_bytes(bytes(cams[v]))
        want_counts = orc.march_count(ocam, bits, res, box, max_steps, cascades=cascades)
        assert np.array_equal(got_counts[v], want_counts), f"view {v}: {np.count_nonzero(got_counts[v] != want_counts)} ray counts differ"
        assert want_counts.max() > 0
        want_rgb, want_rgba, want_c2 = orc.render_rays(oracle_grid(desc), table, dp, cp, ocam, bits, res, box, max_steps, rays, threads=threads, cascades=cascades)
        assert np.array_equal(want_c2, want_counts)
        assert_rel(got_rgb[v], want_rgb, what=f"render rgb view {v}")
        gb = got_rgba[v].view(np.uint8).reshape(-1, 4).astype(int)
        wb = want_rgba.view(np.uint8).reshape(-1, 4).astype(int)
        assert np.abs(gb - wb).max() <= 1
    return got_counts


def test_c5_cascade_bits_bit_exact_reduced_resolution():
    announce("C5 occupancy: 5 cascades at 24^3, 512 gaussians + shell, full compare")
    g = c5_scene()
    bits = ext.occupancy_from_scene(g, 24, 0.01, C5_BOX[:3], C5_BOX[3:], C5_CASCADES, shell=C5_SHELL)
    synchronize()
    want = orc.occupancy_from_scene(g, 24, C5_BOX, 0.01, cascades=C5_CASCADES, shell=C5_SHELL)
    got = bits.numpy()
    assert np.array_equal(got, want), f"{np.count_nonzero(got != want)} words differ"
    words = (24 ** 3 + 31) // 32
    assert all(want[c * words:(c + 1) * words].any() for c in range(C5_CASCADES))


def test_c5_render_multi_view():
    announce("C5 render: 5 x 128^3 cascades, T=2^21, 3 views of 64x36 in one launch, <=4096 steps")
    g = c5_scene()
    bits = ext.occupancy_from_scene(g, 128, 0.01, C5_BOX[:3], C5_BOX[3:], C5_CASCADES, shell=C5_SHELL)
    synchronize()
    check_sampled_bits(bits.numpy(), g, 128, C5_BOX, C5_CASCADES, C5_SHELL)
    desc = ext.grid_desc(21, L.NERF_EXT_F16)
    model = ext.Model.create(desc, seed=3, table_range=1.0)
    focal = 1111.0 * 1280.0 / 800.0 * 64.0 / 1280.0
    cams = [ext.camera_orbit(5, i, 4.0, (0.0, 0.0, 0.0), 64, 36, focal) for i in range(3)]
    counts = render_and_check(model, desc, bits, 128, C5_BOX, C5_CASCADES, cams, 4096)
    # Samples come from several cascades: some rays run past the inner box.
    assert counts.max() > 256


def test_c4_render_large_table():
    announce("C4 render: T=2^22 finest 4096, 256^3 occupancy, 48x27 view of the 1920x1080 field of view, <=2048 steps")
    g = c4_scene()
    bits = ext.occupancy_from_scene(g, 256, 0.01)
    synchronize()
    box = (0.0, 0.0, 0.0, 1.0, 1.0, 1.0)
    check_sampled_bits(bits.numpy(), g, 256, box, 1)
    desc = ext.grid_desc(22, L.NERF_EXT_F16, finest=4096)
    levels, _ = ext.grid_levels(desc)
    assert levels[15] == 4096
    model = ext.Model.create(desc, seed=4, table_range=1.0)
    focal = 1111.0 * 1920.0 / 800.0 * 48.0 / 1920.0
    cams = [ext.camera_orbit(4, 0, 1.32, (0.5, 0.5, 0.5), 48, 27, focal)]
    render_and_check(model, desc, bits, 256, box, 1, cams, 2048)
