"""Rays, AABB clip, occupancy march and compositing in the oracle, pinned by
analytic axis-aligned cases and closed forms."""
import numpy as np

BOX = (0, 0, 0, 1, 1, 1)


def _down_camera(z0=3.0, fx=1e30):
    # 2x2 image, cx = cy = 0.5: pixel (0, 0) looks exactly along -z from (0.5, 0.5, z0).
    c2w = [1, 0, 0, 0.5, 0, 1, 0, 0.5, 0, 0, 1, z0]
    return c2w, fx


def test_axis_ray_t_range(orc):
    c2w, fx = _down_camera()
    cam = orc.camera(c2w, fx, fx, 0.5, 0.5, 2, 2)
    r = orc.pixel_ray(cam, 0, BOX)
    np.testing.assert_array_equal(r, np.array([0.5, 0.5, 3.0, 0, 0, -1, 2.0, 3.0], np.float32))


def test_march_all_occupied_uniform_steps(orc):
    c2w, fx = _down_camera()
    cam = orc.camera(c2w, fx, fx, 0.5, 0.5, 2, 2)
    for steps in (16, 64, 128):
        s = orc.march_ray(cam, None, 128, BOX, steps, 0)
        assert s.shape[0] == steps
        k = np.arange(steps, dtype=np.float64)
        np.testing.assert_array_equal(s[:, 1], np.float32(1.0 / steps))
        np.testing.assert_array_equal(s[:, 0], (2.0 + (k + 0.5) / steps).astype(np.float32))


def test_march_half_occupied(orc):
    res = 16
    bits = np.zeros(res ** 3 // 32, np.uint32)
    cells = np.arange(res ** 3)
    z = cells // (res * res)
    occ = cells[z < res // 2]                                 # lower half in z
    np.bitwise_or.at(bits, occ >> 5, (np.uint32(1) << (occ & 31).astype(np.uint32)))
    c2w, fx = _down_camera()
    cam = orc.camera(c2w, fx, fx, 0.5, 0.5, 2, 2)
    s = orc.march_ray(cam, bits, res, BOX, 64, 0)
    assert s.shape[0] == 32 and np.all(s[:, 0] >= 2.5)
    assert orc.march_count(cam, np.zeros_like(bits), res, BOX, 64, 0, 1)[0] == 0


def test_march_cone_steps_cover_range(orc):
    """With cone stepping the dts of an all-occupied ray tile [t_near, t_far]."""
    c2w = [1, 0, 0, 0.5, 0, 1, 0, 0.5, 0, 0, 1, 1.8]
    cam = orc.camera(c2w, 300.0, 300.0, 0.5, 0.5, 2, 2)
    r = orc.pixel_ray(cam, 0, BOX)
    s = orc.march_ray(cam, None, 128, BOX, 1024, 0)
    assert 0 < s.shape[0] < 1024
    np.testing.assert_allclose(s[:, 1].astype(np.float64).sum(), r[7] - r[6], rtol=1e-5)
    assert np.all(np.diff(s[:, 0]) > 0)
    # dt grows like t * cone once above dt_min = range / max_steps
    cone = 1.0 / 300.0
    mid = s[len(s) // 2]
    np.testing.assert_allclose(mid[1], max((r[7] - r[6]) / 1024, (mid[0] - mid[1] / 2) * cone), rtol=1e-5)


def test_ray_miss_and_parallel(orc):
    c2w = [1, 0, 0, 3.0, 0, 1, 0, 0.5, 0, 0, 1, 3.0]          # x = 3: misses the box
    cam = orc.camera(c2w, 1e30, 1e30, 0.5, 0.5, 2, 2)
    assert orc.pixel_ray(cam, 0, BOX) is None
    assert orc.march_count(cam, None, 16, BOX, 64, 0, 1)[0] == 0


def test_composite_constant_density_closed_form(orc):
    n, sigma, dt = 50, 3.0, 0.01
    rgb = np.array([0.2, 0.5, 0.9], np.float32)
    s = np.tile(np.array([sigma, *rgb], np.float32), (n, 1))
    got, packed, used = orc.composite_ray(s, np.full(n, dt, np.float32), t_stop=0.0)
    T = np.exp(-sigma * dt * n)
    np.testing.assert_allclose(got, rgb * (1 - T) + T, rtol=1e-5)
    assert used == n
    want8 = np.rint(np.clip(rgb * (1 - T) + T, 0, 1) * 255).astype(np.uint32)
    assert packed == (255 << 24) | (int(want8[2]) << 16) | (int(want8[1]) << 8) | int(want8[0])


def test_composite_early_stop(orc):
    n = 100
    s = np.tile(np.array([500.0, 1.0, 0.0, 0.0], np.float32), (n, 1))
    got, _, used = orc.composite_ray(s, np.full(n, 0.01, np.float32), t_stop=1e-4)
    # T after k samples = exp(-5 k) < 1e-4 first at k = 2
    assert used == 2
    np.testing.assert_allclose(got, [1.0, np.exp(-10.0), np.exp(-10.0)], rtol=1e-4, atol=1e-6)


def test_render_rays_stop_index(orc):
    """Zero density-MLP weights give raw density 0, sigma = exp(0) = 1 at every
    sample whatever the table, so an axis ray through an all-occupied box of
    side 20 marched in 256 uniform steps of dt = 20/256 (exact in fp32) has
    T = exp(-k dt) after k samples: the first k with T < 1e-4 is 118
    (k dt = 9.21875; 117 steps leave T = 1.075e-4)."""
    grid = orc.make_grid(16, 12, 0)
    table = np.zeros(16 * (1 << 12) * 2, np.float32)
    dp = np.zeros(3072, np.uint16)
    cp = orc.f32_to_f16_bits(orc.mlp_init(1))
    c2w = [1, 0, 0, 10.0, 0, 1, 0, 10.0, 0, 0, 1, 30.0]
    cam = orc.camera(c2w, 1e30, 1e30, 0.5, 0.5, 2, 2)
    box = (0, 0, 0, 20, 20, 20)
    rgb, _, counts, used, t_prev, t_final = orc.render_rays(grid, table, dp, cp, cam, None, 16, box, 256, np.array([0], np.uint32), stop=True)
    assert counts[0] == 256 and used[0] == 118
    assert t_prev[0] >= 1e-4 > t_final[0]
    np.testing.assert_allclose(t_final[0], np.exp(-118 * 20.0 / 256), rtol=1e-5)
    np.testing.assert_allclose(t_prev[0], np.exp(-117 * 20.0 / 256), rtol=1e-5)
    # Without the stop every sample is composited and T is the full chord's.
    _, _, _, used0, _, t0 = orc.render_rays(grid, table, dp, cp, cam, None, 16, box, 256, np.array([0], np.uint32), t_stop=0.0, stop=True)
    assert used0[0] == 256
    np.testing.assert_allclose(t0[0], np.exp(-20.0), rtol=1e-4)
    # The stop leaves T_final of the background in the pixel: rgb = C + T bg.
    rgb0, *_ = orc.render_rays(grid, table, dp, cp, cam, None, 16, box, 256, np.array([0], np.uint32), t_stop=0.0)
    assert np.all(np.abs(rgb - rgb0) < 2e-4)
