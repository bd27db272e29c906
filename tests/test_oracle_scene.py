"""Analytic scene pinning: det_expf accuracy against libm, density and
occupancy against an fp64 numpy evaluation away from the threshold."""
import numpy as np


def _ulp_diff(a, b):
    ai = a.view(np.int32).astype(np.int64)
    bi = b.view(np.int32).astype(np.int64)
    return np.abs(ai - bi)


def test_det_expf_within_2ulp(orc):
    x = np.linspace(-87.0, 88.0, 2_000_001, dtype=np.float32)
    got = orc.det_expf(x)
    want = np.exp(x.astype(np.float64)).astype(np.float32)
    assert _ulp_diff(got, want).max() <= 2
    assert orc.det_expf(np.array([-87.5, -1000.0, np.nan], np.float32)).tolist() == [0.0, 0.0, 0.0]
    assert orc.det_expf(np.array([0.0], np.float32))[0] == 1.0


def _scene(orc_unused=None, count=32, seed=0):
    from nerf_amd import ext

    return ext.scene_gaussians(count, seed)


def test_scene_generator_formula(orc):
    g = _scene()
    u = orc.uniform_fill(0x6A55, 0, 32 * 8, 0.0, 1.0).reshape(32, 8)
    np.testing.assert_array_equal(g[:, 0:3], (np.float32(0.2) + (np.float32(0.8) - np.float32(0.2)) * u[:, 0:3]).astype(np.float32))
    np.testing.assert_array_equal(g[:, 5:8], u[:, 5:8])
    assert g[:, 3].min() >= 0.02 and g[:, 3].max() < 0.1 and g[:, 4].min() >= 5 and g[:, 4].max() < 50


def test_scene_density_fp64(orc):
    g = _scene()
    rng = np.random.default_rng(7)
    p = rng.random((5000, 3), dtype=np.float32)
    got = orc.scene_density(g, p).astype(np.float64)
    d2 = ((p[:, None, :].astype(np.float64) - g[None, :, :3]) ** 2).sum(-1)
    want = (g[None, :, 4] * np.exp(-d2 / (2 * g[None, :, 3].astype(np.float64) ** 2))).sum(-1)
    np.testing.assert_allclose(got, want, rtol=2e-5, atol=1e-30)


def test_occupancy_bits_fp64(orc):
    g = _scene()
    res = 32
    bits = orc.occupancy_from_scene(g, res)
    c = np.arange(res ** 3)
    x, y, z = c % res, (c // res) % res, c // (res * res)
    step = np.float32(1.0) / np.float32(res)
    p = np.stack([(x + 0.5) * step, (y + 0.5) * step, (z + 0.5) * step], -1).astype(np.float64)
    d2 = ((p[:, None, :] - g[None, :, :3]) ** 2).sum(-1)
    dens = (g[None, :, 4] * np.exp(-d2 / (2 * g[None, :, 3].astype(np.float64) ** 2))).sum(-1)
    got = (bits[c >> 5] >> (c & 31).astype(np.uint32)) & 1
    clear = np.abs(dens - 0.01) > 1e-5
    assert np.array_equal(got[clear], (dens[clear] > 0.01).astype(np.uint32))
    assert 0.05 < got.mean() < 0.95
