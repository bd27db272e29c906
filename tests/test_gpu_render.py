"""GPU scene, occupancy, march and render parity.  Occupancy bits and per-ray
sample counts bit-exact; RGB within 1e-3 relative; RGBA8 within 1 LSB."""
import numpy as np
import pytest

from conftest import announce
from helpers import L, ext, orc, DeviceArray, synchronize, byref, oracle_grid, host_table, host_params, points, assert_rel

pytestmark = pytest.mark.gpu

BOX = (0.0, 0.0, 0.0, 1.0, 1.0, 1.0)
CENTRE = (0.5, 0.5, 0.5)


def test_scene_density_bit_exact():
    announce("scene density 32 gaussians")
    g = ext.scene_gaussians(32, seed=0)
    pos = points(20000, seed=5)
    d_g, d_p, d_o = DeviceArray.from_numpy(g), DeviceArray.from_numpy(pos), DeviceArray((20000,), np.float32)
    L.call("nerf_ext_scene_density", d_g.ptr, 32, d_p.ptr, 20000, d_o.ptr, None)
    synchronize()
    assert np.array_equal(d_o.numpy().view(np.uint32), orc.scene_density(g, pos).view(np.uint32))


@pytest.mark.parametrize("res,count", [(128, 32), (37, 256), (5, 3)])
def test_occupancy_bits_bit_exact(res, count):
    announce(f"occupancy res={res} gaussians={count}")
    g = ext.scene_gaussians(count, seed=2)
    bits = ext.occupancy_from_scene(g, res)
    synchronize()
    want = orc.occupancy_from_scene(g, res)
    got = bits.numpy()
    assert np.array_equal(got, want), f"{np.count_nonzero(got != want)} words differ"


def _scene_setup(res=128, count=32, seed=0):
    g = ext.scene_gaussians(count, seed=seed)
    return g, ext.occupancy_from_scene(g, res)


@pytest.mark.parametrize("w,h,steps", [(64, 48, 1024), (33, 17, 64)])
def test_march_counts_bit_exact(w, h, steps):
    announce(f"march count {w}x{h} steps={steps}")
    g, bits = _scene_setup()
    for index in range(3):
        cam = ext.camera_orbit(0, index, 1.32, CENTRE, w, h, 1111.0 * w / 800.0)
        occ = ext.occupancy_struct(bits, 128)
        d_counts = DeviceArray((w * h,), np.uint32)
        L.call("nerf_ext_march_count", byref(cam), byref(occ), steps, d_counts.ptr, None)
        synchronize()
        ocam = orc.camera_from_bytes(bytes(cam))
        want = orc.march_count(ocam, bits.numpy(), 128, BOX, steps)
        got = d_counts.numpy()
        assert np.array_equal(got, want), f"view {index}: {np.count_nonzero(got != want)} rays differ"
        assert want.max() > 0


@pytest.mark.parametrize("focal,steps", [(1.5, 64), (1.5, 1024), (20.0, 2), (20.0, 3), (20.0, 5)])
def test_march_counts_both_step_chains(focal, steps):
    """The march advances its shared t chain by a three-instruction form
    only where a step that reaches t_far starts beyond t_far / 2 (cone <= 1/2,
    dt_min <= t_far / 4), else by the reference's clamp: a 1.5-pixel focal
    length (cone 2/3) and 2, 3 and 5 steps per ray cover both sides of those
    bounds.  Counts bit-exact against the oracle's sequential recurrence."""
    announce(f"march count, focal {focal} px, {steps} steps")
    g, bits = _scene_setup()
    w, h = 40, 30
    for index in range(2):
        cam = ext.camera_orbit(0, index, 1.32, CENTRE, w, h, focal)
        occ = ext.occupancy_struct(bits, 128)
        d_counts = DeviceArray((w * h,), np.uint32)
        L.call("nerf_ext_march_count", byref(cam), byref(occ), steps, d_counts.ptr, None)
        synchronize()
        want = orc.march_count(orc.camera_from_bytes(bytes(cam)), bits.numpy(), 128, BOX, steps)
        got = d_counts.numpy()
        assert np.array_equal(got, want), f"view {index}: {np.count_nonzero(got != want)} rays differ"
        assert want.max() > 0


@pytest.mark.parametrize("w,h,views", [(24, 20, 1), (16, 12, 3)])
def test_render_parity(w, h, views):
    announce(f"render {w}x{h} views={views}")
    g, bits = _scene_setup()
    desc = ext.grid_desc(19, L.NERF_EXT_F16)
    model = ext.Model.create(desc, seed=0, table_range=1.0)
    cams = [ext.camera_orbit(0, i, 1.32, CENTRE, w, h, 1111.0 * w / 800.0) for i in range(views)]
    occ = ext.occupancy_struct(bits, 128)
    rgb = DeviceArray((views, h, w, 3), np.float32)
    counts = DeviceArray((views, h, w), np.uint32)
    r = ext.Renderer()
    rgba, stats = r.render(model, occ, cams, 1024, rgb=rgb, counts=counts, timed=True)
    synchronize()
    dp, cp = host_params(model)
    got_rgb, got_rgba, got_counts = rgb.numpy().reshape(views, -1, 3), rgba.numpy().reshape(views, -1), counts.numpy().reshape(views, -1)
    assert stats.samples == int(got_counts.sum())
    for v in range(views):
        ocam = orc.camera_from_bytes(bytes(cams[v]))
        rays = np.arange(w * h, dtype=np.uint32)
        want_rgb, want_rgba, want_counts = orc.render_rays(oracle_grid(desc), host_table(model), dp, cp, ocam, bits.numpy(), 128, BOX, 1024, rays, threads=8)
        assert np.array_equal(got_counts[v], want_counts)
        assert_rel(got_rgb[v], want_rgb, what=f"render rgb view {v}")
        gb = got_rgba[v].view(np.uint8).reshape(-1, 4).astype(int)
        wb = want_rgba.view(np.uint8).reshape(-1, 4).astype(int)
        assert np.abs(gb - wb).max() <= 1
    # A second call on the same renderer (cached buffers) gives the same image.
    rgba2, _ = r.render(model, occ, cams, 1024)
    synchronize()
    assert np.array_equal(rgba2.numpy(), rgba.numpy())


def test_render_in_chunks_matches_one_chunk():
    # 2 views of 64x48 = 6 blocks of 1024 rays; a small sample budget splits
    # the render into one chunk per block.  Rays are independent, so the
    # images, counts and statistics are identical.
    announce("render in chunks: 2 views 64x48, chunk budget 1 sample")
    g, bits = _scene_setup()
    desc = ext.grid_desc(19, L.NERF_EXT_F16)
    model = ext.Model.create(desc, seed=0, table_range=1.0)
    cams = [ext.camera_orbit(0, i, 1.32, CENTRE, 64, 48, 1111.0 * 64 / 800.0) for i in range(2)]
    occ = ext.occupancy_struct(bits, 128)
    outs = []
    for chunk in (0, 1):
        rgb = DeviceArray((2, 48, 64, 3), np.float32)
        counts = DeviceArray((2, 48, 64), np.uint32)
        rgba, stats = ext.Renderer().render(model, occ, cams, 1024, rgb=rgb, counts=counts, timed=True, chunk_samples=chunk)
        synchronize()
        outs.append((rgba.numpy(), rgb.numpy(), counts.numpy(), stats.samples, stats.samples_shaded))
    (a0, r0, c0, s0, h0), (a1, r1, c1, s1, h1) = outs
    assert np.array_equal(a0, a1) and np.array_equal(r0.view(np.uint32), r1.view(np.uint32)) and np.array_equal(c0, c1)
    assert s0 == s1 == int(c0.sum()) and h0 == h1 and s0 > 0
