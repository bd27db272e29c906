"""Parity of the benchmarked renders at their full size, and of the early stop.

Each test renders a whole benchmarked view (or, for C5, all eight views in
one call: 29 chunks of whole 1,024-ray blocks, each marched once into
per-ray slots, rounds with per-ray quotas)
and compares a deterministic ray subset with the oracle's render of the same
rays (backend-cuda.cu:601-635 composite, :1870-1909 whole-image loop):
- per-ray occupied sample counts bit-exact (over the whole view for the
  800x800 headline render);
- RGB within 1e-3 relative, RGBA8 within 1 LSB;
- the early-stop index (samples composited up to and including the one after
  which T < 1e-4) equal to the oracle's, except for rays whose oracle
  transmittance before or after that sample lies within 1e-4 relative of the
  threshold (ten times the largest RGB error these renders show), which may
  differ by one sample; at least 99 % of all rays equal;
- the samples the field evaluated per ray at least the composited ones, and
  their sum equal to the renderer's shaded-sample statistic.
"""
from concurrent.futures import ThreadPoolExecutor

import numpy as np
import pytest

from conftest import announce
from helpers import L, ext, orc, DeviceArray, synchronize, oracle_grid, host_table, host_params, assert_rel

pytestmark = pytest.mark.gpu

T_STOP = 1e-4
THREADS = 16


def full_counts(ocam, bits, res, box, max_steps, cascades=1):
    """Oracle march counts of every ray of the view, in THREADS ranges."""
    n = ocam.width * ocam.height
    step = (n + THREADS - 1) // THREADS
    parts = [(b, min(step, n - b)) for b in range(0, n, step)]
    with ThreadPoolExecutor(THREADS) as ex:
        outs = list(ex.map(lambda p: orc.march_count(ocam, bits, res, box, max_steps, p[0], p[1], cascades=cascades), parts))
    return np.concatenate(outs)


def subset(n_rays: int, k: int, seed: int) -> np.ndarray:
    """k distinct rays spread over [0, n_rays): a stride plus a seeded jitter."""
    stride = n_rays // k
    jitter = np.random.default_rng(seed).integers(0, stride, k)
    return (np.arange(k, dtype=np.int64) * stride + jitter).astype(np.uint32)


def render_full(model, occ, cams, max_steps):
    views, w, h = len(cams), cams[0].width, cams[0].height
    rgb = DeviceArray((views, h, w, 3), np.float32)
    counts = DeviceArray((views, h, w), np.uint32)
    comp = DeviceArray((views, h, w), np.uint32)
    shaded = DeviceArray((views, h, w), np.uint32)
    rgba, stats = ext.Renderer().render(model, occ, cams, max_steps, T_STOP, rgb=rgb, counts=counts, timed=True, composited=comp, shaded=shaded)
    synchronize()
    r = lambda a: a.numpy().reshape(views, -1)
    return rgba.numpy().reshape(views, -1), rgb.numpy().reshape(views, -1, 3), r(counts), r(comp), r(shaded), stats


def check_subset(got, want, what):
    """got/want: (rgb, rgba8, counts, composited) of the subset rays; want also
    (t_prev, t_final).  Returns the number of rays that stopped early."""
    g_rgb, g_rgba, g_counts, g_comp = got
    w_rgb, w_rgba, w_counts, w_used, t_prev, t_final = want
    assert np.array_equal(g_counts, w_counts), f"{what}: {np.count_nonzero(g_counts != w_counts)} ray counts differ"
    assert_rel(g_rgb, w_rgb, what=f"{what} rgb")
    gb, wb = g_rgba.view(np.uint8).reshape(-1, 4).astype(int), w_rgba.view(np.uint8).reshape(-1, 4).astype(int)
    assert np.abs(gb - wb).max() <= 1, f"{what}: RGBA8 differs by {np.abs(gb - wb).max()}"
    near = (np.abs(t_prev / T_STOP - 1.0) < 1e-4) | (np.abs(t_final / T_STOP - 1.0) < 1e-4)
    far = ~near
    bad = far & (g_comp != w_used)
    assert not bad.any(), f"{what}: early-stop index differs on {int(bad.sum())} rays, e.g. ray {np.flatnonzero(bad)[0]}: got {g_comp[bad][0]} want {w_used[bad][0]}"
    assert np.all(np.abs(g_comp[near].astype(np.int64) - w_used[near]) <= 1)
    equal = int(np.count_nonzero(g_comp == w_used))
    assert equal >= 0.99 * g_comp.size
    stopped = int(np.count_nonzero(t_final < T_STOP))
    print(f"[stop] {what}: {g_counts.size} rays, {stopped} stopped early, {int(near.sum())} near the threshold, stop index equal on {equal}", flush=True)
    return stopped


def headline_setup(table_range=1e-4, w_density_out0=None):
    """The 800x800 headline workload: 32 Gaussians (seed 0), 128^3 occupancy at
    0.01, hash grid T = 2^19 fp16 from seed 0, the reference's MLP init,
    camera on the radius-1.32 orbit about (0.5, 0.5, 0.5) at focal 1111."""
    g = ext.scene_gaussians(32, seed=0)
    bits = ext.occupancy_from_scene(g, 128, threshold=0.01)
    desc = ext.grid_desc(19, L.NERF_EXT_F16)
    model = ext.Model.create(desc, seed=0, table_range=table_range)
    if w_density_out0 is not None:
        # Raw density = w x (sum of the density MLP's hidden ReLUs): an opaque
        # medium in which most rays stop, at spread-out sample indices.
        d32 = model.density_f32.copy()
        d32[2048:2112] = w_density_out0
        model.density_f32 = d32
        model.density = DeviceArray.from_numpy(d32.astype(np.float16))
    cam = ext.camera_orbit(0, 0, 1.32, (0.5, 0.5, 0.5), 800, 800, 1111.0)
    return desc, model, bits, cam


def oracle_subset(desc, model, bits, ocam, res, box, max_steps, rays, cascades=1):
    dp, cp = host_params(model)
    return orc.render_rays(oracle_grid(desc), host_table(model), dp, cp, ocam, bits, res, box, max_steps, rays, T_STOP, threads=THREADS, cascades=cascades, stop=True)


def test_headline_800x800_full_size():
    announce("full-size 800x800 headline render (random-init model, T=2^19, <=1024 steps), whole-view counts + 4,000-ray subset")
    desc, model, bits, cam = headline_setup()
    occ = ext.occupancy_struct(bits, 128)
    rgba, rgb, counts, comp, shaded, stats = render_full(model, occ, [cam], 1024)
    ocam = orc.camera_from_bytes(bytes(cam))
    b = bits.numpy()
    want_counts = full_counts(ocam, b, 128, (0, 0, 0, 1, 1, 1), 1024)
    assert np.array_equal(counts[0], want_counts), f"{np.count_nonzero(counts[0] != want_counts)} ray counts differ"
    assert stats.samples == int(want_counts.sum())
    assert stats.samples_shaded == int(shaded.sum())
    assert np.all(shaded >= comp) and np.all(comp <= counts)
    rays = subset(800 * 800, 4000, 1)
    want = oracle_subset(desc, model, b, ocam, 128, (0, 0, 0, 1, 1, 1), 1024, rays)
    check_subset((rgb[0][rays], rgba[0][rays], counts[0][rays], comp[0][rays]), want, "800x800")


def test_headline_800x800_early_stop_dense_model():
    announce("full-size 800x800 render of an opaque model (table U(-1,1), density output row 0.5): early-stop index vs oracle")
    desc, model, bits, cam = headline_setup(table_range=1.0, w_density_out0=0.5)
    occ = ext.occupancy_struct(bits, 128)
    rgba, rgb, counts, comp, shaded, stats = render_full(model, occ, [cam], 1024)
    assert stats.samples_shaded == int(shaded.sum())
    assert np.all(shaded >= comp) and np.all(comp <= counts)
    # Most rays stop: far fewer samples shaded than marched.
    assert stats.samples_shaded < 0.9 * stats.samples
    ocam = orc.camera_from_bytes(bytes(cam))
    rays = subset(800 * 800, 4000, 2)
    want = oracle_subset(desc, model, bits.numpy(), ocam, 128, (0, 0, 0, 1, 1, 1), 1024, rays)
    stopped = check_subset((rgb[0][rays], rgba[0][rays], counts[0][rays], comp[0][rays]), want, "800x800 opaque")
    assert stopped > 2000


def test_c4_1920x1080_full_size():
    announce("full-size C4 render: 1920x1080, T=2^22 finest 4096, 256^3 occupancy, <=2048 steps; 2,000-ray subset")
    g = ext.scene_gaussians(256, seed=4)
    bits = ext.occupancy_from_scene(g, 256, 0.01)
    desc = ext.grid_desc(22, L.NERF_EXT_F16, finest=4096)
    model = ext.Model.create(desc, seed=0)
    cam = ext.camera_orbit(0, 0, 1.32, (0.5, 0.5, 0.5), 1920, 1080, 1111.0 * 1920 / 800.0)
    occ = ext.occupancy_struct(bits, 256)
    rgba, rgb, counts, comp, shaded, stats = render_full(model, occ, [cam], 2048)
    assert stats.samples == int(counts.sum()) and stats.samples_shaded == int(shaded.sum())
    assert np.all(shaded >= comp) and np.all(comp <= counts)
    rays = subset(1920 * 1080, 2000, 4)
    want = oracle_subset(desc, model, bits.numpy(), orc.camera_from_bytes(bytes(cam)), 256, (0, 0, 0, 1, 1, 1), 2048, rays)
    check_subset((rgb[0][rays], rgba[0][rays], counts[0][rays], comp[0][rays]), want, "C4 1920x1080")


def test_c5_eight_views_one_call_full_size():
    announce("full-size C5 render: 8 x 1280x720 in one call, 5 x 128^3 cascades + shell, T=2^21, <=4096 steps; 375 rays per view")
    box = (-1.0, -1.0, -1.0, 1.0, 1.0, 1.0)
    g = ext.scene_gaussians(512, seed=5, centre=(-16.0, 16.0), sigma=(0.3, 1.5), amplitude=(5.0, 50.0))
    bits = ext.occupancy_from_scene(g, 128, 0.01, box[:3], box[3:], 5, shell=((0.0, 0.0, 0.0), 12.0, 15.5))
    desc = ext.grid_desc(21, L.NERF_EXT_F16)
    model = ext.Model.create(desc, seed=0)
    occ = ext.occupancy_struct(bits, 128, box[:3], box[3:], 5)
    cams = [ext.camera_orbit(5, i, 4.0, (0.0, 0.0, 0.0), 1280, 720, 1111.0 * 1280 / 800.0) for i in range(8)]
    rgba, rgb, counts, comp, shaded, stats = render_full(model, occ, cams, 4096)
    assert stats.samples == int(counts.sum()) and stats.samples_shaded == int(shaded.sum())
    assert np.all(shaded >= comp) and np.all(comp <= counts)
    b = bits.numpy()
    stopped = 0
    for v in range(8):
        rays = subset(1280 * 720, 375, 10 + v)
        want = oracle_subset(desc, model, b, orc.camera_from_bytes(bytes(cams[v])), 128, box, 4096, rays, cascades=5)
        stopped += check_subset((rgb[v][rays], rgba[v][rays], counts[v][rays], comp[v][rays]), want, f"C5 view {v}")
    # The random-init field is a medium of density about 1: every ray that
    # crosses the scene stops, between 1,400 and 1,900 samples in.
    assert stopped > 0.9 * 8 * 375
    hit = comp > 0
    waste = (shaded[hit].astype(np.int64) - comp[hit]).mean()
    print(f"[stop] C5: shaded {stats.samples_shaded / counts.size:.1f} per ray, composited {comp.mean():.1f}, waste {waste:.1f} per ray", flush=True)
