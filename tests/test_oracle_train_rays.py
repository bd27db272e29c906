"""Pins of the oracle's training-ray sampler and ground-truth renderer by
closed forms: bilinear interpolation reproduces a linear ramp, transparent
pixels composite to white, the march of an all-occupied box covers [tn, tf]
with contiguous steps, and a constant-density medium gives alpha
1 - exp(-density * length)."""
import numpy as np

from oracle import oracle as orc

W, H = 48, 40
BOX = (0.0, 0.0, 0.0, 1.0, 1.0, 1.0)


def _camera(w=W, h=H):
    # A camera 1.5 units from the box centre looking at it along -z.
    c2w = [1, 0, 0, 0.5, 0, 1, 0, 0.5, 0, 0, 1, 2.0]
    return orc.camera(c2w, 60.0, 60.0, 0.5 * (w - 1), 0.5 * (h - 1), w, h)


def _ramp_image():
    img = np.zeros((H, W, 4), np.uint8)
    img[..., 0] = np.arange(W, dtype=np.uint8)[None, :] * 5
    img[..., 1] = np.arange(H, dtype=np.uint8)[:, None] * 6
    img[..., 2] = 77
    img[..., 3] = 255
    return img


def test_bilinear_reproduces_ramp():
    counts, gt, pix, offs, _ = orc.train_rays(_camera(), _ramp_image(), None, 1, BOX, 64, 3, 500, 500 * 64)
    hit = counts > 0
    assert hit.sum() > 200
    px = np.clip(pix[:, 0], 0, W - 1)
    py = np.clip(pix[:, 1], 0, H - 1)
    np.testing.assert_allclose(gt[hit, 0], (5.0 * px / 255.0)[hit], atol=2e-6)
    np.testing.assert_allclose(gt[hit, 1], (6.0 * py / 255.0)[hit], atol=2e-6)
    np.testing.assert_allclose(gt[hit, 2], 77.0 / 255.0, atol=1e-7)
    assert np.all(gt[hit, 3] == 1.0)
    # Missed rays keep the white, transparent default.
    assert np.all(gt[~hit] == np.array([1, 1, 1, 0], np.float32))
    # Offsets are the exclusive prefix sum of the counts.
    assert np.array_equal(offs, np.concatenate([[0], np.cumsum(counts)[:-1]]).astype(np.uint32))


def test_transparent_pixels_are_white():
    img = _ramp_image()
    img[..., 3] = 0
    counts, gt, _, _, _ = orc.train_rays(_camera(), img, None, 1, BOX, 64, 0, 300, 300 * 64)
    assert np.all(gt == np.array([1, 1, 1, 0], np.float32))


def test_pixels_uniform_in_image():
    _, _, pix, _, _ = orc.train_rays(_camera(), _ramp_image(), None, 1, BOX, 8, 11, 20000, 20000 * 8)
    assert pix[:, 0].min() >= 0 and pix[:, 0].max() < W and pix[:, 1].min() >= 0 and pix[:, 1].max() < H
    assert abs(pix[:, 0].mean() / W - 0.5) < 0.01 and abs(pix[:, 1].mean() / H - 0.5) < 0.01
    # Different frames draw different pixels.
    _, _, pix2, _, _ = orc.train_rays(_camera(), _ramp_image(), None, 1, BOX, 8, 12, 20000, 20000 * 8)
    assert np.mean(pix == pix2) < 0.01


def test_march_covers_ray_interval():
    steps = 4096  # large enough that no ray is cut by the step budget
    cam = _camera()
    counts, _, pix, offs, tdt = orc.train_rays(cam, _ramp_image(), None, 1, BOX, steps, 5, 200, 200 * steps)
    assert counts.min() > 0  # every ray of this camera crosses the box
    for r in range(50):
        s = tdt[offs[r]:offs[r] + counts[r]]
        t0 = s[:, 0] - 0.5 * s[:, 1]
        t1 = s[:, 0] + 0.5 * s[:, 1]
        assert np.all(s[:, 1] > 0)
        np.testing.assert_allclose(t0[1:], t1[:-1], atol=1e-5)  # contiguous steps
        # The camera sits on the axis at z = 2 looking along -z, so every ray
        # enters through the face z = 1 at t = |(dx, dy, -1)| (unit direction).
        dx = (pix[r, 0] - cam.cx) / cam.fx
        dy = (H - 1 - pix[r, 1] - cam.cy) / cam.fy
        assert abs(t0[0] - np.sqrt(dx * dx + dy * dy + 1.0)) < 1e-5
        assert counts[r] < steps


def test_train_camera_spread():
    picks = np.array([orc.train_camera(f, 7) for f in range(7000)])
    hist = np.bincount(picks, minlength=7)
    assert hist.min() > 850 and hist.max() < 1150


def test_scene_render_closed_forms():
    cam = _camera(w=9, h=7)
    # No density: white and transparent.
    empty = np.array([[0.5, 0.5, 0.5, 0.1, 0.0, 1, 0, 0]], np.float32)
    img = orc.scene_render(empty, cam, 64)
    assert np.all(img == 0x00FFFFFF)
    # A very wide Gaussian is a constant medium of density A inside the box:
    # alpha = 1 - exp(-A L), L = 1 for the axis-aligned centre ray.
    A = 0.7
    medium = np.array([[0.5, 0.5, 0.5, 1e4, A, 0.2, 0.4, 0.6]], np.float32)
    img = orc.scene_render(medium, cam, 256).view(np.uint8).reshape(7, 9, 4).astype(int)
    centre = img[3, 4]
    T = np.exp(-A * 1.0)
    assert abs(centre[3] - round((1 - T) * 255)) <= 1
    for k, c in enumerate((0.2, 0.4, 0.6)):
        assert abs(centre[k] - round(((1 - T) * c + T) * 255)) <= 1
