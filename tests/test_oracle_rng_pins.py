"""Bit-exact pins of the oracle's training RNG and its Huber loss value.

The reference's integer recurrences are restated here in numpy uint32,
independently of the oracle, and compared with the oracle's outputs bit for
bit:
- hash_u32 (backend-cuda.cu:321-327, == :1439-1446);
- rand01's low-24-bit select and scale (:329-332), on seeds chosen through
  the inverse hash so that the low and high 24 bits of the hash differ (a
  `h >> 8` for `h & 0xFFFFFF` slip fails);
- the per-ray seed `frame * 1315423911 ^ ray * 9781` and the two pixel draws
  with 0xA511E9B3 / 0x63D83595 (:438-440), through orc_train_rays' pixel
  outputs over several frames;
- the camera pick `hash_u32(frame * 747796405 + 2891336453) % count` (:1482)
  over 20,000 frames.
The Huber loss value (Huber 1964, delta 0.1) of a one-sample ray is checked
against its closed form in both branches, together with the clamped
gradient the same closed form gives.
"""
import numpy as np

from oracle import oracle as orc

U32 = np.uint32


def hash_u32_np(x: np.ndarray) -> np.ndarray:
    """backend-cuda.cu:321-327 in numpy uint32 (wrapping multiplies)."""
    x = np.asarray(x, U32).copy()
    with np.errstate(over="ignore"):
        x ^= x >> U32(16)
        x *= U32(0x7FEB352D)
        x ^= x >> U32(15)
        x *= U32(0x846CA68B)
        x ^= x >> U32(16)
    return x


def rand01_np(seed: np.ndarray) -> np.ndarray:
    """backend-cuda.cu:329-332: float(h & 0xFFFFFF) / float(2^24), both in fp32."""
    h = hash_u32_np(seed)
    return (h & U32(0x00FFFFFF)).astype(np.float32) / np.float32(16777216.0)


def _inverse_hash_u32(y: int) -> int:
    m = 0xFFFFFFFF

    def unxorshift(v, s):
        r = v
        for _ in range(32 // s + 1):
            r = v ^ (r >> s)
        return r & m

    y = unxorshift(y, 16)
    y = (y * pow(0x846CA68B, -1, 2 ** 32)) & m
    y = unxorshift(y, 15)
    y = (y * pow(0x7FEB352D, -1, 2 ** 32)) & m
    return unxorshift(y, 16)


def test_hash_u32_restated_matches_oracle():
    rng = np.random.default_rng(5)
    xs = np.concatenate([rng.integers(0, 2 ** 32, 20000, dtype=np.uint64).astype(U32), np.array([0, 1, 0xFFFFFFFF, 0x80000000, 0x12345678], U32)])
    want = hash_u32_np(xs)
    h = orc.lib().orc_hash_u32
    got = np.array([h(int(x)) for x in xs], U32)
    assert np.array_equal(got, want)


def test_rand01_low_24_bits():
    # Hash values whose low 24 bits and high 24 bits differ widely, reached
    # through the inverse hash.
    targets = [0x00FFFFFF, 0xFF000000, 0xFF000001, 0x12345678, 0xABCDEF01, 0x80000000, 0x00000001, 0xFFFFFFFF, 0x01000000, 0x7F00FF00]
    seeds = np.array([_inverse_hash_u32(t) for t in targets], U32)
    assert np.array_equal(hash_u32_np(seeds), np.array(targets, U32))
    r = orc.lib().orc_rand01
    got = np.array([r(int(s)) for s in seeds], np.float32)
    want = np.array([(t & 0xFFFFFF) / 16777216.0 for t in targets], np.float32)
    assert np.array_equal(got.view(U32), want.view(U32))
    # The high-bit select would give different values on every target whose
    # low and high 24 bits differ.
    wrong = np.array([(t >> 8) / 16777216.0 for t in targets], np.float32)
    assert np.sum(got != wrong) >= 9
    # And on a dense range of seeds, against the numpy restatement.
    seeds = np.arange(0, 40000, dtype=U32) * U32(2654435761 & 0xFFFF) + U32(17)
    got = np.array([r(int(s)) for s in seeds], np.float32)
    assert np.array_equal(got.view(U32), rand01_np(seeds).view(U32))


def _train_pixels_np(frame: int, n: int, w: int, h: int):
    r = np.arange(n, dtype=U32)
    with np.errstate(over="ignore"):
        seed = (U32(frame) * U32(1315423911)) ^ (r * U32(9781))
    px = rand01_np(seed ^ U32(0xA511E9B3)) * np.float32(w)
    py = rand01_np(seed ^ U32(0x63D83595)) * np.float32(h)
    return px.astype(np.float32), py.astype(np.float32)


def test_train_ray_pixels_restated():
    w, h = 800, 600
    c2w = [1, 0, 0, 0.5, 0, 1, 0, 0.5, 0, 0, 1, 2.0]
    cam = orc.camera(c2w, 700.0, 700.0, 0.5 * (w - 1), 0.5 * (h - 1), w, h)
    img = np.full((h, w, 4), 255, np.uint8)
    n = 3000
    for frame in (0, 1, 7, 1000, 123457, 0xFFFFFFF0):
        _, _, pix, _, _ = orc.train_rays(cam, img, None, 1, (0, 0, 0, 1, 1, 1), 4, frame, n, n * 4)
        px, py = _train_pixels_np(frame, n, w, h)
        assert np.array_equal(pix[:, 0].view(U32), px.view(U32)), frame
        assert np.array_equal(pix[:, 1].view(U32), py.view(U32)), frame
    # A regrouped seed ((frame * 1315423911) ^ ray) * 9781 differs, so this
    # restatement tells the two apart.
    r = np.arange(n, dtype=U32)
    with np.errstate(over="ignore"):
        regrouped = ((U32(7) * U32(1315423911)) ^ r) * U32(9781)
    alt = rand01_np(regrouped ^ U32(0xA511E9B3)) * np.float32(w)
    assert np.mean(alt != _train_pixels_np(7, n, w, h)[0]) > 0.99


def test_train_camera_restated():
    frames = np.arange(20000, dtype=U32)
    for count in (1, 7, 100, 1000):
        with np.errstate(over="ignore"):
            want = hash_u32_np(frames * U32(747796405) + U32(2891336453)) % U32(count)
        got = np.array([orc.train_camera(int(f), count) for f in frames], U32)
        assert np.array_equal(got, want), count
    # Frames near the wrap of the u32 frame counter.
    top = np.arange(0xFFFFFF00, 0x100000000, dtype=np.uint64).astype(U32)
    with np.errstate(over="ignore"):
        want = hash_u32_np(top * U32(747796405) + U32(2891336453)) % U32(100)
    assert np.array_equal(np.array([orc.train_camera(int(f), 100) for f in top], U32), want)


def _one_sample(sraw, rgbraw, dt, gt, bg):
    sigma = np.exp(np.float64(sraw))
    c = 1.0 / (1.0 + np.exp(-np.asarray(rgbraw, np.float64)))
    alpha = 1.0 - np.exp(-sigma * dt)
    pred = alpha * c + (1.0 - alpha) * np.asarray(bg, np.float64)
    return alpha, c, pred


def test_huber_closed_form_both_branches():
    delta = 0.1
    sraw, rgbraw, dt = np.float32(0.5), np.array([0.3, -1.2, 2.0], np.float32), np.float32(0.25)
    bg = (1.0, 1.0, 1.0)
    alpha, c, pred = _one_sample(sraw, rgbraw, np.float64(dt), None, bg)
    # Residuals chosen per channel: 0.04 (quadratic), -0.35 (linear, negative),
    # 0.1 - 0.02 (quadratic near delta).
    x = np.array([0.04, -0.35, 0.08])
    gt = (pred - x).astype(np.float32)
    x = pred - gt.astype(np.float64)  # the residual the fp32 ground truth leaves
    want = np.where(np.abs(x) <= delta, 0.5 * x * x, delta * (np.abs(x) - 0.5 * delta)).sum()
    for inv_norm in (1.0, 0.25):
        loss, ds, drgb, p = orc.composite_backward_ray([sraw], rgbraw, [dt], gt, bg, delta, inv_norm)
        np.testing.assert_allclose(p, pred, rtol=1e-6)
        assert abs(loss - want) <= 1e-6 * want
        # d raw_rgb = w g c (1 - c), w = alpha for the only sample, g the
        # clamped residual: -delta on the linear channel.
        g = np.clip(x, -delta, delta) * inv_norm
        assert g[1] == -delta * inv_norm
        np.testing.assert_allclose(drgb[0], alpha * g * c * (1.0 - c), rtol=1e-5)
        # d raw_sigma = dt sigma (1 - alpha) sum_c g_c (c_c - bg_c).
        sigma = np.exp(np.float64(sraw))
        want_ds = dt * sigma * (1.0 - alpha) * np.sum(g * (c - 1.0))
        np.testing.assert_allclose(ds[0], want_ds, rtol=1e-5)
    # A squared loss (delta large) and an absolute loss (delta tiny) bracket
    # the Huber value.
    loss_sq, *_ = orc.composite_backward_ray([sraw], rgbraw, [dt], gt, bg, 1e6, 1.0)
    assert abs(loss_sq - 0.5 * np.sum(x * x)) <= 1e-6 * loss_sq
    loss_abs, *_ = orc.composite_backward_ray([sraw], rgbraw, [dt], gt, bg, 1e-9, 1.0)
    assert abs(loss_abs - 1e-9 * np.sum(np.abs(x))) <= 1e-3 * loss_abs
