"""The oracle's restatement of the reference's inference sampling and
composite (backend-cuda.cu:534-635), pinned by closed forms.

* A constant medium: every sample has the same sigma and colour, so the
  composite over the chord of length L through the box is
  c (1 - e^{-sigma L}) + e^{-sigma L} over white, whatever the sample count;
  the axis camera's chord is exactly [2, 3].
* A ray that misses the box has no samples and shows the background.
* A density that grows along the ray (the reference network with weights that
  carry the x coordinate to the raw density): the transmittance is the
  midpoint-rule sum over samples at t_near + (i + 1/2) dt, which a shifted
  placement (t_near + i dt) misses by several percent.
"""
import math

import numpy as np

from oracle import oracle as orc
from refmodel_cases import COLOR_SHAPES, DENSITY_SHAPES, pack

BOX = (0.0, 0.0, 0.0, 1.0, 1.0, 1.0)


def _axis_camera(origin, rot_rows, fx=1.0):
    """2x2-pixel camera whose pixel (0, 0) looks along its -z axis (cx = cy =
    0.5 with pixel centres and the row flip), pixel (1, 0) far off axis."""
    c2w = []
    for r in range(3):
        c2w += list(rot_rows[r]) + [origin[r]]
    return orc.camera(c2w, fx, fx, 0.5, 0.5, 2, 2)


DOWN_Z = ((1, 0, 0), (0, 1, 0), (0, 0, 1))          # looks along -z
ALONG_MINUS_X = ((0, 0, 1), (0, 1, 0), (-1, 0, 0))  # looks along -x


def _zero_models():
    grid = orc.make_grid(16, 12, 1)
    table = np.zeros(16 * (1 << 12) * 2, np.uint16)
    hd = np.zeros(orc.lib().orc_mlp_param_count(0), np.uint16)
    hc = np.zeros(orc.lib().orc_mlp_param_count(1), np.uint16)
    rd = np.zeros(orc.ref_param_count(0), np.uint16)
    rc = np.zeros(orc.ref_param_count(1), np.uint16)
    # zero raw outputs: hash grid sigma = exp(0) = 1, reference sigma =
    # softplus(0) = ln 2; rgb = sigmoid(0) = 1/2 for both.
    return [(dict(grid=grid, table=table, dp=hd, cp=hc, kind=0), 1.0), (dict(grid=None, table=None, dp=rd, cp=rc, kind=1), math.log(2.0))]


def _render(m, cam, spp, rays):
    return orc.render_uniform(m["grid"], m["table"], m["dp"], m["cp"], cam, BOX, spp, np.asarray(rays, np.uint32), kind=m["kind"])


def test_constant_medium_closed_form():
    cam = _axis_camera((0.5, 0.5, 3.0), DOWN_Z, fx=0.1)
    for m, sigma in _zero_models():
        for spp in (1, 7, 64, 300):
            rgb, rgba, counts = _render(m, cam, spp, [0, 1])
            assert counts.tolist() == [spp, 0]
            T = math.exp(-sigma * 1.0)
            want = 0.5 * (1.0 - T) + T
            np.testing.assert_allclose(rgb[0], [want] * 3, rtol=2e-6 * max(1, spp / 10))
            assert rgb[1].tolist() == [1.0, 1.0, 1.0], "a ray that misses the box shows the background"
            assert rgba[1] == 0xFFFFFFFF
            assert (rgba[0] & 0xFF) == int(np.rint(np.float32(want) * 255.0))


def _x_density_weights():
    """Density hidden neuron 0 = relu(x) (the first position-encoding value is
    x itself), carried by identity layers to raw density output 0; colour
    weights zero (rgb 1/2)."""
    d = [np.zeros(s, np.float32) for s in DENSITY_SHAPES]
    d[0][0, 0] = 1.0
    for k in range(1, 5):
        d[k][:, :] = np.eye(128)
    d[5][0, 0] = 1.0
    c = [np.zeros(s, np.float32) for s in COLOR_SHAPES]
    return pack(d), pack(c)


def _softplus(x):
    return x if x > 20 else (math.exp(x) if x < -20 else math.log1p(math.exp(x)))


def test_midpoint_sample_placement():
    dp, cp = _x_density_weights()
    m = dict(grid=None, table=None, dp=dp, cp=cp, kind=1)
    cam = _axis_camera((3.0, 0.5, 0.5), ALONG_MINUS_X)  # enters x = 1 at t = 2, leaves x = 0 at t = 3
    for spp in (4, 8, 32):
        rgb, _, counts = _render(m, cam, spp, [0])
        assert counts[0] == spp
        dt = 1.0 / spp

        def transmittance(offset):
            s = 0.0
            for i in range(spp):
                x = np.float32(3.0) - np.float32(np.float32(2.0) + np.float32((i + offset) * dt))
                s += _softplus(float(np.float16(x))) * dt
            return math.exp(-s)

        mid, left = transmittance(0.5), transmittance(0.0)
        got_T = 2.0 * float(rgb[0][0]) - 1.0  # rgb = 1/2 (1 - T) + T
        assert abs(got_T - mid) < 1e-5, (spp, got_T, mid)
        assert abs(left - mid) > 50 * abs(got_T - mid), "the test would not see a shifted placement"
