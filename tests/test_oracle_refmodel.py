"""Oracle pins of the reference-model mode (the reference's own network,
backend-cuda.cu:23-54): init = the reference loop restated, frequency
encoding = closed forms, softplus branches, the MLP against an fp64 numpy
GEMM with the same fp16 rounding points, and structured weights whose
outputs have closed forms (input layouts of :918-943)."""
import numpy as np

from refmodel_cases import COLOR_SHAPES, DENSITY_SHAPES, ENCODING_PROBES, encoding_probe, encoding_probe_raw, probe_points, structured, structured_raw, unit_dirs, world_points


def test_ref_init_matches_reference_loop(orc):
    for net, shapes, (a, b) in [(0, DENSITY_SHAPES, (0x1234, 0x5678)), (1, COLOR_SHAPES, (0x9ABC, 0xDEF0))]:
        total = sum(o * i for o, i in shapes)
        assert orc.ref_param_count(net) == total
        z = orc.splitmix_sequence(orc.lib().orc_stream_state(a, b), total)
        u = ((z >> np.uint64(32)).astype(np.uint32) >> np.uint32(8)).astype(np.float32) * np.float32(1.0 / 16777216.0)
        want, off = [], 0
        for o, i in shapes:
            scale = np.sqrt(np.float32(6.0) / np.float32(o + i)).astype(np.float32)
            want.append(((u[off:off + o * i] * np.float32(2.0) - np.float32(1.0)) * scale).astype(np.float32))
            off += o * i
        assert np.array_equal(orc.ref_mlp_init(net), np.concatenate(want))
    assert orc.ref_param_count(0) == 75776 and orc.ref_param_count(1) == 40960


def test_freq_encode_closed_forms(orc):
    # Zero: sin = 0, cos = 1 on every level.
    e = orc.freq_encode(np.zeros(3), 10)[0]
    assert e.shape == (63,)
    assert np.array_equal(e[:3], np.zeros(3)) and np.all(e[3:].reshape(10, 6)[:, :3] == 0) and np.all(e[3:].reshape(10, 6)[:, 3:] == 1)
    # pi/4 on x: level l holds sin/cos of 2^l pi/4 (x first, then y, z).
    p = np.array([np.pi / 4, 0.0, 0.0], np.float32)
    e = orc.freq_encode(p, 4)[0].reshape(-1)
    arg = [np.float32(p[0]) * np.float32(2.0 ** l) for l in range(4)]
    for l in range(4):
        assert e[3 + 6 * l] == np.float32(np.sin(np.float64(arg[l])))
        assert e[3 + 6 * l + 3] == np.float32(np.cos(np.float64(arg[l])))
        assert e[3 + 6 * l + 1] == 0 and e[3 + 6 * l + 4] == 1
    assert abs(e[3 + 6 * 1] - 1.0) < 1e-7          # sin(pi/2)
    assert abs(e[3 + 6 * 2 + 3] + 1.0) < 1e-7      # cos(pi)
    # Random points: identity first, then sin^2 + cos^2 = 1 per axis/level.
    pts = world_points(200, 1)
    e = orc.freq_encode(pts, 10)
    assert np.array_equal(e[:, :3], pts)
    lv = e[:, 3:].reshape(-1, 10, 6).astype(np.float64)
    assert np.abs(lv[..., :3] ** 2 + lv[..., 3:] ** 2 - 1).max() < 1e-6


def test_softplus_branches(orc):
    assert abs(orc.softplus(0.0) - np.log(2.0)) < 1e-7
    assert orc.softplus(25.0) == 25.0
    assert orc.softplus(-25.0) == np.float32(np.exp(-25.0))
    assert abs(orc.softplus(20.0) - 20.0) < 1e-5
    assert abs(orc.softplus(-3.0) - np.log1p(np.exp(-3.0))) < 1e-7


def _f16(x):
    return np.asarray(x, np.float32).astype(np.float16).astype(np.float32)


def _numpy_enc(pos, dirs):
    """fp16 density input (63 values + 0) and direction encoding (27)."""
    def enc(v, levels):
        args = v[:, None, :] * (np.float32(2.0) ** np.arange(levels, dtype=np.float32))[None, :, None]   # exact
        sc = np.concatenate([np.sin(args.astype(np.float64)), np.cos(args.astype(np.float64))], 2).astype(np.float32)
        return np.concatenate([v, sc.reshape(v.shape[0], -1)], 1)
    n = pos.shape[0]
    pe = _f16(np.concatenate([enc(pos, 10)[:, :63], np.zeros((n, 1), np.float32)], 1))
    return pe, _f16(enc(dirs, 4))


def _numpy_ref(dp, cp, pos, dirs):
    def net(bits, shapes, x):
        W = bits.view(np.float16).astype(np.float64)
        off = 0
        for m, (o, i) in enumerate(shapes):
            A = W[off:off + o * i].reshape(o, i)
            off += o * i
            y = (x.astype(np.float64) @ A.T).astype(np.float32)
            x = _f16(np.maximum(y, 0) if m + 1 < len(shapes) else y)
        return x
    n = pos.shape[0]
    pe, de = _numpy_enc(pos, dirs)
    dens = net(dp, DENSITY_SHAPES, pe)
    ci = np.concatenate([dens[:, 1:16], de, np.zeros((n, 6), np.float32)], 1)
    col = net(cp, COLOR_SHAPES, ci)
    raw = np.stack([dens[:, 0], col[:, 0], col[:, 1], col[:, 2]], 1)
    x = raw[:, 0].astype(np.float64)
    sp = np.where(x > 20, x, np.where(x < -20, np.exp(x), np.log1p(np.exp(np.clip(x, -20, 20)))))
    out = np.concatenate([sp[:, None], 1.0 / (1.0 + np.exp(-raw[:, 1:].astype(np.float64)))], 1)
    return out.astype(np.float32), raw


def test_ref_field_matches_fp64_numpy(orc):
    dp = orc.f32_to_f16_bits(orc.ref_mlp_init(0) * 1.5)   # larger weights: raw outputs of order 1
    cp = orc.f32_to_f16_bits(orc.ref_mlp_init(1) * 1.5)
    pos, dirs = world_points(300, 2), unit_dirs(300, 3)
    out, raw = orc.ref_field_forward(dp, cp, pos, dirs)
    want_out, want_raw = _numpy_ref(dp, cp, pos, dirs)
    # fp64 accumulation on both sides; a rare fp16 tie of a hidden activation
    # may round differently in the last place.
    scale = np.abs(want_raw).max()
    assert np.abs(raw - want_raw).max() <= 2e-3 * scale
    assert np.median(np.abs(raw - want_raw)) == 0.0
    np.testing.assert_allclose(out, want_out, rtol=2e-3, atol=1e-5)


def test_ref_structured_weights_closed_form(orc):
    dp, cp = structured()
    pos = world_points(500, 4, 0.05, 1.5)          # x > 0
    dirs = unit_dirs(500, 5)
    _, raw = orc.ref_field_forward(dp, cp, pos, dirs)
    assert np.array_equal(raw, structured_raw(pos, dirs))


def _ray(n, seed):
    rng = np.random.default_rng(seed)
    return (rng.normal(0, 2, n).astype(np.float32), rng.normal(0, 2, (n, 3)).astype(np.float32), rng.uniform(0.001, 0.05, n).astype(np.float32),
            np.array([*rng.uniform(0, 1, 3), rng.uniform(0, 1)], np.float32))


def test_ref_composite_backward_finite_differences(orc):
    # Central differences of the fp64 loss in the raw inputs (h on the fp32 grid).
    for n, seed in ((1, 1), (7, 2), (150, 3)):
        s, c, dt, gt = _ray(n, seed)
        loss, ds, dc, _ = orc.ref_composite_backward_ray(s, c, dt, gt, inv_norm=1.0)
        for i in range(0, n, max(1, n // 10)):
            for k in (-1, 0, 1, 2):
                h = np.float32(1e-2)
                sp, sm, cp_, cm = s.copy(), s.copy(), c.copy(), c.copy()
                if k < 0:
                    sp[i] += h; sm[i] -= h
                    h_eff = (np.float64(sp[i]) - np.float64(sm[i])) / 2
                    got = ds[i]
                else:
                    cp_[i, k] += h; cm[i, k] -= h
                    h_eff = (np.float64(cp_[i, k]) - np.float64(cm[i, k])) / 2
                    got = dc[i, k]
                lp = orc.ref_composite_backward_ray(sp, cp_, dt, gt)[0]
                lm = orc.ref_composite_backward_ray(sm, cm, dt, gt)[0]
                fd = (lp - lm) / (2 * h_eff)
                assert abs(got - fd) <= 1e-4 * max(abs(fd), 1e-3), (n, i, k, got, fd)


def test_ref_composite_alpha_weighting_and_closed_form(orc):
    s, c, dt, gt = _ray(5, 4)
    gt1, gt0 = gt.copy(), gt.copy()
    gt1[3], gt0[3] = 1.0, 0.0
    l1 = orc.ref_composite_backward_ray(s, c, dt, gt1)[0]
    l0 = orc.ref_composite_backward_ray(s, c, dt, gt0)[0]
    assert abs(l0 / l1 - 0.1) < 1e-12           # ray weight 0.1 + 0.9 alpha (:1131-1139)
    # One sample: pred = a c + (1 - a), a = 1 - exp(-softplus(s) dt).
    s1, c1, dt1 = np.array([0.3], np.float32), np.array([[0.5, -1.0, 2.0]], np.float32), np.array([0.2], np.float32)
    g = np.array([0.2, 0.4, 0.6, 0.5], np.float32)
    a = 1 - np.exp(-np.log1p(np.exp(np.float64(np.float32(0.3)))) * np.float64(np.float32(0.2)))
    col = 1 / (1 + np.exp(-c1[0].astype(np.float64)))
    pred = a * col + (1 - a)
    loss, _, dc, p = orc.ref_composite_backward_ray(s1, c1, dt1, g, inv_norm=0.5)
    w = 0.1 + 0.9 * np.float64(np.float32(0.5))
    assert abs(loss - w * np.sum((pred - g[:3].astype(np.float64)) ** 2)) < 1e-12
    np.testing.assert_allclose(dc[0], a * 2 * w * (pred - g[:3]) * 0.5 * col * (1 - col), rtol=1e-6)


def _numpy_ref_backward(dp, cp, pos, dirs, draw, ls):
    """Matrix-form backward over the batch, same fp16 rounding points."""
    def fwd(bits, shapes, x):
        W = bits.view(np.float16).astype(np.float64)
        acts, Ws, off = [x], [], 0
        for m, (o, i) in enumerate(shapes):
            A = W[off:off + o * i].reshape(o, i)
            off += o * i
            Ws.append(A)
            y = (acts[-1].astype(np.float64) @ A.T).astype(np.float32)
            acts.append(_f16(np.maximum(y, 0) if m + 1 < len(shapes) else y))
        return acts, Ws

    def bwd(acts, Ws, delta):
        dWs, din = [None] * len(Ws), None
        for m in reversed(range(len(Ws))):
            a = acts[m].astype(np.float64)
            dWs[m] = delta.astype(np.float64).T @ a
            din = delta.astype(np.float64) @ Ws[m]
            if m > 0:
                delta = np.where(a > 0, _f16(din.astype(np.float32)), 0).astype(np.float32)
        return np.concatenate([w.ravel() for w in dWs]), din

    n = pos.shape[0]
    pe, de = _numpy_enc(pos, dirs)
    dacts, dWs = fwd(dp, DENSITY_SHAPES, pe)
    ci = np.concatenate([dacts[-1][:, 1:16], de, np.zeros((n, 6), np.float32)], 1)
    cacts, cWs = fwd(cp, COLOR_SHAPES, ci)
    dc = np.zeros((n, 16), np.float32)
    dc[:, :3] = _f16(np.float32(ls) * draw[:, 1:4])
    gC, cdin = bwd(cacts, cWs, dc)
    dd = np.zeros((n, 16), np.float32)
    dd[:, 0] = _f16(np.float32(ls) * draw[:, 0])
    dd[:, 1:16] = _f16(cdin[:, :15].astype(np.float32))
    gD, _ = bwd(dacts, dWs, dd)
    return gD, gC


def test_ref_mlp_backward_matches_matrix_form(orc):
    dp = orc.f32_to_f16_bits(orc.ref_mlp_init(0) * 1.5)
    cp = orc.f32_to_f16_bits(orc.ref_mlp_init(1) * 1.5)
    n = 60
    pos, dirs = world_points(n, 7), unit_dirs(n, 8)
    draw = np.random.default_rng(9).normal(0, 1e-2, (n, 4)).astype(np.float32)
    dD, dC = orc.ref_mlp_backward(dp, cp, pos, dirs, draw, loss_scale=128.0)
    gD, gC = _numpy_ref_backward(dp, cp, pos, dirs, draw, 128.0)
    for got, want, what in ((dD, gD, "density"), (dC, gC, "colour")):
        assert np.abs(want).max() > 0
        # Same rounding points; fp64 sums in different orders may put a rare
        # fp16 rounding of a delta on the other side of a tie.
        assert np.linalg.norm(got - want) <= 1e-6 * np.linalg.norm(want), what
    # Only the colour outputs 0..2 carry gradient: the last colour layer's
    # rows 3..15 have none.
    assert np.all(dC[38912 + 3 * 128:] == 0)


def test_ref_encoding_probe_weights(orc):
    # The probe weights route four encoding values to the raw outputs
    # unchanged; the oracle's network gives the numpy closed form exactly.
    pos, dirs = probe_points(500, 41), unit_dirs(504, 42)
    for d_entry, c_entries, from_dir in ENCODING_PROBES:
        dp, cp = encoding_probe(d_entry, c_entries, from_dir)
        _, raw = orc.ref_field_forward(dp, cp, pos, dirs)
        assert np.array_equal(raw, encoding_probe_raw(pos, dirs, d_entry, c_entries, from_dir)), (d_entry, c_entries, from_dir)
