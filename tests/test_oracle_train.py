"""Training oracle pinning: composite backward by central differences of its
own loss, hash-grid scatter-add by the adjoint identity of a linear map, MLP
backward against an fp64 matrix-form backward that is itself checked by
central differences, Adam against closed forms."""
import numpy as np
import pytest


def _ray(n, seed):
    rng = np.random.default_rng(seed)
    return (rng.normal(0.5, 1.0, n).astype(np.float32), rng.normal(0, 1.5, (n, 3)).astype(np.float32), rng.uniform(0.002, 0.05, n).astype(np.float32),
            rng.uniform(0, 1, 3).astype(np.float32))


def test_composite_forward_matches_forward_oracle(orc):
    sraw, rgbraw, dt, gt = _ray(40, 0)
    _, _, _, pred = orc.composite_backward_ray(sraw, rgbraw, dt, gt)
    s4 = np.concatenate([np.exp(sraw)[:, None], 1 / (1 + np.exp(-rgbraw))], 1).astype(np.float32)
    want, _, _ = orc.composite_ray(s4, dt, t_stop=0.0)
    np.testing.assert_allclose(pred, want, rtol=1e-5)


@pytest.mark.parametrize("delta", [0.1, 10.0])
def test_composite_backward_finite_differences(orc, delta):
    sraw, rgbraw, dt, gt = _ray(24, 1)
    _, ds, drgb, _ = orc.composite_backward_ray(sraw, rgbraw, dt, gt, delta=delta)
    eps = 1e-3

    def loss(s, r):
        return orc.composite_backward_ray(s, r, dt, gt, delta=delta)[0]

    for i in range(0, 24, 3):
        sp, sm = sraw.copy(), sraw.copy()
        sp[i] += eps
        sm[i] -= eps
        fd = (loss(sp, rgbraw) - loss(sm, rgbraw)) / (2 * eps)
        assert abs(fd - ds[i]) <= 2e-3 * max(abs(fd), 1e-3), (i, fd, ds[i])
        for c in range(3):
            rp, rm = rgbraw.copy(), rgbraw.copy()
            rp[i, c] += eps
            rm[i, c] -= eps
            fd = (loss(sraw, rp) - loss(sraw, rm)) / (2 * eps)
            assert abs(fd - drgb[i, c]) <= 2e-3 * max(abs(fd), 1e-3), (i, c, fd, drgb[i, c])


def test_encode_backward_is_adjoint_of_encode(orc):
    """<dtable, t> == <dfeat, encode(t)> for any table t: encoding is linear in the table."""
    log2_t = 12
    grid = orc.make_grid(16, log2_t, 0)
    rng = np.random.default_rng(2)
    pos = rng.random((400, 3), dtype=np.float32)
    dfeat = rng.normal(size=(400, 32)).astype(np.float32)
    dtable = orc.encode_backward(grid, pos, dfeat)
    for seed in range(3):
        t = np.random.default_rng(10 + seed).normal(size=16 * (1 << log2_t) * 2).astype(np.float32)
        lhs = float(np.dot(dtable, t.astype(np.float64)))
        rhs = float(np.sum(dfeat.astype(np.float64) * orc.encode(grid, t, pos).astype(np.float64)))
        assert abs(lhs - rhs) <= 1e-5 * max(1.0, abs(rhs))


# --- MLP backward ---------------------------------------------------------
def _unpack(dp, cp):
    D = dp.view(np.float16).astype(np.float64)
    Cw = cp.view(np.float16).astype(np.float64)
    return D[:2048].reshape(64, 32), D[2048:].reshape(16, 64), Cw[:2048].reshape(64, 32), Cw[2048:6144].reshape(64, 64), Cw[6144:].reshape(16, 64)


def _forward64(params, x, sh):
    D1, D2, C1, C2, C3 = params
    hd = np.maximum(x @ D1.T, 0)
    o = hd @ D2.T
    xc = np.concatenate([o[:, 1:16], sh, np.zeros((x.shape[0], 1))], 1)
    h1 = np.maximum(xc @ C1.T, 0)
    h2 = np.maximum(h1 @ C2.T, 0)
    o3 = h2 @ C3.T
    return o[:, 0], o3[:, :3], (hd, o, xc, h1, h2)


def _backward64(params, x, sh, ds, drgb):
    D1, D2, C1, C2, C3 = params
    _, _, (hd, o, xc, h1, h2) = _forward64(params, x, sh)
    do3 = np.zeros((x.shape[0], 16))
    do3[:, :3] = drgb
    dh2 = (do3 @ C3) * (h2 > 0)
    dh1 = (dh2 @ C2) * (h1 > 0)
    dxc = dh1 @ C1
    do = np.concatenate([ds[:, None], dxc[:, :15]], 1)
    dhd = (do @ D2) * (hd > 0)
    dx = dhd @ D1
    return dx, (dhd.T @ x, do.T @ hd, dh1.T @ xc, dh2.T @ h1, do3.T @ h2)


def test_matrix_backward_finite_differences(orc):
    """The fp64 matrix-form backward is the exact derivative of its forward."""
    rng = np.random.default_rng(3)
    params = tuple(rng.normal(0, 0.3, s) for s in [(64, 32), (16, 64), (64, 32), (64, 64), (16, 64)])
    x = rng.normal(0, 1, (5, 32))
    sh = rng.normal(0, 0.5, (5, 16))
    ds, drgb = rng.normal(size=5), rng.normal(size=(5, 3))

    def L(p, xx):
        s, r, _ = _forward64(p, xx, sh)
        return float(np.sum(ds * s) + np.sum(drgb * r))

    dx, dW = _backward64(params, x, sh, ds, drgb)
    eps = 1e-6
    for (i, j) in [(0, 0), (2, 7), (4, 31)]:
        xp, xm = x.copy(), x.copy()
        xp[i, j] += eps
        xm[i, j] -= eps
        assert abs((L(params, xp) - L(params, xm)) / (2 * eps) - dx[i, j]) < 1e-6
    for li, (a, b) in [(0, (3, 5)), (1, (0, 9)), (2, (10, 20)), (3, (7, 63)), (4, (2, 1))]:
        pp = [q.copy() for q in params]
        pm = [q.copy() for q in params]
        pp[li][a, b] += eps
        pm[li][a, b] -= eps
        assert abs((L(tuple(pp), x) - L(tuple(pm), x)) / (2 * eps) - dW[li][a, b]) < 1e-6


def test_oracle_mlp_backward_matches_matrix_form(orc):
    from nerf_amd import ext

    rng = np.random.default_rng(4)
    dp = ext.mlp_init(0).astype(np.float16).view(np.uint16)
    cp = ext.mlp_init(1).astype(np.float16).view(np.uint16)
    n = 256
    feat = rng.normal(0, 1, (n, 32)).astype(np.float16).astype(np.float32)
    d = rng.normal(size=(n, 3))
    d = (d / np.linalg.norm(d, axis=1, keepdims=True)).astype(np.float32)
    ds = rng.normal(0, 1e-3, n).astype(np.float32)
    drgb = rng.normal(0, 1e-3, (n, 3)).astype(np.float32)
    ls = 128.0
    dfeat, dD, dC = orc.mlp_backward(dp, cp, feat, d, ds, drgb, ls)
    params = _unpack(dp, cp)
    sh = orc.sh4(d).astype(np.float64)
    dx, dW = _backward64(params, feat.astype(np.float64), sh, ds.astype(np.float64) * ls, drgb.astype(np.float64) * ls)

    def close(a, b, what):
        # Weight gradients sum over the batch: relative Frobenius error (the
        # fp16 rounding points move them ~1 % from exact fp64 math; a wrong
        # index or transpose moves them by O(1)).
        err = np.linalg.norm(a - b) / (np.linalg.norm(b) + 1e-30)
        assert err < 3e-2, f"{what}: {err:.3e}"

    # Per-sample input gradients: a ReLU whose fp16-rounded activation is 0
    # while the fp64 one is not flips a mask in a few samples, so the bar is
    # on the median and the upper percentiles of the per-sample error.
    scale = np.sqrt(np.mean(dx ** 2))
    row_err = np.abs(dfeat - dx).max(axis=1) / scale
    assert np.median(row_err) < 1e-3 and np.quantile(row_err, 0.95) < 2e-2 and np.quantile(row_err, 0.98) < 5e-2, (np.median(row_err), np.quantile(row_err, 0.98))
    close(dD[:2048].reshape(64, 32), dW[0], "dD1")
    close(dD[2048:].reshape(16, 64), dW[1], "dD2")
    close(dC[:2048].reshape(64, 32), dW[2], "dC1")
    close(dC[2048:6144].reshape(64, 64), dW[3], "dC2")
    close(dC[6144:].reshape(16, 64), dW[4], "dC3")


# --- Adam -----------------------------------------------------------------
def test_adam_first_step_closed_form(orc):
    rng = np.random.default_rng(5)
    n = 1000
    w0 = rng.normal(size=n).astype(np.float32)
    g = (rng.normal(size=n) * 128).astype(np.float32)  # scaled by loss_scale 128
    w, m, v = w0.copy(), np.zeros(n, np.float32), np.zeros(n, np.float32)
    norm = float(np.linalg.norm(g / 128))
    skipped = orc.adam(w, m, v, g, 1e-2, 0.9, 0.99, 1e-15, 1e9, 1e9, 128.0, 0, 1, norm)
    assert skipped == 0
    # t = 1: m_hat = g, v_hat = g^2 -> step = lr * g / |g| = lr * sign(g)
    np.testing.assert_allclose(w, w0 - 1e-2 * np.sign(g), rtol=0, atol=2e-6)
    np.testing.assert_allclose(m, 0.1 * g / 128, rtol=1e-6)
    np.testing.assert_allclose(v, 0.01 * (g / 128) ** 2, rtol=1e-5)


def test_adam_guard_clip_decay(orc):
    n = 10
    g = np.full(n, 2.0, np.float32)
    w, m, v = np.zeros(n, np.float32), np.zeros(n, np.float32), np.zeros(n, np.float32)
    assert orc.adam(w, m, v, g, 1e-2, 0.9, 0.99, 1e-8, 1.0, 5.0, 1.0, 0, 1, 6.0) == 1       # norm > guard: skipped
    assert orc.adam(w, m, v, g, 1e-2, 0.9, 0.99, 1e-8, 1.0, 5.0, 1.0, 0, 1, float("nan")) == 1
    assert orc.adam(w, m, v, g, 1e-2, 0.9, 0.99, 1e-8, 1.0, 5.0, 1.0, 0, 1, 1.0, 1) == 1
    assert np.all(w == 0) and np.all(m == 0)
    # clip: norm 4 > clip 1 -> grads scaled by 1/4; first step still lr * sign
    assert orc.adam(w, m, v, g, 1e-2, 0.9, 0.99, 1e-8, 1.0, 5.0, 1.0, 0, 1, 4.0) == 0
    np.testing.assert_allclose(m, 0.1 * 0.5, rtol=1e-6)
    # lr decay: 0.1 ** (t / (k * 1000)) with k = 1, t = 500 -> lr * 10^-0.5
    w2, m2, v2 = np.zeros(n, np.float32), np.zeros(n, np.float32), np.zeros(n, np.float32)
    orc.adam(w2, m2, v2, g, 1e-2, 0.0, 0.0, 0.0, 1e9, 1e9, 1.0, 1, 500, 1.0)
    np.testing.assert_allclose(w2, -1e-2 * 10 ** -0.5, rtol=1e-5)
