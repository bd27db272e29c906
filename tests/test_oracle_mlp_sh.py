"""MLP and SH pinning: an fp64 numpy GEMM with the same fp16 rounding points,
identity weights, SH orthonormality by exact quadrature, SH values on axes."""
import numpy as np


def _f16(x):
    return np.asarray(x, np.float32).astype(np.float16).astype(np.float64)


def _numpy_density(w_bits, feat):
    W = w_bits.view(np.float16).astype(np.float64)
    W1, W2 = W[:2048].reshape(64, 32), W[2048:].reshape(16, 64)
    h = _f16(np.maximum(_f16(feat) @ W1.T, 0.0).astype(np.float32))
    return (h @ W2.T).astype(np.float32)


def test_density_mlp_matches_fp64_numpy(orc):
    rng = np.random.default_rng(5)
    w = rng.uniform(-0.4, 0.4, 3072).astype(np.float16).view(np.uint16)
    feat = rng.normal(0, 1, (4000, 32)).astype(np.float32)
    got = orc.density_mlp(w, feat)
    want = _numpy_density(w, feat)
    np.testing.assert_allclose(got, want, rtol=1e-5, atol=1e-6)


def test_density_mlp_identity_weights(orc):
    W1 = np.zeros((64, 32), np.float32)
    W1[:32, :32] = np.eye(32)
    W2 = np.zeros((16, 64), np.float32)
    W2[:, :16] = np.eye(16)
    w = np.concatenate([W1.ravel(), W2.ravel()]).astype(np.float16).view(np.uint16)
    rng = np.random.default_rng(6)
    feat = rng.normal(0, 3, (100, 32)).astype(np.float32)
    got = orc.density_mlp(w, feat)
    want = np.maximum(feat[:, :16].astype(np.float16).astype(np.float32), 0)
    assert np.array_equal(got, want)


def _gauss_legendre_sphere(n_theta=16, n_phi=32):
    x, wx = np.polynomial.legendre.leggauss(n_theta)  # cos(theta)
    phi = (np.arange(n_phi) + 0.5) * 2 * np.pi / n_phi
    ct, ph = np.meshgrid(x, phi, indexing="ij")
    st = np.sqrt(1 - ct ** 2)
    d = np.stack([st * np.cos(ph), st * np.sin(ph), ct], -1).reshape(-1, 3)
    w = (wx[:, None] * np.full(n_phi, 2 * np.pi / n_phi)[None, :]).reshape(-1)
    return d.astype(np.float32), w


def test_sh4_orthonormal(orc):
    d, w = _gauss_legendre_sphere()
    Y = orc.sh4(d).astype(np.float64)
    G = (Y * w[:, None]).T @ Y
    np.testing.assert_allclose(G, np.eye(16), atol=2e-5)


def test_sh4_axis_values(orc):
    y = orc.sh4(np.array([[0, 0, 1], [1, 0, 0], [0, 1, 0]], np.float32))
    c1 = np.sqrt(3 / (4 * np.pi))
    np.testing.assert_allclose(y[0, [0, 1, 2, 3]], [0.5 / np.sqrt(np.pi), 0, c1, 0], atol=1e-6)
    np.testing.assert_allclose(y[0, 6], 0.25 * np.sqrt(5 / np.pi) * 2, rtol=1e-6)      # Y20(z=1)
    np.testing.assert_allclose(y[0, 12], 0.25 * np.sqrt(7 / np.pi) * 2, rtol=1e-6)     # Y30(z=1)
    np.testing.assert_allclose(y[1, 3], -c1, rtol=1e-6)                                # Y11 = -c x (Condon-Shortley)
    np.testing.assert_allclose(y[2, 1], -c1, rtol=1e-6)                                # Y1-1 = -c y
    np.testing.assert_allclose(y[1, 8], 0.25 * np.sqrt(15 / np.pi), rtol=1e-6)         # Y22(x=1)


def test_field_mlp_composes_with_encode(orc):
    """field_mlp(encode(x), d) reproduces field_forward(x, d) exactly."""
    g = orc.make_grid(16, 12, 0)
    table = orc.uniform_fill(0x7ab1e, 5, 16 * 4096 * 2, -0.5, 0.5)
    rng = np.random.default_rng(3)
    pos = rng.random((500, 3), dtype=np.float32)
    d = rng.normal(size=(500, 3)).astype(np.float32)
    d /= np.linalg.norm(d, axis=1, keepdims=True)
    dp = orc.f32_to_f16_bits(orc.mlp_init(0))
    cp = orc.f32_to_f16_bits(orc.mlp_init(1))
    feats = orc.encode(g, table, pos)
    assert np.array_equal(orc.field_mlp(dp, cp, feats, d), orc.field_forward(g, table, dp, cp, pos, d))
