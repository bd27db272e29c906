"""GPU MLP parity (fp16 MFMA, fp32 accumulate) against the oracle (fp16
rounding points, fp64 accumulation): within 1e-3 relative."""
import numpy as np
import pytest

from conftest import announce
from helpers import L, ext, orc, DeviceArray, synchronize, byref, oracle_grid, host_table, host_params, points, unit_dirs, assert_rel

pytestmark = pytest.mark.gpu


def test_density_mlp_on_features():
    n = 4099  # ragged: not a multiple of 16
    announce(f"density mlp n={n}")
    rng = np.random.default_rng(11)
    feat = rng.normal(0, 1, (n, 32)).astype(np.float16)
    w = ext.mlp_init(0).astype(np.float16)
    d_w = DeviceArray.from_numpy(w)
    d_f = DeviceArray.from_numpy(feat)
    d_o = DeviceArray((n, 16), np.float32)
    L.call("nerf_ext_density_mlp", d_w.ptr, d_f.ptr, n, d_o.ptr, None)
    synchronize()
    want = orc.density_mlp(w.view(np.uint16), feat.astype(np.float32))
    assert_rel(d_o.numpy(), want, what="density mlp", mlp=True)


def test_density_mlp_structured_weights():
    """Identity-like weights: output k is relu(feature k) — checks MFMA operand layouts row by row."""
    n = 64
    announce("density mlp identity weights")
    W1 = np.zeros((64, 32), np.float32)
    W1[:32, :32] = np.eye(32)
    W1[32:, :] = -np.eye(32)
    W2 = np.zeros((16, 64), np.float32)
    W2[:, :16] = np.eye(16)
    W2[:, 32:48] += 0.5 * np.eye(16)[:, :16][:, ::-1]
    w = np.concatenate([W1.ravel(), W2.ravel()]).astype(np.float16)
    rng = np.random.default_rng(12)
    feat = rng.normal(0, 2, (n, 32)).astype(np.float16)
    d_w, d_f, d_o = DeviceArray.from_numpy(w), DeviceArray.from_numpy(feat), DeviceArray((n, 16), np.float32)
    L.call("nerf_ext_density_mlp", d_w.ptr, d_f.ptr, n, d_o.ptr, None)
    synchronize()
    x = feat.astype(np.float32)
    want = np.maximum(x[:, :16], 0) + 0.5 * np.maximum(-x[:, 15::-1], 0)
    np.testing.assert_allclose(d_o.numpy(), want, rtol=1e-3, atol=1e-3)
    np.testing.assert_allclose(d_o.numpy(), orc.density_mlp(w.view(np.uint16), x), rtol=1e-6, atol=1e-6)


@pytest.mark.parametrize("n", [1 << 16, 1000])
def test_density_forward_hash_grid_f32_2p16(n):
    """Hash encode + density MLP, 16 levels x 2 fp32 features, T = 2^16, points
    from seed 0; output (exp(raw0), raw1..15)."""
    announce(f"density forward n={n}")
    desc = ext.grid_desc(16, L.NERF_EXT_F32)
    model = ext.Model.create(desc, seed=0)
    pos = points(n, seed=0)
    d_pos = DeviceArray.from_numpy(pos)
    d_o = DeviceArray((n, 16), np.float32)
    L.call("nerf_ext_density_forward", byref(desc), model.table.ptr, model.density.ptr, d_pos.ptr, n, d_o.ptr, None)
    synchronize()
    want = orc.density_forward(oracle_grid(desc), host_table(model), host_params(model)[0], pos)
    assert_rel(d_o.numpy(), want, what="density forward", mlp=True)


def test_density_forward_large_table_values():
    """A table with O(1) entries drives hidden activations across the fp16 range."""
    n = 8192
    announce(f"density forward O(1) table n={n}")
    desc = ext.grid_desc(16, L.NERF_EXT_F32)
    model = ext.Model.create(desc, seed=5, table_range=1.0)
    pos = points(n, seed=2)
    d_pos, d_o = DeviceArray.from_numpy(pos), DeviceArray((n, 16), np.float32)
    L.call("nerf_ext_density_forward", byref(desc), model.table.ptr, model.density.ptr, d_pos.ptr, n, d_o.ptr, None)
    synchronize()
    want = orc.density_forward(oracle_grid(desc), host_table(model), host_params(model)[0], pos)
    assert_rel(d_o.numpy(), want, what="density forward O(1) table", mlp=True)


@pytest.mark.parametrize("log2_t,dtype", [(19, L.NERF_EXT_F16), (16, L.NERF_EXT_F32)])
def test_field_forward(log2_t, dtype):
    n = 8195
    announce(f"field forward n={n} log2_t={log2_t}")
    desc = ext.grid_desc(log2_t, dtype)
    model = ext.Model.create(desc, seed=1, table_range=0.5)
    pos = points(n, seed=3)
    dirs = unit_dirs(n, seed=4)
    d_pos, d_dir, d_o = DeviceArray.from_numpy(pos), DeviceArray.from_numpy(dirs), DeviceArray((n, 4), np.float32)
    ms = model.struct()
    L.call("nerf_ext_field_forward", byref(ms), d_pos.ptr, d_dir.ptr, n, d_o.ptr, None)
    synchronize()
    dp, cp = host_params(model)
    want = orc.field_forward(oracle_grid(desc), host_table(model), dp, cp, pos, dirs)
    assert_rel(d_o.numpy(), want, what="field forward", mlp=True)


@pytest.mark.parametrize("log2_t,dtype", [(19, L.NERF_EXT_F16), (17, L.NERF_EXT_F32)])
def test_field_forward_level_major_launch(log2_t, dtype):
    # More than 2^20 points take the level-major field kernel (renders); the
    # smaller launches above take the tile kernel.  Rows compared with the
    # oracle on a sample; the first 2^20 rows bit for bit with the tile
    # kernel (the same fp32 feature sums in the oracle's order, the same MFMA
    # chain), whatever lanes fetch which corners.
    n = (1 << 20) + 4099
    announce(f"field forward level-major n={n} log2_t={log2_t} dtype={dtype}")
    desc = ext.grid_desc(log2_t, dtype)
    model = ext.Model.create(desc, seed=2, table_range=0.5)
    pos = points(n, seed=13)
    dirs = unit_dirs(n, seed=14)
    d_pos, d_dir, d_o = DeviceArray.from_numpy(pos), DeviceArray.from_numpy(dirs), DeviceArray((n, 4), np.float32)
    ms = model.struct()
    L.call("nerf_ext_field_forward", byref(ms), d_pos.ptr, d_dir.ptr, n, d_o.ptr, None)
    d_tile = DeviceArray((1 << 20, 4), np.float32)
    L.call("nerf_ext_field_forward", byref(ms), d_pos.ptr, d_dir.ptr, 1 << 20, d_tile.ptr, None)
    synchronize()
    got = d_o.numpy()
    rows = np.unique(np.concatenate([np.random.default_rng(5).integers(0, n, 4000), np.arange(n - 70, n)]))
    dp, cp = host_params(model)
    want = orc.field_forward(oracle_grid(desc), host_table(model), dp, cp, np.ascontiguousarray(pos[rows]), np.ascontiguousarray(dirs[rows]))
    assert_rel(got[rows], want, what="field forward (level-major)", mlp=True)
    tile = d_tile.numpy()
    diff = np.count_nonzero(got[: 1 << 20].view(np.uint32) != tile.view(np.uint32))
    assert diff == 0, f"{diff} values differ between the level-major and the tile kernel"


@pytest.mark.parametrize("n", [65536, 1000])
def test_field_mlp_on_features(n):
    announce(f"field mlp on features n={n}")
    rng = np.random.default_rng(11)
    feats = rng.uniform(-1.0, 1.0, size=(n, 32)).astype(np.float16)
    dirs = unit_dirs(n, seed=12)
    dp = orc.f32_to_f16_bits(orc.mlp_init(0))
    cp = orc.f32_to_f16_bits(orc.mlp_init(1))
    d_f, d_d, d_o = DeviceArray.from_numpy(feats), DeviceArray.from_numpy(dirs), DeviceArray((n, 4), np.float32)
    d_dp, d_cp = DeviceArray.from_numpy(dp), DeviceArray.from_numpy(cp)
    L.call("nerf_ext_field_mlp", d_dp.ptr, d_cp.ptr, d_f.ptr, d_d.ptr, n, d_o.ptr, None)
    synchronize()
    want = orc.field_mlp(dp, cp, feats.astype(np.float32), dirs)
    assert_rel(d_o.numpy(), want, what="field mlp", mlp=True)


@pytest.mark.parametrize("log2_t", [17, 19])
def test_split_encode_then_mlp_equals_fused_field(log2_t):
    """The sparse training forward (level-split encode into fp16 features,
    then the MLP pass) gives the fused tile kernel's outputs bit for bit:
    same corner entries, weights and summation order, same fp16 rounding of
    the features and SH coefficients, same MFMA chain.  T = 2^17 takes four
    levels per XCD, T = 2^19 two."""
    n = 1 << 16
    announce(f"split encode + field mlp vs fused field forward, T=2^{log2_t}, n={n}")
    desc = ext.grid_desc(log2_t, L.NERF_EXT_F16)
    model = ext.Model.create(desc, seed=2, table_range=1.0)
    pos, dirs = points(n, seed=21), unit_dirs(n, seed=22)
    d_pos, d_dir = DeviceArray.from_numpy(pos), DeviceArray.from_numpy(dirs)
    feats = DeviceArray((n, 32), np.float16)
    split, fused = DeviceArray((n, 4), np.float32), DeviceArray((n, 4), np.float32)
    ext.encode_forward(desc, model.table, d_pos, n, feats)
    L.call("nerf_ext_field_mlp", model.density.ptr, model.color.ptr, feats.ptr, d_dir.ptr, n, split.ptr, None)
    L.call("nerf_ext_field_forward", byref(model.struct()), d_pos.ptr, d_dir.ptr, n, fused.ptr, None)
    synchronize()
    diff = np.count_nonzero(split.numpy().view(np.uint32) != fused.numpy().view(np.uint32))
    assert diff == 0, f"{diff} of {4 * n} values differ"
