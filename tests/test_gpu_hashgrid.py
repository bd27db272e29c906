"""GPU hash-grid parity: table init and indices bit-exact, features against
the oracle (the level-major kernel performs the oracle's exact fp32 sequence,
so they are expected bit-identical; the bar asserted is 1e-6 relative)."""
import numpy as np
import pytest

from conftest import announce
from helpers import L, ext, orc, DeviceArray, synchronize, byref, oracle_grid, points

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("dtype", [L.NERF_EXT_F32, L.NERF_EXT_F16])
def test_table_init_bit_exact(dtype):
    announce(f"table init dtype={dtype} T=2^16")
    desc = ext.grid_desc(16, dtype)
    table = ext.init_table(desc, seed=0)
    synchronize()
    got = table.numpy()
    want = orc.uniform_fill(0x7AB1E, 0, ext.table_elements(desc), -1e-4, 1e-4)
    if dtype == L.NERF_EXT_F32:
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    else:
        assert np.array_equal(got.view(np.uint16), orc.f32_to_f16_bits(want))


@pytest.mark.parametrize("log2_t,finest", [(16, 0), (19, 0), (22, 4096)])
def test_indices_bit_exact(log2_t, finest):
    n = 1 << 14
    announce(f"encode indices n={n} log2_t={log2_t} finest={finest}")
    desc = ext.grid_desc(log2_t, L.NERF_EXT_F32, per_level_scale=0.0 if finest else 1.3819, finest=finest)
    pos = points(n)
    pos[:6] = [[0, 0, 0], [1, 1, 1], [1, 0, 0.5], [-0.25, 1.25, 0.5], [0.5, 0.5, 0.5], [0.999999, 1e-7, 1]]
    d_pos = DeviceArray.from_numpy(pos)
    d_idx = DeviceArray((n, 16, 8), np.uint32)
    d_w = DeviceArray((n, 16, 8), np.float32)
    L.call("nerf_ext_encode_indices", byref(desc), d_pos.ptr, n, d_idx.ptr, d_w.ptr, None)
    synchronize()
    g = oracle_grid(desc)
    _, idx, w = orc.encode(g, np.zeros(16 * (1 << log2_t) * 2, np.float32), pos, with_indices=True)
    assert np.array_equal(d_idx.numpy(), idx)
    assert np.array_equal(d_w.numpy().view(np.uint32), w.view(np.uint32))


# Launch shapes covered: four levels per XCD (fp32 T = 2^16, fp16 T = 2^17),
# two levels per XCD (fp32 T = 2^17 and 2^18, fp16 T = 2^19), all levels per
# workgroup (fp16 T = 2^20); point counts that are and are not multiples of
# the 256-point blocks.
@pytest.mark.parametrize(
    "table_dtype,out_dtype,log2_t,n",
    [
        (L.NERF_EXT_F32, np.float32, 16, 1 << 16),
        (L.NERF_EXT_F32, np.float32, 16, 1000),
        (L.NERF_EXT_F16, np.float16, 17, 777),
        (L.NERF_EXT_F32, np.float32, 17, 3001),
        (L.NERF_EXT_F16, np.float32, 19, 1 << 16),
        (L.NERF_EXT_F16, np.float16, 19, 1 << 16),
        (L.NERF_EXT_F32, np.float32, 18, 4099),
        (L.NERF_EXT_F16, np.float16, 20, 5000),
    ],
)
def test_encode_forward(table_dtype, out_dtype, log2_t, n):
    announce(f"encode forward n={n} table={table_dtype} out={np.dtype(out_dtype).name} log2_t={log2_t}")
    desc = ext.grid_desc(log2_t, table_dtype)
    table = ext.init_table(desc, seed=3, value_range=1.0)
    pos = points(n, seed=1)
    d_pos = DeviceArray.from_numpy(pos)
    d_out = DeviceArray((n, 32), out_dtype)
    ext.encode_forward(desc, table, d_pos, n, d_out)
    synchronize()
    t = table.numpy()
    want = orc.encode(oracle_grid(desc), t if t.dtype == np.float32 else t.view(np.uint16), pos)
    got = d_out.numpy().astype(np.float32)
    if out_dtype == np.float32:
        np.testing.assert_allclose(got, want, rtol=1e-6, atol=1e-7)
    else:
        assert np.array_equal(got, want.astype(np.float16).astype(np.float32))
