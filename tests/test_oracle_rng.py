"""Integer RNG pinning: splitmix64 (published vectors), the reference's stream
seeding and Xavier init, and structural checks of hash_u32."""
import numpy as np

M32 = 0xFFFFFFFF


def test_splitmix64_published_seed0(orc):
    # First outputs of splitmix64 started from state 0 (Vigna's reference C
    # implementation, splitmix64.c).
    want = [0xE220A8397B1DCDAF, 0x6E789E6AA1B965F4, 0x06C45D188009454F, 0xF88BB8A8724C81EC]
    assert [int(v) for v in orc.splitmix_sequence(0, 4)] == want


def test_stream_state_formula(orc):
    # backend-cuda.cu:1811 seeds with (a + golden) ^ (b * mix1), u64 wraparound.
    g, m1 = 0x9E3779B97F4A7C15, 0xBF58476D1CE4E5B9
    for a, b in [(0x1234, 0x5678), (0x9ABC, 0xDEF0), (0, 0), (2 ** 64 - 1, 3)]:
        assert orc.lib().orc_stream_state(a, b) == (((a + g) & (2 ** 64 - 1)) ^ ((b * m1) & (2 ** 64 - 1)))


def _inverse_hash_u32(y: int) -> int:
    def unxorshift(x, s):
        r = x
        for _ in range(32 // s + 1):
            r = x ^ (r >> s)
        return r & M32

    y = unxorshift(y, 16)
    y = (y * pow(0x846CA68B, -1, 2 ** 32)) & M32
    y = unxorshift(y, 15)
    y = (y * pow(0x7FEB352D, -1, 2 ** 32)) & M32
    return unxorshift(y, 16)


def test_hash_u32_bijective_and_avalanche(orc):
    rng = np.random.default_rng(1)
    xs = [int(v) for v in rng.integers(0, 2 ** 32, 2000, dtype=np.uint64)]
    h = orc.lib().orc_hash_u32
    assert all(_inverse_hash_u32(h(x)) == x for x in xs)
    flips = []
    for x in xs[:500]:
        hx = h(x)
        for b in range(32):
            flips.append(bin(hx ^ h(x ^ (1 << b))).count("1"))
    assert 15.0 < np.mean(flips) < 17.0
    assert h(0) == 0


def test_rand01_grid(orc):
    r = orc.lib().orc_rand01
    vals = np.array([r(s) for s in range(5000)], np.float64)
    assert np.all((vals >= 0) & (vals < 1))
    assert np.all(np.abs(vals * 2 ** 24 - np.round(vals * 2 ** 24)) == 0)


def test_mlp_init_matches_reference_loop(orc):
    # Sequential reference loop restated (backend-cuda.cu:1810-1847) from the
    # splitmix64 stream, on the target shapes.
    for net, shapes, (a, b) in [(0, [(64, 32), (16, 64)], (0x1234, 0x5678)), (1, [(64, 32), (64, 64), (16, 64)], (0x9ABC, 0xDEF0))]:
        total = sum(o * i for o, i in shapes)
        z = orc.splitmix_sequence(orc.lib().orc_stream_state(a, b), total)
        u = ((z >> np.uint64(32)).astype(np.uint32) >> np.uint32(8)).astype(np.float32) * np.float32(1.0 / 16777216.0)
        want, off = [], 0
        for o, i in shapes:
            scale = np.sqrt(np.float32(6.0) / np.float32(o + i)).astype(np.float32)
            want.append(((u[off:off + o * i] * np.float32(2.0) - np.float32(1.0)) * scale).astype(np.float32))
            off += o * i
        assert np.array_equal(orc.mlp_init(net), np.concatenate(want))


def test_product_mlp_init_bit_exact_with_oracle(orc):
    from nerf_amd import ext

    for net in (0, 1):
        assert np.array_equal(ext.mlp_init(net).view(np.uint32), orc.mlp_init(net).view(np.uint32))


def test_uniform_fill_range(orc):
    v = orc.uniform_fill(0x7AB1E, 0, 100_000, -1e-4, 1e-4)
    assert v.min() >= -1e-4 and v.max() < 1e-4
    assert abs(v.mean()) < 1e-6
