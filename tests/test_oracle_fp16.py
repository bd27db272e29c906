"""Oracle binary16 conversion pinned against numpy's IEEE-754 conversion."""
import numpy as np


def test_f32_to_f16_matches_numpy_random(orc):
    rng = np.random.default_rng(0)
    parts = [
        rng.standard_normal(200_000).astype(np.float32) * 10.0,
        rng.uniform(-70000, 70000, 50_000).astype(np.float32),
        (rng.uniform(-1, 1, 50_000) * 2.0 ** -14).astype(np.float32),  # half subnormals
        (rng.uniform(-1, 1, 20_000) * 2.0 ** -24).astype(np.float32),  # around the smallest subnormal
        np.frombuffer(rng.integers(0, 2 ** 32, 100_000, dtype=np.uint64).astype(np.uint32).tobytes(), np.float32),
    ]
    x = np.concatenate(parts)
    x = x[np.isfinite(x)]
    want = x.astype(np.float16).view(np.uint16)
    got = orc.f32_to_f16_bits(x)
    bad = np.nonzero(got != want)[0]
    assert bad.size == 0, f"{bad.size} mismatches, first x={x[bad[0]]!r} got={got[bad[0]]:#06x} want={want[bad[0]]:#06x}"


def test_f32_to_f16_edges(orc):
    edges = np.array([0.0, -0.0, 65504.0, 65519.0, 65519.996, 65520.0, 1e9, -1e9, 2.0 ** -24, 2.0 ** -25, 3 * 2.0 ** -26, 2.0 ** -26, 2.0 ** -14, 2.0 ** -14 * (1 - 2 ** -11),
                      1.0 + 2 ** -11, 1.0 + 3 * 2 ** -11, np.inf, -np.inf], np.float32)
    want = edges.astype(np.float16).view(np.uint16)
    assert np.array_equal(orc.f32_to_f16_bits(edges), want)
    assert orc.f32_to_f16_bits(np.array([np.nan], np.float32))[0] & 0x7C00 == 0x7C00


def test_f16_to_f32_all_patterns(orc):
    bits = np.arange(65536, dtype=np.uint16)
    want = bits.view(np.float16).astype(np.float32)
    got = orc.f16_bits_to_f32(bits)
    finite = np.isfinite(want)
    assert np.array_equal(got[finite].view(np.uint32), want[finite].view(np.uint32))
    assert np.all(np.isnan(got[np.isnan(want)]))
    assert np.array_equal(np.isinf(got), np.isinf(want))
