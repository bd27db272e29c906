"""Oracle pins of the nested-cascade occupancy grid (unbounded scenes).

Cascade c of a box is the box scaled by 2^c about its centre.  On the unit
box every cascade bound 0.5 -/+ 0.5 * 2^c is exact in fp32, so the expected
cascade and cell of a point follow from the geometry alone: these tests
place points at cell centres computed in fp64 and check the oracle's index
against the closed form, check that a cascaded bitfield equals one-box
bitfields built over each cascade's box, and that a march with every cell
occupied sees the outermost box.
"""
import numpy as np
import pytest

from oracle import oracle as orc

UNIT = (0.0, 0.0, 0.0, 1.0, 1.0, 1.0)
OUT = 0xFFFFFFFF


def box_of(c):
    lo, hi = 0.5 - 0.5 * 2.0 ** c, 0.5 + 0.5 * 2.0 ** c
    return (lo, lo, lo, hi, hi, hi)


@pytest.mark.parametrize("res,cascades", [(8, 1), (8, 5), (5, 3)])
def test_cell_index_closed_form(res, cascades):
    rng = np.random.default_rng(res * 10 + cascades)
    words = (res ** 3 + 31) // 32
    pts, want = [], []
    for c in range(cascades):
        lo, hi = 0.5 - 0.5 * 2.0 ** c, 0.5 + 0.5 * 2.0 ** c
        step = (hi - lo) / res
        for _ in range(200):
            ijk = rng.integers(0, res, size=3)
            p = lo + (ijk + 0.5) * step
            # Skip cells that lie inside the previous cascade's box (they belong to it).
            if c > 0:
                plo, phi = 0.5 - 0.5 * 2.0 ** (c - 1), 0.5 + 0.5 * 2.0 ** (c - 1)
                if np.all((p >= plo) & (p < phi)):
                    continue
            pts.append(p)
            want.append(c * 32 * words + int(ijk[0]) + int(ijk[1]) * res + int(ijk[2]) * res * res)
    got = orc.occ_cell(res, cascades, UNIT, np.array(pts, np.float32))
    assert np.array_equal(got, np.array(want, np.uint32))


def test_points_outside_every_cascade():
    far = np.array([[0.5 + 0.5 * 2.0 ** 3 + 1e-3, 0.5, 0.5], [0.5, -8.0, 0.5], [100.0, 100.0, 100.0]], np.float32)
    assert np.all(orc.occ_cell(8, 4, UNIT, far) == OUT)
    # Inside the 4th cascade box, outside the first three.
    inside = np.array([[0.5 + 0.5 * 2.0 ** 3 - 1e-3, 0.5, 0.5]], np.float32)
    assert orc.occ_cell(8, 4, UNIT, inside)[0] // (32 * ((8 ** 3 + 31) // 32)) == 3


def test_cascaded_bitfield_equals_per_box_bitfields():
    g = np.array([[0.5, 0.5, 0.5, 0.3, 20.0, 1, 0, 0], [3.0, 0.5, -2.0, 1.5, 30.0, 0, 1, 0], [-5.0, 6.0, 0.5, 2.0, 10.0, 0, 0, 1]], np.float32)
    res, C = 12, 4
    words = (res ** 3 + 31) // 32
    bits = orc.occupancy_from_scene(g, res, UNIT, 0.01, cascades=C)
    for c in range(C):
        one = orc.occupancy_from_scene(g, res, box_of(c), 0.01)
        assert np.array_equal(bits[c * words:(c + 1) * words], one), f"cascade {c}"
        assert one.any()


def test_shell_marks_cells_between_radii():
    res, C = 16, 3
    centre = (0.5, 0.5, 0.5)
    bits = orc.occupancy_from_scene(np.zeros((0, 8), np.float32), res, UNIT, 0.01, cascades=C, shell=(centre, 1.0, 1.6))
    words = (res ** 3 + 31) // 32
    for c in range(C):
        lo, hi = 0.5 - 0.5 * 2.0 ** c, 0.5 + 0.5 * 2.0 ** c
        idx = np.arange(res ** 3)
        x, y, z = idx % res, (idx // res) % res, idx // (res * res)
        q = lo + (np.stack([x, y, z], 1) + 0.5) * ((hi - lo) / res)
        r = np.linalg.norm(q - 0.5, axis=1)
        got = (bits[c * words + (idx >> 5)] >> (idx & 31).astype(np.uint32)) & 1
        clear = np.abs(r - 1.0) > 1e-4
        clear &= np.abs(r - 1.6) > 1e-4
        want = (r >= 1.0) & (r <= 1.6)
        assert np.array_equal(got[clear].astype(bool), want[clear]), f"cascade {c}"
    assert bits.any()


def test_march_with_all_cells_occupied_sees_the_outer_box():
    # With no bitfield every cell of every cascade is occupied: the march is
    # the plain march over the outermost box.
    cam = orc.camera([1, 0, 0, 0.5, 0, 1, 0, 0.5, 0, 0, 1, 6.0], 40.0, 40.0, 15.5, 15.5, 32, 32)
    for C in (1, 3, 5):
        got = orc.march_count(cam, None, 8, UNIT, 512, cascades=C)
        want = orc.march_count(cam, None, 8, box_of(C - 1), 512)
        assert np.array_equal(got, want)
        assert got.max() > 0
