"""The host harness pieces (nerf_amd/harness) on the CPU, through
libnerf_host.so: PNG decoding against Python's zlib (an independent deflate)
over every block type, filter type and colour type; PNG writing; CRC-32 and
Adler-32 against zlib; the JSON reader; the NeRF-synthetic camera transform
against its closed form (benchmark.cpp:148-303: Blender world axes (x, -z, y),
translation x 0.33 + 0.5); the dataset loader end to end; PSNR against its
closed form (benchmark.cpp:47-86)."""
import ctypes as C
import os
import json
import math
import struct
import zlib
from pathlib import Path

import numpy as np
import pytest

# NERF_HOST_LIB selects another build of the harness (the sanitizer build of
# tests/test_sanitizers.py).
LIB_PATH = Path(os.environ["NERF_HOST_LIB"]) if os.environ.get("NERF_HOST_LIB") else Path(__file__).resolve().parent.parent / "nerf_amd" / "libnerf_host.so"


@pytest.fixture(scope="module")
def lib():
    if not LIB_PATH.exists():
        pytest.fail("libnerf_host.so is not built (run __graft_entry__.build())")
    h = C.CDLL(str(LIB_PATH))
    h.nerf_host_last_error.restype = C.c_char_p
    h.nerf_host_png_decode.argtypes = [C.c_void_p, C.c_uint64, C.POINTER(C.c_uint32), C.POINTER(C.c_uint32), C.c_void_p, C.c_uint64]
    h.nerf_host_png_encode.argtypes = [C.c_uint32, C.c_uint32, C.c_void_p, C.c_void_p, C.c_uint64]
    h.nerf_host_png_encode.restype = C.c_uint64
    h.nerf_host_crc32.argtypes = [C.c_void_p, C.c_uint64]
    h.nerf_host_crc32.restype = C.c_uint32
    h.nerf_host_adler32.argtypes = [C.c_void_p, C.c_uint64]
    h.nerf_host_adler32.restype = C.c_uint32
    h.nerf_host_json_check.argtypes = [C.c_char_p, C.POINTER(C.c_uint32)]
    h.nerf_host_transform_camera.argtypes = [C.c_void_p, C.c_void_p]
    h.nerf_host_load_dataset.argtypes = [C.c_char_p, C.POINTER(C.c_uint32), C.POINTER(C.c_uint32), C.POINTER(C.c_uint32), C.c_void_p, C.c_void_p, C.c_uint64, C.c_void_p, C.c_uint64]
    h.nerf_host_psnr.argtypes = [C.c_void_p, C.c_void_p, C.c_uint32, C.c_uint32, C.POINTER(C.c_double)]
    h.nerf_host_psnr.restype = C.c_double
    return h


def _chunk(t: bytes, body: bytes) -> bytes:
    return struct.pack(">I", len(body)) + t + body + struct.pack(">I", zlib.crc32(t + body) & 0xFFFFFFFF)


def _filter(rows: np.ndarray, bpp: int, kinds) -> bytes:
    """PNG filtering (types 0-4) of raw scanlines, one filter type per row."""
    out = bytearray()
    prev = np.zeros(rows.shape[1], np.int32)
    for y, row in enumerate(rows.astype(np.int32)):
        f = kinds[y % len(kinds)]
        a = np.concatenate([np.zeros(bpp, np.int32), row[:-bpp]])
        c = np.concatenate([np.zeros(bpp, np.int32), prev[:-bpp]])
        b = prev
        if f == 0:
            v = row
        elif f == 1:
            v = row - a
        elif f == 2:
            v = row - b
        elif f == 3:
            v = row - (a + b) // 2
        else:
            p = a + b - c
            pa, pb, pc = np.abs(p - a), np.abs(p - b), np.abs(p - c)
            pred = np.where((pa <= pb) & (pa <= pc), a, np.where(pb <= pc, b, c))
            v = row - pred
        out.append(f)
        out += (v & 255).astype(np.uint8).tobytes()
        prev = row
    return bytes(out)


def _png(pixels: np.ndarray, ctype: int, level: int, kinds=(0, 1, 2, 3, 4), plte: bytes = b"", trns: bytes = b"") -> bytes:
    h, w = pixels.shape[:2]
    ch = {0: 1, 2: 3, 3: 1, 4: 2, 6: 4}[ctype]
    raw = _filter(pixels.reshape(h, w * ch), ch, kinds)
    body = _chunk(b"IHDR", struct.pack(">IIBBBBB", w, h, 8, ctype, 0, 0, 0))
    if plte:
        body += _chunk(b"PLTE", plte)
    if trns:
        body += _chunk(b"tRNS", trns)
    z = zlib.compress(raw, level)
    # Two IDAT chunks: the decoder must concatenate them.
    body += _chunk(b"IDAT", z[: len(z) // 2]) + _chunk(b"IDAT", z[len(z) // 2:]) + _chunk(b"IEND", b"")
    return b"\x89PNG\r\n\x1a\n" + body


def _decode(lib, data: bytes):
    w, h = C.c_uint32(), C.c_uint32()
    assert lib.nerf_host_png_decode(data, len(data), C.byref(w), C.byref(h), None, 0) == 0, lib.nerf_host_last_error()
    out = np.zeros((h.value, w.value, 4), np.uint8)
    assert lib.nerf_host_png_decode(data, len(data), C.byref(w), C.byref(h), out.ctypes.data, out.nbytes) == 0
    return out


@pytest.mark.parametrize("level", [0, 1, 6, 9])  # stored blocks, fixed and dynamic Huffman codes
def test_png_decode_rgba_all_filters(lib, level):
    rng = np.random.default_rng(level)
    # Smooth content (long matches, short distances) plus noise (literals).
    y, x = np.mgrid[0:37, 0:53]
    img = np.stack([(x * 5) % 256, (y * 7) % 256, (x + y) % 256, rng.integers(0, 256, (37, 53))], -1).astype(np.uint8)
    got = _decode(lib, _png(img, 6, level))
    assert np.array_equal(got, img)


def test_png_decode_colour_types(lib):
    rng = np.random.default_rng(7)
    g = rng.integers(0, 256, (9, 11), np.uint8)
    rgb = rng.integers(0, 256, (9, 11, 3), np.uint8)
    ga = rng.integers(0, 256, (9, 11, 2), np.uint8)
    assert np.array_equal(_decode(lib, _png(g, 0, 6)), np.stack([g, g, g, np.full_like(g, 255)], -1))
    assert np.array_equal(_decode(lib, _png(rgb, 2, 6)), np.concatenate([rgb, np.full((9, 11, 1), 255, np.uint8)], -1))
    assert np.array_equal(_decode(lib, _png(ga, 4, 6)), np.stack([ga[..., 0], ga[..., 0], ga[..., 0], ga[..., 1]], -1))
    pal = rng.integers(0, 256, (16, 3), np.uint8)
    alpha = rng.integers(0, 256, 10, np.uint8)  # tRNS shorter than the palette: the rest are opaque
    idx = rng.integers(0, 16, (9, 11), np.uint8)
    want = np.concatenate([pal[idx], np.where(idx < 10, alpha[np.minimum(idx, 9)], 255)[..., None].astype(np.uint8)], -1)
    assert np.array_equal(_decode(lib, _png(idx, 3, 6, plte=pal.tobytes(), trns=alpha.tobytes())), want)


def test_png_rejects_corruption(lib):
    img = np.zeros((4, 4, 4), np.uint8)
    good = _png(img, 6, 6)
    w, h = C.c_uint32(), C.c_uint32()
    bad = bytearray(good)
    bad[40] ^= 0xFF  # inside IHDR/IDAT: CRC mismatch
    assert lib.nerf_host_png_decode(bytes(bad), len(bad), C.byref(w), C.byref(h), None, 0) != 0
    assert lib.nerf_host_png_decode(good[:20], 20, C.byref(w), C.byref(h), None, 0) != 0
    inter = good.replace(struct.pack(">IIBBBBB", 4, 4, 8, 6, 0, 0, 0), struct.pack(">IIBBBBB", 4, 4, 8, 6, 0, 0, 1))
    assert lib.nerf_host_png_decode(inter, len(inter), C.byref(w), C.byref(h), None, 0) != 0  # CRC now wrong as well


def test_png_encode_round_trip(lib):
    rng = np.random.default_rng(3)
    img = rng.integers(0, 256, (70000 // 64 + 3, 64, 4), np.uint8)  # > 65535 raw bytes: several stored blocks
    n = lib.nerf_host_png_encode(64, img.shape[0], img.ctypes.data, None, 0)
    buf = (C.c_uint8 * n)()
    assert lib.nerf_host_png_encode(64, img.shape[0], img.ctypes.data, buf, n) == n
    data = bytes(buf)
    # Independent check of the container: zlib inflates the IDAT payload.
    assert data[:8] == b"\x89PNG\r\n\x1a\n"
    pos, idat = 8, b""
    while pos < len(data):
        (ln,) = struct.unpack(">I", data[pos:pos + 4])
        t = data[pos + 4:pos + 8]
        assert zlib.crc32(data[pos + 4:pos + 8 + ln]) & 0xFFFFFFFF == struct.unpack(">I", data[pos + 8 + ln:pos + 12 + ln])[0]
        if t == b"IDAT":
            idat += data[pos + 8:pos + 8 + ln]
        pos += 12 + ln
    raw = np.frombuffer(zlib.decompress(idat), np.uint8).reshape(img.shape[0], 1 + 64 * 4)
    assert np.all(raw[:, 0] == 0) and np.array_equal(raw[:, 1:].reshape(img.shape), img)
    assert np.array_equal(_decode(lib, data), img)


def test_checksums(lib):
    for data in [b"", b"a", b"123456789", bytes(range(256)) * 300]:
        assert lib.nerf_host_crc32(data, len(data)) == zlib.crc32(data) & 0xFFFFFFFF
        assert lib.nerf_host_adler32(data, len(data)) == zlib.adler32(data) & 0xFFFFFFFF


def test_json_reader(lib):
    keys = C.c_uint32()
    doc = {"camera_angle_x": 0.6911112070083618, "frames": [{"file_path": "./train/r_0", "transform_matrix": [[1, 0, 0, 0]] * 4}], "s": "a\\\"é\U0001F600", "n": None, "t": True}
    assert lib.nerf_host_json_check(json.dumps(doc).encode(), C.byref(keys)) == 0 and keys.value == 5
    assert lib.nerf_host_json_check(json.dumps(doc, ensure_ascii=False).encode(), C.byref(keys)) == 0
    for bad in [b"{", b"[1,]", b'{"a" 1}', b"01x", b'"\\q"', b"[1] 2", b"nul"]:
        assert lib.nerf_host_json_check(bad, C.byref(keys)) != 0, bad


def _transform_closed_form(m: np.ndarray) -> np.ndarray:
    W = np.array([[1, 0, 0], [0, 0, 1], [0, -1, 0]], np.float32)  # Blender (x, y, z) -> (x, z, -y)
    out = np.zeros((4, 4), np.float32)
    out[:3, :3] = W @ m[:3, :3]
    out[:3, 3] = (W @ m[:3, 3]) * np.float32(0.33) + np.float32(0.5)
    out[3, 3] = 1.0
    return out


def test_camera_transform_closed_form(lib):
    rng = np.random.default_rng(11)
    for _ in range(20):
        m = rng.normal(size=(4, 4)).astype(np.float32)
        m[3] = (0, 0, 0, 1)
        got = np.zeros(16, np.float32)
        lib.nerf_host_transform_camera(m.ctypes.data, got.ctypes.data)
        assert np.array_equal(got.reshape(4, 4), _transform_closed_form(m))


def _write_dataset(root: Path, frames: int, w: int, h: int, angle: float):
    rng = np.random.default_rng(5)
    imgs, mats = [], []
    (root / "train").mkdir(parents=True)
    meta = {"camera_angle_x": angle, "frames": []}
    for i in range(frames):
        img = rng.integers(0, 256, (h, w, 4), np.uint8)
        (root / "train" / f"r_{i}.png").write_bytes(_png(img, 6, 6))
        m = np.eye(4, dtype=np.float32)
        m[:3, :3] = np.linalg.qr(rng.normal(size=(3, 3)))[0]
        m[:3, 3] = rng.normal(size=3) * 4
        meta["frames"].append({"file_path": f"./train/r_{i}", "rotation": 0.0, "transform_matrix": m.tolist()})
        imgs.append(img)
        mats.append(m.astype(np.float32))
    (root / "transforms_train.json").write_text(json.dumps(meta, indent=2))
    return imgs, mats


def test_dataset_loader(lib, tmp_path):
    w, h, n, angle = 24, 16, 3, 0.6911112070083618
    imgs, mats = _write_dataset(tmp_path / "lego", n, w, h, angle)
    cnt, wd, ht = C.c_uint32(), C.c_uint32(), C.c_uint32()
    intr = np.zeros(4, np.float32)
    cams = np.zeros((n, 16), np.float32)
    out = np.zeros((n, h, w, 4), np.uint8)
    assert lib.nerf_host_load_dataset(str(tmp_path / "lego").encode(), C.byref(cnt), C.byref(wd), C.byref(ht), intr.ctypes.data, cams.ctypes.data, cams.size, out.ctypes.data, out.nbytes) == 0, lib.nerf_host_last_error()
    assert (cnt.value, wd.value, ht.value) == (n, w, h)
    for i in range(n):
        assert np.array_equal(out[i], imgs[i])
        assert np.allclose(cams[i].reshape(4, 4), _transform_closed_form(mats[i]), rtol=0, atol=0)  # bit-exact: permutation maps
    fx = 0.5 * w / math.tan(angle * 0.5)
    np.testing.assert_allclose(intr, [fx, fx, 0.5 * (w - 1), 0.5 * (h - 1)], rtol=1e-6)
    # The .json path form and a missing frame.
    assert lib.nerf_host_load_dataset(str(tmp_path / "lego" / "transforms_train.json").encode(), C.byref(cnt), C.byref(wd), C.byref(ht), intr.ctypes.data, None, 0, None, 0) == 0
    (tmp_path / "lego" / "train" / "r_1.png").unlink()
    assert lib.nerf_host_load_dataset(str(tmp_path / "lego").encode(), C.byref(cnt), C.byref(wd), C.byref(ht), intr.ctypes.data, None, 0, None, 0) != 0
    assert b"r_1" in lib.nerf_host_last_error()


def test_psnr_closed_forms(lib):
    rng = np.random.default_rng(9)
    gt = rng.integers(0, 250, (20, 30, 4), np.uint8)
    gt[..., 3] = 255  # opaque: the composite over white is the colour itself
    luma = C.c_double()
    assert math.isinf(lib.nerf_host_psnr(gt.ctypes.data, gt.ctypes.data, 30, 20, C.byref(luma)))
    pred = gt.copy()
    pred[..., :3] += 3
    psnr = lib.nerf_host_psnr(gt.ctypes.data, pred.ctypes.data, 30, 20, C.byref(luma))
    assert abs(psnr - (-10.0 * math.log10((3 / 255) ** 2))) < 1e-4
    p = pred[..., :3].astype(np.float32) / np.float32(255)
    want_luma = float(np.mean((np.float32(0.2126) * p[..., 0] + np.float32(0.7152) * p[..., 1]) + np.float32(0.0722) * p[..., 2]))
    assert abs(luma.value - want_luma) < 1e-6
    # Transparent ground truth composites to white.
    clear = np.zeros((20, 30, 4), np.uint8)
    white = np.full((20, 30, 4), 255, np.uint8)
    assert math.isinf(lib.nerf_host_psnr(clear.ctypes.data, white.ctypes.data, 30, 20, None))
