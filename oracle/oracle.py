"""ctypes binding of oracle/liboracle.so — the scalar CPU oracle.

TEST INFRASTRUCTURE ONLY: imported by tests/, by the smoke check of
__graft_entry__.py and by the cpu_baseline leg of bench.py.  The product
(nerf_amd) never imports it.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB_PATH = HERE / "liboracle.so"


class OrcGrid(C.Structure):
    _fields_ = [
        ("n_levels", C.c_uint32),
        ("n_features", C.c_uint32),
        ("table_size", C.c_uint32),
        ("table_dtype", C.c_uint32),
        ("resolution", C.c_uint32 * 16),
        ("dense", C.c_uint32 * 16),
    ]


class OrcCamera(C.Structure):
    _fields_ = [
        ("c2w", C.c_float * 12),
        ("fx", C.c_float),
        ("fy", C.c_float),
        ("cx", C.c_float),
        ("cy", C.c_float),
        ("width", C.c_uint32),
        ("height", C.c_uint32),
    ]


class OrcModel(C.Structure):
    _fields_ = [
        ("grid", OrcGrid),
        ("table", C.c_void_p),
        ("density_params", C.c_void_p),
        ("color_params", C.c_void_p),
        ("kind", C.c_uint32),
    ]


_P = C.c_void_p
_U32 = C.c_uint32
_U64 = C.c_uint64
_F = C.c_float

_PROTOS = {
    "orc_f32_to_f16": (C.c_uint16, [_F]),
    "orc_f16_to_f32": (_F, [C.c_uint16]),
    "orc_f32_to_f16_array": (None, [_P, _P, _U64]),
    "orc_hash_u32": (_U32, [_U32]),
    "orc_rand01": (_F, [_U32]),
    "orc_splitmix_sequence": (None, [_U64, _U64, _P]),
    "orc_stream_state": (_U64, [_U64, _U64]),
    "orc_uniform_fill": (None, [_U64, _U64, _U64, _F, _F, _P]),
    "orc_mlp_param_count": (_U32, [_U32]),
    "orc_mlp_init": (None, [_U32, _P]),
    "orc_grid_levels": (None, [_U32, _U32, _F, _U32, _U32, _P, _P]),
    "orc_encode": (None, [C.POINTER(OrcGrid), _P, _P, _U32, _P, _P, _P]),
    "orc_density_mlp": (None, [_P, _P, _U32, _P]),
    "orc_density_forward": (None, [C.POINTER(OrcGrid), _P, _P, _P, _U32, _P]),
    "orc_sh4": (None, [_P, _P]),
    "orc_field_forward": (None, [C.POINTER(OrcGrid), _P, _P, _P, _P, _P, _U32, _P]),
    "orc_ref_param_count": (_U32, [_U32]),
    "orc_ref_mlp_init": (None, [_U32, _P]),
    "orc_freq_encode": (None, [_P, _U32, _P]),
    "orc_softplus": (_F, [_F]),
    "orc_ref_field_forward": (None, [_P, _P, _P, _P, _U32, _P, _P]),
    "orc_ref_composite_backward_ray": (C.c_double, [_P, _P, _P, _U32, _P, _F, _P, _P, _P]),
    "orc_ref_mlp_backward": (None, [_P, _P, _P, _P, _P, _U32, _F, _P, _P]),
    "orc_det_expf": (_F, [_F]),
    "orc_det_expf_array": (None, [_P, _U64, _P]),
    "orc_scene_density": (None, [_P, _U32, _P, _U32, _P]),
    "orc_occupancy_from_scene": (None, [_P, _U32, _U32, _U32, _P, _F, _P]),
    "orc_occupancy_mark_shell": (None, [_U32, _U32, _P, _P, _F, _F, _P]),
    "orc_occ_cell": (None, [_U32, _U32, _P, _P, _U32, _P]),
    "orc_march_count": (None, [C.POINTER(OrcCamera), _P, _U32, _U32, _P, _U32, _U32, _U32, _P]),
    "orc_march_ray": (_U32, [C.POINTER(OrcCamera), _P, _U32, _U32, _P, _U32, _U32, _P, _U32]),
    "orc_pixel_ray": (C.c_int, [C.POINTER(OrcCamera), _U32, _P, _P]),
    "orc_composite_ray": (_U32, [_P, _P, _U32, _F, _P, _P, _P]),
    "orc_composite_backward_ray": (C.c_double, [_P, _P, _P, _U32, _P, _P, _F, _F, _P, _P, _P]),
    "orc_composite_backward_act": (C.c_double, [_P, _P, _P, _U32, _P, _P, _F, _F, _P, _P, _P]),
    "orc_mlp_backward": (None, [_P, _P, _P, _P, _P, _P, _U32, _F, _P, _P, _P]),
    "orc_encode_backward": (None, [C.POINTER(OrcGrid), _P, _P, _U32, _P]),
    "orc_adam": (C.c_int, [_P, _P, _P, _P, _U64, _F, _F, _F, _F, _F, _F, _F, _U32, _U32, C.c_double, C.c_int]),
    "orc_train_rays": (None, [C.POINTER(OrcCamera), _P, _P, _U32, _P, _U32, _U32, _U32, _P, _P, _P, _P, _P, _U32]),
    "orc_train_camera": (_U32, [_U32, _U32]),
    "orc_field_mlp": (None, [_P, _P, _P, _P, _U32, _P]),
    "orc_scene_render": (None, [_P, _U32, C.POINTER(OrcCamera), _P, _U32, _P]),
    "orc_render_rays": (None, [C.POINTER(OrcModel), C.POINTER(OrcCamera), _P, _U32, _U32, _P, _U32, _F, _P, _P, _U32, _P, _P, _P, _U32, _P, _P, _P]),
    "orc_render_uniform": (None, [C.POINTER(OrcModel), C.POINTER(OrcCamera), _P, _U32, _P, _P, _U32, _P, _P, _P, _U32]),
}

_lib = None


def build() -> None:
    subprocess.run(["make", "-s", "-C", str(HERE)], check=True)


def lib() -> C.CDLL:
    global _lib
    if _lib is None:
        # NERF_ORACLE_LIB selects another build of the same sources (the
        # sanitizer build of tests/test_sanitizers.py).
        path = Path(os.environ["NERF_ORACLE_LIB"]) if os.environ.get("NERF_ORACLE_LIB") else LIB_PATH
        if not path.exists():
            build()
        L = C.CDLL(str(path))
        for name, (res, args) in _PROTOS.items():
            f = getattr(L, name)
            f.restype = res
            f.argtypes = args
        _lib = L
    return _lib


def _p(a: np.ndarray) -> int:
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data


# ------------------------------------------------------------------ helpers
def f32_to_f16_bits(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, np.float32)
    out = np.empty(x.shape, np.uint16)
    lib().orc_f32_to_f16_array(_p(x), _p(out), x.size)
    return out


def f16_bits_to_f32(h: np.ndarray) -> np.ndarray:
    f = lib().orc_f16_to_f32
    return np.array([f(int(v)) for v in np.asarray(h).ravel()], np.float32).reshape(np.shape(h))


def splitmix_sequence(state: int, n: int) -> np.ndarray:
    out = np.empty(n, np.uint64)
    lib().orc_splitmix_sequence(state, n, _p(out))
    return out


def uniform_fill(a: int, b: int, n: int, lo: float, hi: float) -> np.ndarray:
    out = np.empty(n, np.float32)
    lib().orc_uniform_fill(a, b, n, lo, hi, _p(out))
    return out


def mlp_init(network: int) -> np.ndarray:
    out = np.empty(lib().orc_mlp_param_count(network), np.float32)
    lib().orc_mlp_init(network, _p(out))
    return out


def grid_levels(n_levels: int, base: int, scale: float, finest: int, log2_t: int) -> tuple[np.ndarray, np.ndarray]:
    res = np.zeros(16, np.uint32)
    dense = np.zeros(16, np.uint32)
    lib().orc_grid_levels(n_levels, base, scale, finest, log2_t, _p(res), _p(dense))
    return res[:n_levels], dense[:n_levels]


def make_grid(n_levels: int, log2_t: int, table_dtype: int, base: int = 16, scale: float = 1.3819, finest: int = 0) -> OrcGrid:
    res, dense = grid_levels(n_levels, base, scale, finest, log2_t)
    g = OrcGrid()
    g.n_levels = n_levels
    g.n_features = 2
    g.table_size = 1 << log2_t
    g.table_dtype = table_dtype
    for i in range(n_levels):
        g.resolution[i] = int(res[i])
        g.dense[i] = int(dense[i])
    return g


def encode(grid: OrcGrid, table: np.ndarray, pos: np.ndarray, with_indices: bool = False):
    pos = np.ascontiguousarray(pos, np.float32)
    n = pos.shape[0]
    feat = np.empty((n, grid.n_levels * 2), np.float32)
    idx = np.empty((n, grid.n_levels, 8), np.uint32) if with_indices else None
    w = np.empty((n, grid.n_levels, 8), np.float32) if with_indices else None
    lib().orc_encode(C.byref(grid), _p(table), _p(pos), n, _p(feat), _p(idx) if with_indices else None, _p(w) if with_indices else None)
    return (feat, idx, w) if with_indices else feat


def density_mlp(params_f16_bits: np.ndarray, features: np.ndarray) -> np.ndarray:
    features = np.ascontiguousarray(features, np.float32)
    out = np.empty((features.shape[0], 16), np.float32)
    lib().orc_density_mlp(_p(params_f16_bits), _p(features), features.shape[0], _p(out))
    return out


def density_forward(grid: OrcGrid, table: np.ndarray, params_f16_bits: np.ndarray, pos: np.ndarray) -> np.ndarray:
    pos = np.ascontiguousarray(pos, np.float32)
    out = np.empty((pos.shape[0], 16), np.float32)
    lib().orc_density_forward(C.byref(grid), _p(table), _p(params_f16_bits), _p(pos), pos.shape[0], _p(out))
    return out


def sh4(d: np.ndarray) -> np.ndarray:
    d = np.ascontiguousarray(d, np.float32).reshape(-1, 3)
    out = np.empty((d.shape[0], 16), np.float32)
    for i in range(d.shape[0]):
        lib().orc_sh4(_p(d[i]), out[i].ctypes.data)
    return out


def field_forward(grid: OrcGrid, table: np.ndarray, dparams_bits: np.ndarray, cparams_bits: np.ndarray, pos: np.ndarray, dirs: np.ndarray) -> np.ndarray:
    pos = np.ascontiguousarray(pos, np.float32)
    dirs = np.ascontiguousarray(dirs, np.float32)
    out = np.empty((pos.shape[0], 4), np.float32)
    lib().orc_field_forward(C.byref(grid), _p(table), _p(dparams_bits), _p(cparams_bits), _p(pos), _p(dirs), pos.shape[0], _p(out))
    return out


def ref_param_count(network: int) -> int:
    return int(lib().orc_ref_param_count(network))


def ref_mlp_init(network: int) -> np.ndarray:
    """The reference's init (backend-cuda.cu:1810-1847) on its own shapes."""
    out = np.empty(lib().orc_ref_param_count(network), np.float32)
    lib().orc_ref_mlp_init(network, _p(out))
    return out


def freq_encode(p: np.ndarray, levels: int) -> np.ndarray:
    p = np.ascontiguousarray(p, np.float32).reshape(-1, 3)
    out = np.empty((p.shape[0], 3 + 6 * levels), np.float32)
    for i in range(p.shape[0]):
        lib().orc_freq_encode(_p(p[i]), levels, _p(out[i]))
    return out


def softplus(x: float) -> float:
    return float(lib().orc_softplus(float(x)))


def ref_field_forward(dparams_bits: np.ndarray, cparams_bits: np.ndarray, pos: np.ndarray, dirs: np.ndarray):
    """Reference-model field at world positions: (out [n][4] = (sigma, r, g,
    b), raw [n][4] = fp16-rounded raw density 0 and colour 0..2)."""
    pos = np.ascontiguousarray(pos, np.float32)
    dirs = np.ascontiguousarray(dirs, np.float32)
    n = pos.shape[0]
    out = np.empty((n, 4), np.float32)
    raw = np.empty((n, 4), np.float32)
    lib().orc_ref_field_forward(_p(np.ascontiguousarray(dparams_bits)), _p(np.ascontiguousarray(cparams_bits)), _p(pos), _p(dirs), n, _p(out), _p(raw))
    return out, raw


def ref_composite_backward_ray(sraw, rgbraw, dt, gt4, inv_norm: float = 1.0):
    """The reference's loss on one ray (softplus, alpha-weighted MSE, white
    background): (loss, d raw sigma [n], d raw rgb [n][3], pred [3])."""
    sraw = np.ascontiguousarray(sraw, np.float32)
    rgbraw = np.ascontiguousarray(rgbraw, np.float32).reshape(-1, 3)
    dt = np.ascontiguousarray(dt, np.float32)
    gt4 = np.ascontiguousarray(gt4, np.float32)
    n = sraw.size
    ds, dc, pred = np.zeros(n, np.float32), np.zeros((n, 3), np.float32), np.zeros(3, np.float32)
    loss = lib().orc_ref_composite_backward_ray(_p(sraw), _p(rgbraw), _p(dt), n, _p(gt4), float(inv_norm), _p(ds), _p(dc), _p(pred))
    return float(loss), ds, dc, pred


def ref_mlp_backward(dparams_bits, cparams_bits, pos, dirs, draw, loss_scale: float = 1.0):
    """Reference-model weight gradients (fp64, x loss_scale) for d loss / d raw
    outputs draw [n][4]: (dD [75776], dC [40960])."""
    pos = np.ascontiguousarray(pos, np.float32)
    dirs = np.ascontiguousarray(dirs, np.float32)
    draw = np.ascontiguousarray(draw, np.float32)
    dD, dC = np.zeros(ref_param_count(0), np.float64), np.zeros(ref_param_count(1), np.float64)
    lib().orc_ref_mlp_backward(_p(np.ascontiguousarray(dparams_bits)), _p(np.ascontiguousarray(cparams_bits)), _p(pos), _p(dirs), _p(draw), pos.shape[0], float(loss_scale), _p(dD), _p(dC))
    return dD, dC


def det_expf(x) -> np.ndarray:
    x = np.ascontiguousarray(x, np.float32)
    out = np.empty_like(x)
    lib().orc_det_expf_array(_p(x), x.size, _p(out))
    return out


def scene_density(gaussians: np.ndarray, pos: np.ndarray) -> np.ndarray:
    g = np.ascontiguousarray(gaussians, np.float32)
    pos = np.ascontiguousarray(pos, np.float32)
    out = np.empty(pos.shape[0], np.float32)
    lib().orc_scene_density(_p(g), g.shape[0], _p(pos), pos.shape[0], _p(out))
    return out


def occupancy_words(res: int, cascades: int = 1) -> int:
    return cascades * ((res ** 3 + 31) // 32)


def occupancy_from_scene(gaussians: np.ndarray, res: int, aabb=(0, 0, 0, 1, 1, 1), threshold: float = 0.01, cascades: int = 1, shell=None) -> np.ndarray:
    """Bits of density(cell centre) > threshold for every cascade; shell =
    (centre3, r_inner, r_outer) also marks a uniform shell."""
    g = np.ascontiguousarray(gaussians, np.float32)
    box = np.array(aabb, np.float32)
    bits = np.zeros(occupancy_words(res, cascades), np.uint32)
    lib().orc_occupancy_from_scene(_p(g), g.shape[0], res, cascades, _p(box), threshold, _p(bits))
    if shell is not None:
        centre, r_in, r_out = shell
        c3 = np.array(centre, np.float32)
        lib().orc_occupancy_mark_shell(res, cascades, _p(box), _p(c3), r_in, r_out, _p(bits))
    return bits


def occ_cell(res: int, cascades: int, aabb, pos: np.ndarray) -> np.ndarray:
    """Bit index of each point's cell (0xFFFFFFFF outside every cascade)."""
    box = np.array(aabb, np.float32)
    p = np.ascontiguousarray(pos, np.float32)
    out = np.empty(p.shape[0], np.uint32)
    lib().orc_occ_cell(res, cascades, _p(box), _p(p), p.shape[0], _p(out))
    return out


def camera(c2w12, fx, fy, cx, cy, width, height) -> OrcCamera:
    cam = OrcCamera()
    for i in range(12):
        cam.c2w[i] = float(c2w12[i])
    cam.fx, cam.fy, cam.cx, cam.cy = fx, fy, cx, cy
    cam.width, cam.height = width, height
    return cam


def camera_from_bytes(raw: bytes) -> OrcCamera:
    """An OrcCamera from the bytes of a layout-identical NerfExtCamera."""
    cam = OrcCamera()
    C.memmove(C.addressof(cam), raw, C.sizeof(OrcCamera))
    return cam


def march_count(cam: OrcCamera, bits: np.ndarray | None, res: int, aabb, max_steps: int, ray_begin: int = 0, n: int | None = None, cascades: int = 1) -> np.ndarray:
    if n is None:
        n = cam.width * cam.height - ray_begin
    box = np.array(aabb, np.float32)
    out = np.empty(n, np.uint32)
    lib().orc_march_count(C.byref(cam), _p(bits) if bits is not None else None, res, cascades, _p(box), max_steps, ray_begin, n, _p(out))
    return out


def march_ray(cam: OrcCamera, bits: np.ndarray | None, res: int, aabb, max_steps: int, ray: int, cascades: int = 1) -> np.ndarray:
    box = np.array(aabb, np.float32)
    cap = max_steps
    buf = np.empty((cap, 2), np.float32)
    k = lib().orc_march_ray(C.byref(cam), _p(bits) if bits is not None else None, res, cascades, _p(box), max_steps, ray, _p(buf), cap)
    return buf[:k].copy()


def pixel_ray(cam: OrcCamera, ray: int, aabb) -> np.ndarray | None:
    box = np.array(aabb, np.float32)
    out = np.empty(8, np.float32)
    ok = lib().orc_pixel_ray(C.byref(cam), ray, _p(box), _p(out))
    return out if ok else None


def composite_ray(sigma_rgb: np.ndarray, dt: np.ndarray, t_stop: float = 1e-4, bg=(1.0, 1.0, 1.0)):
    s = np.ascontiguousarray(sigma_rgb, np.float32)
    d = np.ascontiguousarray(dt, np.float32)
    b = np.array(bg, np.float32)
    rgb = np.empty(3, np.float32)
    rgba = np.empty(1, np.uint32)
    used = lib().orc_composite_ray(_p(s), _p(d), s.shape[0], t_stop, _p(b), _p(rgb), _p(rgba))
    return rgb, int(rgba[0]), int(used)


def render_rays(grid: OrcGrid | None, table: np.ndarray | None, dparams_bits: np.ndarray, cparams_bits: np.ndarray, cam: OrcCamera, bits: np.ndarray | None, res: int, aabb, max_steps: int, rays: np.ndarray, t_stop: float = 1e-4,
                bg=(1.0, 1.0, 1.0), threads: int = 1, cascades: int = 1, kind: int = 0, stop: bool = False):
    """kind 0: hash-grid model (grid, table); kind 1: the reference's own
    network (ref_* parameter sets; grid and table unused).  Returns (rgb,
    rgba8, counts); with stop=True also (used, t_prev, t_final) per ray: the
    samples composited before the early stop, and the transmittance before and
    after the last of them."""
    model = OrcModel()
    if grid is not None:
        model.grid = grid
    model.table = _p(table) if table is not None else None
    model.kind = kind
    model.density_params = _p(dparams_bits)
    model.color_params = _p(cparams_bits)
    rays = np.ascontiguousarray(rays, np.uint32)
    box = np.array(aabb, np.float32)
    b = np.array(bg, np.float32)
    rgb = np.empty((rays.size, 3), np.float32)
    rgba = np.empty(rays.size, np.uint32)
    counts = np.empty(rays.size, np.uint32)
    used = np.empty(rays.size, np.uint32) if stop else None
    t_prev = np.empty(rays.size, np.float32) if stop else None
    t_final = np.empty(rays.size, np.float32) if stop else None
    lib().orc_render_rays(C.byref(model), C.byref(cam), _p(bits) if bits is not None else None, res, cascades, _p(box), max_steps, t_stop, _p(b), _p(rays), rays.size, _p(rgb), _p(rgba), _p(counts), threads,
                          _p(used) if stop else None, _p(t_prev) if stop else None, _p(t_final) if stop else None)
    if stop:
        return rgb, rgba, counts, used, t_prev, t_final
    return rgb, rgba, counts


def render_uniform(grid: OrcGrid | None, table: np.ndarray | None, dparams_bits: np.ndarray, cparams_bits: np.ndarray, cam: OrcCamera, aabb, spp: int, rays: np.ndarray, bg=(1.0, 1.0, 1.0), threads: int = 1, kind: int = 0):
    """The reference's inference sampling and composite for the given pixel
    rays: (rgb [n][3], rgba8 [n], sample counts [n])."""
    model = OrcModel()
    if grid is not None:
        model.grid = grid
    model.table = _p(table) if table is not None else None
    model.kind = kind
    model.density_params = _p(dparams_bits)
    model.color_params = _p(cparams_bits)
    rays = np.ascontiguousarray(rays, np.uint32)
    box = np.array(aabb, np.float32)
    b = np.array(bg, np.float32)
    rgb = np.empty((rays.size, 3), np.float32)
    rgba = np.empty(rays.size, np.uint32)
    counts = np.empty(rays.size, np.uint32)
    lib().orc_render_uniform(C.byref(model), C.byref(cam), _p(box), spp, _p(b), _p(rays), rays.size, _p(rgb), _p(rgba), _p(counts), threads)
    return rgb, rgba, counts


# ------------------------------------------------------------------ training
def composite_backward_ray(sraw, rgbraw, dt, gt, bg=(1.0, 1.0, 1.0), delta=0.1, inv_norm=1.0):
    sraw = np.ascontiguousarray(sraw, np.float32)
    rgbraw = np.ascontiguousarray(rgbraw, np.float32).reshape(-1, 3)
    dt = np.ascontiguousarray(dt, np.float32)
    gt = np.array(gt, np.float32)
    b = np.array(bg, np.float32)
    n = sraw.size
    ds = np.empty(n, np.float32)
    drgb = np.empty((n, 3), np.float32)
    pred = np.empty(3, np.float32)
    loss = lib().orc_composite_backward_ray(_p(sraw), _p(rgbraw), _p(dt), n, _p(gt), _p(b), delta, inv_norm, _p(ds), _p(drgb), _p(pred))
    return float(loss), ds, drgb, pred


def composite_backward_act(sigma, rgb, dt, gt, bg=(1.0, 1.0, 1.0), delta=0.1, inv_norm=1.0):
    """Composite backward from activations (sigma, rgb); gradients wrt raw outputs."""
    sigma = np.ascontiguousarray(sigma, np.float32)
    rgb = np.ascontiguousarray(rgb, np.float32).reshape(-1, 3)
    dt = np.ascontiguousarray(dt, np.float32)
    gt = np.array(gt, np.float32)
    b = np.array(bg, np.float32)
    n = sigma.size
    ds = np.empty(n, np.float32)
    drgb = np.empty((n, 3), np.float32)
    pred = np.empty(3, np.float32)
    loss = lib().orc_composite_backward_act(_p(sigma), _p(rgb), _p(dt), n, _p(gt), _p(b), delta, inv_norm, _p(ds), _p(drgb), _p(pred))
    return float(loss), ds, drgb, pred


def mlp_backward(dparams_bits, cparams_bits, features, dirs, dsraw, drgbraw, loss_scale):
    features = np.ascontiguousarray(features, np.float32)
    dirs = np.ascontiguousarray(dirs, np.float32)
    dsraw = np.ascontiguousarray(dsraw, np.float32)
    drgbraw = np.ascontiguousarray(drgbraw, np.float32)
    n = features.shape[0]
    dfeat = np.empty((n, 32), np.float32)
    dD = np.zeros(3072, np.float64)
    dC = np.zeros(7168, np.float64)
    lib().orc_mlp_backward(_p(dparams_bits), _p(cparams_bits), _p(features), _p(dirs), _p(dsraw), _p(drgbraw), n, loss_scale, _p(dfeat), _p(dD), _p(dC))
    return dfeat, dD, dC


def encode_backward(grid: OrcGrid, pos, dfeat):
    pos = np.ascontiguousarray(pos, np.float32)
    dfeat = np.ascontiguousarray(dfeat, np.float32)
    out = np.zeros(grid.n_levels * grid.table_size * 2, np.float64)
    lib().orc_encode_backward(C.byref(grid), _p(pos), _p(dfeat), pos.shape[0], _p(out))
    return out


def adam(w, m, v, g, lr, b1, b2, eps, clip, guard, loss_scale, decay_ksteps, step, grad_norm, nonfinite=0):
    for a in (w, m, v):
        assert a.dtype == np.float32 and a.flags["C_CONTIGUOUS"]
    g = np.ascontiguousarray(g, np.float32)
    return lib().orc_adam(_p(w), _p(m), _p(v), _p(g), w.size, lr, b1, b2, eps, clip, guard, loss_scale, decay_ksteps, step, grad_norm, nonfinite)


def train_rays(cam: OrcCamera, image: np.ndarray, bits, res: int, aabb, max_steps: int, frame: int, n_rays: int, cap: int):
    image = np.ascontiguousarray(image, np.uint8)
    box = np.array(aabb, np.float32)
    counts = np.empty(n_rays, np.uint32)
    gt = np.empty((n_rays, 4), np.float32)
    pix = np.empty((n_rays, 2), np.float32)
    offs = np.empty(n_rays, np.uint32)
    tdt = np.zeros((cap, 2), np.float32)
    lib().orc_train_rays(C.byref(cam), _p(image), _p(bits) if bits is not None else None, res, _p(box), max_steps, frame, n_rays, _p(counts), _p(gt), _p(pix), _p(offs), _p(tdt), cap)
    return counts, gt, pix, offs, tdt


def train_camera(frame: int, image_count: int) -> int:
    return int(lib().orc_train_camera(frame, image_count))


def scene_render(gaussians: np.ndarray, cam: OrcCamera, steps: int, aabb=(0, 0, 0, 1, 1, 1)) -> np.ndarray:
    """RGBA8 image [H][W] as uint32 words (R in the low byte)."""
    g = np.ascontiguousarray(gaussians, np.float32)
    box = np.array(aabb, np.float32)
    out = np.empty((cam.height, cam.width), np.uint32)
    lib().orc_scene_render(_p(g), g.shape[0], C.byref(cam), _p(box), steps, _p(out))
    return out


def field_mlp(dparams_bits, cparams_bits, features, dirs) -> np.ndarray:
    """Field MLPs on [n][32] features (fp16-rounded inside) and [n][3] unit directions -> [n][4]."""
    features = np.ascontiguousarray(features, np.float32)
    dirs = np.ascontiguousarray(dirs, np.float32)
    out = np.empty((features.shape[0], 4), np.float32)
    lib().orc_field_mlp(_p(dparams_bits), _p(cparams_bits), _p(features), _p(dirs), features.shape[0], _p(out))
    return out
