"""Python mirror of include/nerf_ext.h: hash grids, MLP weights, the analytic
scene, cameras and rendering, all on device buffers.

The configurations of the benchmark plan are named here by their contents
(hash-grid shape, scene size, image size), not by number.
"""
from __future__ import annotations

import ctypes as C
from dataclasses import dataclass

import numpy as np

from . import _lib as L
from .device import DeviceArray, Stream

# 16 levels x 2 features, N_min 16, b 1.3819, uniform table init in +-1e-4.
HASH_PRIMES = (1, 2654435761, 805459861)


def grid_desc(log2_table_size: int, dtype: int, n_levels: int = 16, base: int = 16, per_level_scale: float = 1.3819, finest: int = 0) -> L.NerfExtGridDesc:
    return L.NerfExtGridDesc(n_levels, 2, log2_table_size, base, per_level_scale, finest, dtype, 0)


def grid_levels(desc: L.NerfExtGridDesc) -> tuple[np.ndarray, np.ndarray]:
    out = L.NerfExtGridLevels()
    L.call("nerf_ext_grid_levels", C.byref(desc), C.byref(out))
    n = out.n_levels
    return np.array(out.resolution[:n], np.uint32), np.array(out.dense[:n], np.uint32)


def table_elements(desc: L.NerfExtGridDesc) -> int:
    return desc.n_levels * (1 << desc.log2_table_size) * desc.n_features


def init_table(desc: L.NerfExtGridDesc, seed: int = 0, value_range: float = 1e-4) -> DeviceArray:
    dtype = np.float32 if desc.table_dtype == L.NERF_EXT_F32 else np.float16
    table = DeviceArray((table_elements(desc),), dtype)
    L.call("nerf_ext_grid_init_table", C.byref(desc), seed, value_range, table.ptr, None)
    return table


def mlp_init(network: int) -> np.ndarray:
    n = L.NERF_EXT_DENSITY_PARAMS if network == 0 else L.NERF_EXT_COLOR_PARAMS
    out = np.empty(n, np.float32)
    L.call("nerf_ext_mlp_init", network, out.ctypes.data)
    return out


def encode_forward(desc, table: DeviceArray, positions: DeviceArray, n: int, out: DeviceArray, stream: Stream | None = None) -> None:
    dt = L.NERF_EXT_F32 if out.dtype == np.float32 else L.NERF_EXT_F16
    L.call("nerf_ext_encode_forward", C.byref(desc), table.ptr, positions.ptr, n, out.ptr, dt, stream.handle if stream else None)


@dataclass
class Model:
    """Hash grid + density/colour MLP weights resident on the device."""

    grid: L.NerfExtGridDesc
    table: DeviceArray
    density_f32: np.ndarray
    color_f32: np.ndarray
    density: DeviceArray
    color: DeviceArray

    @classmethod
    def create(cls, grid: L.NerfExtGridDesc, seed: int = 0, table_range: float = 1e-4) -> "Model":
        table = init_table(grid, seed, table_range)
        d32 = mlp_init(0)
        c32 = mlp_init(1)
        return cls(grid, table, d32, c32, DeviceArray.from_numpy(d32.astype(np.float16)), DeviceArray.from_numpy(c32.astype(np.float16)))

    def struct(self) -> L.NerfExtModel:
        return L.NerfExtModel(self.grid, self.table.ptr, self.density.ptr, self.color.ptr)


def ref_mlp_init(network: int) -> np.ndarray:
    """The reference's init (backend-cuda.cu:1810-1847) on its own network."""
    n = L.NERF_EXT_REF_DENSITY_PARAMS if network == 0 else L.NERF_EXT_REF_COLOR_PARAMS
    out = np.empty(n, np.float32)
    L.call("nerf_ext_ref_mlp_init", network, out.ctypes.data)
    return out


@dataclass
class RefModel:
    """Reference-model mode: the reference's own network (frequency encoding,
    128-wide MLPs, softplus density) with fp16 weights on the device."""

    density_f32: np.ndarray
    color_f32: np.ndarray
    density: DeviceArray
    color: DeviceArray

    @classmethod
    def create(cls, density_f32: np.ndarray | None = None, color_f32: np.ndarray | None = None) -> "RefModel":
        d32 = ref_mlp_init(0) if density_f32 is None else np.asarray(density_f32, np.float32)
        c32 = ref_mlp_init(1) if color_f32 is None else np.asarray(color_f32, np.float32)
        return cls(d32, c32, DeviceArray.from_numpy(d32.astype(np.float16)), DeviceArray.from_numpy(c32.astype(np.float16)))

    def struct(self) -> L.NerfExtModel:
        m = L.NerfExtModel()
        m.density_params = self.density.ptr
        m.color_params = self.color.ptr
        m.kind = L.NERF_EXT_MODEL_REFERENCE
        return m


def scene_gaussians(count: int, seed: int = 0, centre=(0.2, 0.8), sigma=(0.02, 0.1), amplitude=(5.0, 50.0)) -> np.ndarray:
    """Analytic scene records as a structured array (cx cy cz sigma A r g b)."""
    desc = L.NerfExtSceneDesc(count, 0, seed, centre[0], centre[1], sigma[0], sigma[1], amplitude[0], amplitude[1])
    out = (L.NerfExtGaussian * count)()
    L.call("nerf_ext_scene_gaussians", C.byref(desc), C.cast(out, C.c_void_p))
    return np.frombuffer(out, dtype=np.float32).reshape(count, 8).copy()


def occupancy_struct(bits: DeviceArray, res: int, aabb_min=(0.0, 0.0, 0.0), aabb_max=(1.0, 1.0, 1.0), cascades: int = 1) -> L.NerfExtOccupancy:
    return L.NerfExtOccupancy(bits.ptr, res, (C.c_float * 3)(*aabb_min), (C.c_float * 3)(*aabb_max), cascades)


def occupancy_words(res: int, cascades: int = 1) -> int:
    """Bitfield length: one word-aligned grid of res^3 bits per cascade."""
    return cascades * ((res ** 3 + 31) // 32)


def occupancy_from_scene(gaussians: np.ndarray, res: int, threshold: float = 0.01, aabb_min=(0.0, 0.0, 0.0), aabb_max=(1.0, 1.0, 1.0), cascades: int = 1, shell=None) -> DeviceArray:
    """Bitfield of the scene's density > threshold at cell centres, every
    cascade; shell = (centre3, r_inner, r_outer) also marks a uniform shell."""
    bits = DeviceArray.zeros((occupancy_words(res, cascades),), np.uint32)
    g = DeviceArray.from_numpy(np.ascontiguousarray(gaussians, np.float32))
    occ = occupancy_struct(bits, res, aabb_min, aabb_max, cascades)
    L.call("nerf_ext_occupancy_from_scene", g.ptr, gaussians.shape[0], threshold, C.byref(occ), None)
    if shell is not None:
        centre, r_in, r_out = shell
        c3 = (C.c_float * 3)(*centre)
        L.call("nerf_ext_occupancy_mark_shell", C.byref(occ), C.cast(c3, C.c_void_p), r_in, r_out, None)
    return bits


def camera_orbit(seed: int, index: int, radius: float, centre, width: int, height: int, focal: float) -> L.NerfExtCamera:
    cam = L.NerfExtCamera()
    c3 = (C.c_float * 3)(*centre)
    L.call("nerf_ext_camera_orbit", seed, index, radius, C.cast(c3, C.c_void_p), width, height, focal, C.byref(cam))
    return cam


def camera_array(cam: L.NerfExtCamera) -> np.ndarray:
    """Camera as the 18-word host record the oracle takes (floats then u32s)."""
    buf = np.frombuffer(bytes(cam), dtype=np.uint8).copy()
    return buf


class Renderer:
    def __init__(self):
        self._h = C.c_void_p()
        L.call("nerf_ext_renderer_create", C.byref(self._h))

    def render(self, model: "Model | RefModel", occupancy: L.NerfExtOccupancy, cameras: list, max_steps: int, min_transmittance: float = 1e-4, background=(1.0, 1.0, 1.0), rgba8: DeviceArray | None = None, rgb: DeviceArray | None = None,
               counts: DeviceArray | None = None, stream: Stream | None = None, timed: bool = False, chunk_samples: int = 0, composited: DeviceArray | None = None, shaded: DeviceArray | None = None):
        n_views = len(cameras)
        w, h = cameras[0].width, cameras[0].height
        if rgba8 is None:
            rgba8 = DeviceArray((n_views, h, w), np.uint32)
        cams = (L.NerfExtCamera * n_views)(*cameras)
        ms = model.struct()
        desc = L.NerfExtRenderDesc(C.pointer(ms), C.pointer(occupancy), cams, n_views, max_steps, min_transmittance, (C.c_float * 3)(*background), stream.handle if stream else None, chunk_samples,
                                   composited.ptr if composited else None, shaded.ptr if shaded else None)
        stats = L.NerfExtRenderStats()
        L.call("nerf_ext_render", self._h, C.byref(desc), rgba8.ptr, rgb.ptr if rgb else None, counts.ptr if counts else None, C.byref(stats) if timed else None)
        return rgba8, (stats if timed else None)

    def __del__(self):
        try:
            if self._h.value and L._lib is not None:
                L._lib.nerf_ext_renderer_destroy(self._h)
        except Exception:
            pass


def read_device(ptr: int, shape, dtype) -> np.ndarray:
    """Copies `shape` elements of `dtype` from a raw device pointer."""
    out = np.empty(shape, dtype)
    if out.nbytes:
        L.call("nerf_ext_memcpy", out.ctypes.data, int(ptr), out.nbytes, L.NERF_EXT_D2H)
    return out


def write_device(ptr: int, values: np.ndarray) -> None:
    """Copies a host array into device memory at a raw device pointer."""
    values = np.ascontiguousarray(values)
    if values.nbytes:
        L.call("nerf_ext_memcpy", int(ptr), values.ctypes.data, values.nbytes, L.NERF_EXT_H2D)


def scene_render(gaussians: np.ndarray, cameras: list, steps: int, aabb=(0.0, 0.0, 0.0, 1.0, 1.0, 1.0), stream: Stream | None = None) -> DeviceArray:
    """Renders the analytic scene into RGBA8 images [views][H][W] (alpha =
    1 - transmittance, composited over white)."""
    g = DeviceArray.from_numpy(np.ascontiguousarray(gaussians, np.float32))
    n_views = len(cameras)
    w, h = cameras[0].width, cameras[0].height
    out = DeviceArray((n_views, h, w), np.uint32)
    cams = (L.NerfExtCamera * n_views)(*cameras)
    box = (C.c_float * 6)(*aabb)
    L.call("nerf_ext_scene_render", g.ptr, gaussians.shape[0], cams, n_views, C.cast(box, C.c_void_p), steps, out.ptr, stream.handle if stream else None)
    if stream is not None:
        stream.synchronize()
    else:
        from .device import synchronize

        synchronize()
    return out


def hyper_params(lr=1e-2, beta1=0.9, beta2=0.99, eps=1e-15, clip=1e30, guard=1e30, loss_scale=1.0, lr_decay_ksteps=0) -> L.NerfHyperParams:
    return L.NerfHyperParams(lr, beta1, beta2, eps, clip, guard, loss_scale, lr_decay_ksteps)


def occupancy_params(decay=0.95, threshold=0.01, cells_per_update=1 << 30, update_interval=16, warmup_steps=256) -> L.NerfOccupancyParams:
    return L.NerfOccupancyParams(decay, threshold, cells_per_update, update_interval, warmup_steps)


class Trainer:
    """One training run (nerf_ext_trainer_*): dataset, model, optimiser state
    and the buffers of one step, all on the device."""

    def __init__(self, grid: L.NerfExtGridDesc, images_rgba8: np.ndarray, cameras: list, *, occupancy_res=128, aabb_min=(0.0, 0.0, 0.0), aabb_max=(1.0, 1.0, 1.0), hyper: L.NerfHyperParams | None = None,
                 occupancy: L.NerfOccupancyParams | None = None, initial_rays=4096, max_rays=1 << 18, target_samples=0, sample_capacity=1 << 20, max_steps_per_ray=1024, huber_delta=0.1, table_init_range=1e-4, seed=0,
                 model_kind=L.NERF_EXT_MODEL_HASHGRID):
        images = np.ascontiguousarray(images_rgba8)
        n = len(cameras)
        self._cams = (L.NerfExtCamera * n)(*cameras)
        d = L.NerfExtTrainDesc()
        d.grid = grid
        d.images_rgba8 = images.ctypes.data
        d.cameras = self._cams
        d.image_count = n
        d.occupancy_res = occupancy_res
        d.aabb_min = (C.c_float * 3)(*aabb_min)
        d.aabb_max = (C.c_float * 3)(*aabb_max)
        d.hyper = hyper or hyper_params()
        d.occupancy = occupancy or occupancy_params()
        d.initial_rays = initial_rays
        d.max_rays = max_rays
        d.target_samples = target_samples
        d.sample_capacity = sample_capacity
        d.max_steps_per_ray = max_steps_per_ray
        d.huber_delta = huber_delta
        d.table_init_range = table_init_range
        d.seed = seed
        d.model_kind = model_kind
        self.desc = d
        self._h = C.c_void_p()
        L.call("nerf_ext_trainer_create", C.byref(d), C.byref(self._h))

    @property
    def handle(self) -> int:
        return int(self._h.value or 0)

    def step(self, steps: int = 1) -> None:
        L.call("nerf_ext_trainer_step", self._h, steps)

    def run_stages(self, first: int, last: int) -> None:
        L.call("nerf_ext_trainer_run_stages", self._h, first, last)

    def synchronize(self) -> None:
        L.call("nerf_ext_trainer_synchronize", self._h)

    def stats(self) -> L.NerfExtTrainStats:
        out = L.NerfExtTrainStats()
        L.call("nerf_ext_trainer_stats", self._h, C.byref(out))
        return out

    def buffers(self) -> L.NerfExtTrainBuffers:
        out = L.NerfExtTrainBuffers()
        L.call("nerf_ext_trainer_buffers", self._h, C.byref(out))
        return out

    def model(self) -> tuple[L.NerfExtModel, L.NerfExtOccupancy]:
        m, o = L.NerfExtModel(), L.NerfExtOccupancy()
        L.call("nerf_ext_trainer_model", self._h, C.byref(m), C.byref(o))
        return m, o

    def stream(self) -> int:
        return int(L.load().nerf_ext_trainer_stream(self._h) or 0)

    def close(self) -> None:
        if self._h.value:
            L.call("nerf_ext_trainer_destroy", self._h)
            self._h = C.c_void_p()

    def __del__(self):
        try:
            if self._h.value and L._lib is not None:
                L._lib.nerf_ext_trainer_destroy(self._h)
        except Exception:
            pass
