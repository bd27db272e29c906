"""ctypes bindings of libnerf.so: the reference ABI (include/nerf.h) and the
extension interface (include/nerf_ext.h).

Loading is strict: if libnerf.so is missing or lacks a symbol the import
fails loudly.  There is no fallback path of any kind.
"""
from __future__ import annotations

import ctypes as C
import os
from pathlib import Path

PKG = Path(__file__).resolve().parent
LIB_PATH = Path(os.environ.get("NERF_AMD_LIB", PKG / "libnerf.so"))

# ----------------------------------------------------------------- nerf.h
NERF_STATUS_OK = 0
NERF_STATUS_INVALID_USAGE = 1
NERF_STATUS_STATE_ERROR = 2
NERF_STATUS_IO_ERROR = 3
NERF_STATUS_CUDA_ERROR = 4
NERF_STATUS_FAILURE = 5
STATUS_NAMES = {0: "OK", 1: "INVALID_USAGE", 2: "STATE_ERROR", 3: "IO_ERROR", 4: "CUDA_ERROR", 5: "FAILURE"}

NERF_MEMORY_HOST = 1
NERF_MEMORY_CUDA_DEVICE = 2


class NerfCreateDesc(C.Structure):
    _fields_ = [
        ("occupancy_grid_res", C.c_uint32),
        ("max_sample_steps", C.c_uint32),
        ("max_batch_rays", C.c_uint32),
        ("arena_alignment_bytes", C.c_uint64),
        ("images_rgba8", C.c_void_p),
        ("images_bytes", C.c_uint64),
        ("cameras_4x4_packed", C.c_void_p),
        ("cameras_bytes", C.c_uint64),
        ("image_count", C.c_uint32),
        ("image_width", C.c_uint32),
        ("image_height", C.c_uint32),
        ("fx", C.c_float),
        ("fy", C.c_float),
        ("cx", C.c_float),
        ("cy", C.c_float),
    ]


class NerfHyperParams(C.Structure):
    _fields_ = [
        ("learning_rate", C.c_float),
        ("adam_beta1", C.c_float),
        ("adam_beta2", C.c_float),
        ("adam_eps", C.c_float),
        ("grad_clip_norm", C.c_float),
        ("update_guard_grad_norm", C.c_float),
        ("loss_scale", C.c_float),
        ("lr_decay_ksteps", C.c_uint32),
    ]


class NerfOccupancyParams(C.Structure):
    _fields_ = [
        ("decay", C.c_float),
        ("threshold", C.c_float),
        ("cells_per_update", C.c_uint32),
        ("update_interval", C.c_uint32),
        ("warmup_steps", C.c_uint32),
    ]


class NerfTrainingConfig(C.Structure):
    _fields_ = [
        ("aabb_min_x", C.c_float),
        ("aabb_min_y", C.c_float),
        ("aabb_min_z", C.c_float),
        ("aabb_max_x", C.c_float),
        ("aabb_max_y", C.c_float),
        ("aabb_max_z", C.c_float),
        ("hyper_params", NerfHyperParams),
        ("occupancy_params", NerfOccupancyParams),
        ("rays_per_batch", C.c_uint32),
        ("max_sample_steps_per_ray", C.c_uint32),
    ]


class NerfTrainStats(C.Structure):
    _fields_ = [
        ("loss", C.c_float),
        ("grad_norm", C.c_float),
        ("has_nonfinite", C.c_uint32),
        ("completed_steps", C.c_uint32),
        ("last_train_camera", C.c_uint32),
    ]


class NerfInferenceRequest(C.Structure):
    _fields_ = [
        ("camera_idx", C.c_uint32),
        ("samples_per_ray", C.c_uint32),
        ("memory_kind", C.c_uint32),
        ("dst_rgba8", C.c_void_p),
        ("dst_bytes", C.c_uint64),
    ]


class NerfInferenceInfo(C.Structure):
    _fields_ = [
        ("capacity_bytes", C.c_uint64),
        ("valid_bytes", C.c_uint64),
        ("row_stride_bytes", C.c_uint32),
        ("width", C.c_uint32),
        ("height", C.c_uint32),
        ("generation", C.c_uint32),
    ]


class NerfCheckpointFileDesc(C.Structure):
    _fields_ = [("path_utf8", C.c_char_p)]


# ------------------------------------------------------------- nerf_ext.h
NERF_EXT_F32 = 0
NERF_EXT_F16 = 1
NERF_EXT_MODEL_HASHGRID = 0
NERF_EXT_MODEL_REFERENCE = 1
NERF_EXT_SAMPLING_DEFAULT = 0
NERF_EXT_SAMPLING_UNIFORM = 1
NERF_EXT_SAMPLING_MARCH = 2
NERF_EXT_REF_DENSITY_PARAMS = 75776
NERF_EXT_REF_COLOR_PARAMS = 40960
NERF_EXT_H2D = 1
NERF_EXT_D2H = 2
NERF_EXT_D2D = 3
NERF_EXT_DENSITY_PARAMS = 3072
NERF_EXT_COLOR_PARAMS = 7168


class NerfExtDeviceInfo(C.Structure):
    _fields_ = [
        ("name", C.c_char * 64),
        ("arch", C.c_char * 32),
        ("compute_units", C.c_uint32),
        ("lds_bytes_per_block", C.c_uint32),
        ("global_mem_bytes", C.c_uint64),
        ("clock_khz", C.c_uint32),
        ("memory_clock_khz", C.c_uint32),
        ("memory_bus_bits", C.c_uint32),
        ("l2_bytes", C.c_uint32),
    ]


class NerfExtGridDesc(C.Structure):
    _fields_ = [
        ("n_levels", C.c_uint32),
        ("n_features", C.c_uint32),
        ("log2_table_size", C.c_uint32),
        ("base_resolution", C.c_uint32),
        ("per_level_scale", C.c_float),
        ("finest_resolution", C.c_uint32),
        ("table_dtype", C.c_uint32),
        ("reserved", C.c_uint32),
    ]


class NerfExtGridLevels(C.Structure):
    _fields_ = [
        ("n_levels", C.c_uint32),
        ("table_size", C.c_uint32),
        ("resolution", C.c_uint32 * 16),
        ("dense", C.c_uint32 * 16),
    ]


class NerfExtModel(C.Structure):
    _fields_ = [
        ("grid", NerfExtGridDesc),
        ("table", C.c_void_p),
        ("density_params", C.c_void_p),
        ("color_params", C.c_void_p),
        ("kind", C.c_uint32),
        ("reserved", C.c_uint32),
    ]


class NerfExtGaussian(C.Structure):
    _fields_ = [(k, C.c_float) for k in ("cx", "cy", "cz", "sigma", "amplitude", "r", "g", "b")]


class NerfExtSceneDesc(C.Structure):
    _fields_ = [
        ("count", C.c_uint32),
        ("reserved", C.c_uint32),
        ("seed", C.c_uint64),
        ("centre_lo", C.c_float),
        ("centre_hi", C.c_float),
        ("sigma_lo", C.c_float),
        ("sigma_hi", C.c_float),
        ("amplitude_lo", C.c_float),
        ("amplitude_hi", C.c_float),
    ]


class NerfExtOccupancy(C.Structure):
    _fields_ = [
        ("bitfield", C.c_void_p),
        ("resolution", C.c_uint32),
        ("aabb_min", C.c_float * 3),
        ("aabb_max", C.c_float * 3),
        ("cascades", C.c_uint32),
    ]


class NerfExtCamera(C.Structure):
    _fields_ = [
        ("c2w", C.c_float * 12),
        ("fx", C.c_float),
        ("fy", C.c_float),
        ("cx", C.c_float),
        ("cy", C.c_float),
        ("width", C.c_uint32),
        ("height", C.c_uint32),
    ]


class NerfExtRenderDesc(C.Structure):
    _fields_ = [
        ("model", C.POINTER(NerfExtModel)),
        ("occupancy", C.POINTER(NerfExtOccupancy)),
        ("cameras", C.POINTER(NerfExtCamera)),
        ("view_count", C.c_uint32),
        ("max_steps", C.c_uint32),
        ("min_transmittance", C.c_float),
        ("background", C.c_float * 3),
        ("stream", C.c_void_p),
        ("chunk_samples", C.c_uint64),
        ("composited", C.c_void_p),
        ("shaded", C.c_void_p),
    ]


class NerfExtRenderStats(C.Structure):
    _fields_ = [
        ("rays", C.c_uint64),
        ("samples", C.c_uint64),
        ("ms_count", C.c_float),
        ("ms_scan", C.c_float),
        ("ms_samples", C.c_float),
        ("ms_field", C.c_float),
        ("ms_composite", C.c_float),
        ("ms_total", C.c_float),
        ("samples_shaded", C.c_uint64),
    ]


class NerfExtContextOptions(C.Structure):
    _fields_ = [("model_kind", C.c_uint32), ("inference_sampling", C.c_uint32)]


class NerfExtTrainDesc(C.Structure):
    _fields_ = [
        ("grid", NerfExtGridDesc),
        ("images_rgba8", C.c_void_p),
        ("cameras", C.POINTER(NerfExtCamera)),
        ("image_count", C.c_uint32),
        ("occupancy_res", C.c_uint32),
        ("aabb_min", C.c_float * 3),
        ("aabb_max", C.c_float * 3),
        ("hyper", NerfHyperParams),
        ("occupancy", NerfOccupancyParams),
        ("initial_rays", C.c_uint32),
        ("max_rays", C.c_uint32),
        ("target_samples", C.c_uint32),
        ("sample_capacity", C.c_uint32),
        ("max_steps_per_ray", C.c_uint32),
        ("huber_delta", C.c_float),
        ("table_init_range", C.c_float),
        ("model_kind", C.c_uint32),
        ("seed", C.c_uint64),
    ]


class NerfExtTrainStats(C.Structure):
    _fields_ = [
        ("last", NerfTrainStats),
        ("rays", C.c_uint32),
        ("samples", C.c_uint32),
        ("active_rays", C.c_uint32),
        ("skipped", C.c_uint32),
        ("occupied_samples", C.c_uint64),
        ("samples_total", C.c_uint64),
    ]


class NerfExtTrainBuffers(C.Structure):
    _fields_ = [(k, C.c_void_p) for k in ("state", "rays", "gt", "counts", "kept", "offsets", "samples", "sample_ray", "field", "features", "draw", "table_grad", "mlp_grad", "table_f32", "mlp_f32",
                                          "table_m", "table_v", "mlp_m", "mlp_v", "bitfield", "density_grid")] + [("max_rays", C.c_uint32), ("sample_capacity", C.c_uint32), ("table_elems", C.c_uint64), ("dfeat", C.c_void_p),
                                                                                                                                       ("features_lm", C.c_void_p)]


NERF_EXT_STAGE_BEGIN, NERF_EXT_STAGE_OCCUPANCY, NERF_EXT_STAGE_SAMPLE, NERF_EXT_STAGE_FORWARD, NERF_EXT_STAGE_COMPOSITE, NERF_EXT_STAGE_BACKWARD, NERF_EXT_STAGE_ADAM, NERF_EXT_STAGE_END = range(8)

_S = C.c_int  # NerfStatus
_P = C.c_void_p
_U32 = C.c_uint32
_U64 = C.c_uint64
_F = C.c_float

# name -> (restype, argtypes).  Every symbol declared in include/nerf.h and
# include/nerf_ext.h appears here; tests/test_library.py checks the headers
# against this table and the library's exports.
PROTOTYPES: dict[str, tuple] = {
    # nerf.h
    "nerf_create_context": (_S, [C.POINTER(NerfCreateDesc), C.POINTER(_P)]),
    "nerf_destroy_context": (_S, [_P]),
    "nerf_configure_training": (_S, [_P, C.POINTER(NerfTrainingConfig)]),
    "nerf_train_step": (_S, [_P]),
    "nerf_read_train_stats": (_S, [_P, C.POINTER(NerfTrainStats)]),
    "nerf_inference": (_S, [_P, C.POINTER(NerfInferenceRequest), C.POINTER(NerfInferenceInfo)]),
    "nerf_save_network_weights": (_S, [_P, C.POINTER(NerfCheckpointFileDesc)]),
    "nerf_load_network_weights": (_S, [_P, C.POINTER(NerfCheckpointFileDesc)]),
    # nerf_ext.h: runtime
    "nerf_ext_last_error": (C.c_char_p, []),
    "nerf_ext_device_info": (_S, [C.POINTER(NerfExtDeviceInfo)]),
    "nerf_ext_malloc": (_S, [C.POINTER(_P), _U64]),
    "nerf_ext_free": (_S, [_P]),
    "nerf_ext_memcpy": (_S, [_P, _P, _U64, _U32]),
    "nerf_ext_memset": (_S, [_P, C.c_int, _U64]),
    "nerf_ext_synchronize": (_S, []),
    "nerf_ext_stream_create": (_S, [C.POINTER(_P)]),
    "nerf_ext_stream_destroy": (_S, [_P]),
    "nerf_ext_stream_synchronize": (_S, [_P]),
    "nerf_ext_event_create": (_S, [C.POINTER(_P)]),
    "nerf_ext_event_destroy": (_S, [_P]),
    "nerf_ext_event_record": (_S, [_P, _P]),
    "nerf_ext_event_elapsed_ms": (_S, [_P, _P, C.POINTER(_F)]),
    # hash grid
    "nerf_ext_grid_levels": (_S, [C.POINTER(NerfExtGridDesc), C.POINTER(NerfExtGridLevels)]),
    "nerf_ext_grid_init_table": (_S, [C.POINTER(NerfExtGridDesc), _U64, _F, _P, _P]),
    "nerf_ext_encode_forward": (_S, [C.POINTER(NerfExtGridDesc), _P, _P, _U32, _P, _U32, _P]),
    "nerf_ext_encode_indices": (_S, [C.POINTER(NerfExtGridDesc), _P, _U32, _P, _P, _P]),
    # MLPs
    "nerf_ext_mlp_init": (_S, [_U32, _P]),
    "nerf_ext_float_to_half": (_S, [_P, _P, _U64, _P]),
    "nerf_ext_density_mlp": (_S, [_P, _P, _U32, _P, _P]),
    "nerf_ext_density_forward": (_S, [C.POINTER(NerfExtGridDesc), _P, _P, _P, _U32, _P, _P]),
    "nerf_ext_field_mlp": (_S, [_P, _P, _P, _P, _U32, _P, _P]),
    "nerf_ext_field_forward": (_S, [C.POINTER(NerfExtModel), _P, _P, _U32, _P, _P]),
    "nerf_ext_ref_mlp_init": (_S, [_U32, _P]),
    "nerf_ext_ref_field_forward": (_S, [_P, _P, _P, _P, _U32, _P, _P, _P]),
    "nerf_ext_ref_composite_backward": (_S, [_P, _P, _P, _P, _P, _U32, _F, _P, _P, _P]),
    "nerf_ext_ref_backward": (_S, [_P, _P, _P, _P, _P, _U32, _F, _P, _P, _P]),
    "nerf_ext_ref_backward_rows": (_S, [_P, _P, _P, _P, _P, _U32, _F, _P, _P, _P, _P, _P]),
    # scene
    "nerf_ext_scene_gaussians": (_S, [C.POINTER(NerfExtSceneDesc), _P]),
    "nerf_ext_scene_density": (_S, [_P, _U32, _P, _U32, _P, _P]),
    "nerf_ext_occupancy_from_scene": (_S, [_P, _U32, _F, C.POINTER(NerfExtOccupancy), _P]),
    "nerf_ext_occupancy_mark_shell": (_S, [C.POINTER(NerfExtOccupancy), _P, _F, _F, _P]),
    # cameras, march, render
    "nerf_ext_camera_orbit": (_S, [_U64, _U32, _F, _P, _U32, _U32, _F, C.POINTER(NerfExtCamera)]),
    "nerf_ext_box_relative": (_S, [_P, _U32, C.POINTER(C.c_float), C.POINTER(C.c_float), _P, _P]),
    "nerf_ext_march_count": (_S, [C.POINTER(NerfExtCamera), C.POINTER(NerfExtOccupancy), _U32, _P, _P]),
    "nerf_ext_march_count_noalloc": (_S, [C.POINTER(NerfExtCamera), C.POINTER(NerfExtOccupancy), _U32, _P, _P]),
    "nerf_ext_renderer_create": (_S, [C.POINTER(_P)]),
    "nerf_ext_renderer_destroy": (_S, [_P]),
    "nerf_ext_render": (_S, [_P, C.POINTER(NerfExtRenderDesc), _P, _P, _P, C.POINTER(NerfExtRenderStats)]),
    "nerf_ext_render_uniform": (_S, [_P, C.POINTER(NerfExtModel), C.POINTER(NerfExtCamera), _U32, _P, _U32, _P, _P, _P, _P]),
    "nerf_ext_context_configure": (_S, [_P, C.POINTER(NerfExtContextOptions)]),
    "nerf_ext_context_options": (_S, [_P, C.POINTER(NerfExtContextOptions)]),
    "nerf_ext_scene_render": (_S, [_P, _U32, C.POINTER(NerfExtCamera), _U32, _P, _U32, _P, _P]),
    # training
    "nerf_ext_trainer_create": (_S, [C.POINTER(NerfExtTrainDesc), C.POINTER(_P)]),
    "nerf_ext_trainer_destroy": (_S, [_P]),
    "nerf_ext_trainer_step": (_S, [_P, _U32]),
    "nerf_ext_trainer_run_stages": (_S, [_P, _U32, _U32]),
    "nerf_ext_trainer_synchronize": (_S, [_P]),
    "nerf_ext_trainer_stats": (_S, [_P, C.POINTER(NerfExtTrainStats)]),
    "nerf_ext_trainer_buffers": (_S, [_P, C.POINTER(NerfExtTrainBuffers)]),
    "nerf_ext_trainer_model": (_S, [_P, C.POINTER(NerfExtModel), C.POINTER(NerfExtOccupancy)]),
    "nerf_ext_trainer_stream": (_P, [_P]),
}


class NerfError(RuntimeError):
    def __init__(self, fn: str, status: int, message: str):
        super().__init__(f"{fn} -> {STATUS_NAMES.get(status, status)}: {message}")
        self.status = status


_lib: C.CDLL | None = None


def load() -> C.CDLL:
    """Loads libnerf.so and binds every prototype; raises if anything is missing."""
    global _lib
    if _lib is not None:
        return _lib
    if not LIB_PATH.exists():
        raise FileNotFoundError(f"{LIB_PATH} is not built: run `python -m nerf_amd.build` (the HIP backend has no fallback)")
    lib = C.CDLL(str(LIB_PATH), mode=C.RTLD_LOCAL)
    for name, (res, args) in PROTOTYPES.items():
        fn = getattr(lib, name)  # AttributeError if the symbol is not exported
        fn.restype = res
        fn.argtypes = args
    _lib = lib
    return lib


def last_error() -> str:
    msg = load().nerf_ext_last_error()
    return msg.decode() if msg else ""


def call(name: str, *args) -> None:
    """Calls a NerfStatus-returning entry point and raises NerfError on failure."""
    status = getattr(load(), name)(*args)
    if status != NERF_STATUS_OK:
        raise NerfError(name, status, last_error())


def status_of(name: str, *args) -> int:
    """Calls an entry point and returns its raw NerfStatus (for error-path tests)."""
    return int(getattr(load(), name)(*args))
