"""Error behaviour of the reference ABI that is decided on the host before
any GPU work (backend-cuda.cu:1995, :2099, :2126, :2406, :2422, :2437, :2467,
:2527): null arguments and a null context."""
import ctypes as C

from nerf_amd import _lib as L


def test_null_arguments(lib):
    assert L.status_of("nerf_create_context", None, None) == L.NERF_STATUS_INVALID_USAGE
    out = C.c_void_p()
    assert L.status_of("nerf_create_context", None, C.byref(out)) == L.NERF_STATUS_INVALID_USAGE
    assert L.status_of("nerf_destroy_context", None) == L.NERF_STATUS_OK
    assert L.status_of("nerf_configure_training", None, None) == L.NERF_STATUS_INVALID_USAGE
    assert L.status_of("nerf_train_step", None) == L.NERF_STATUS_INVALID_USAGE
    assert L.status_of("nerf_read_train_stats", None, None) == L.NERF_STATUS_INVALID_USAGE
    assert L.status_of("nerf_inference", None, None, None) == L.NERF_STATUS_INVALID_USAGE
    assert L.status_of("nerf_save_network_weights", None, None) == L.NERF_STATUS_INVALID_USAGE
    assert L.status_of("nerf_load_network_weights", None, None) == L.NERF_STATUS_INVALID_USAGE


def test_bad_alignment_rejected_before_gpu(lib):
    d = L.NerfCreateDesc()
    d.arena_alignment_bytes = 48  # not a power of two
    out = C.c_void_p()
    assert L.status_of("nerf_create_context", C.byref(d), C.byref(out)) == L.NERF_STATUS_INVALID_USAGE
    assert out.value is None


def test_ext_argument_checks(lib):
    # Grid validation happens on the host.
    g = L.NerfExtGridDesc(17, 2, 19, 16, 1.3819, 0, 1, 0)
    lv = L.NerfExtGridLevels()
    assert L.status_of("nerf_ext_grid_levels", C.byref(g), C.byref(lv)) == L.NERF_STATUS_INVALID_USAGE
    assert "n_levels" in L.last_error()
    g = L.NerfExtGridDesc(16, 3, 19, 16, 1.3819, 0, 1, 0)
    assert L.status_of("nerf_ext_grid_levels", C.byref(g), C.byref(lv)) == L.NERF_STATUS_INVALID_USAGE
