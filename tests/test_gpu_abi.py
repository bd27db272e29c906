"""The reference ABI (include/nerf.h) end to end on the GPU: context creation
from a rendered dataset, inference parity with the oracle, training steps and
statistics, checkpoint save/load round trips and the state-error paths that
need a live context (backend-cuda.cu:1994-2592)."""
import ctypes as C
import json
import struct

import numpy as np
import pytest

from conftest import announce
from helpers import L, ext, orc, oracle_grid

pytestmark = pytest.mark.gpu

W, H, VIEWS = 40, 32, 4
FOCAL = 1111.0 * W / 800.0
CENTRE = (0.5, 0.5, 0.5)
BOX = (0.0, 0.0, 0.0, 1.0, 1.0, 1.0)


@pytest.fixture(scope="module")
def dataset():
    g = ext.scene_gaussians(16, seed=4)
    cams = [ext.camera_orbit(11, i, 1.32, CENTRE, W, H, FOCAL) for i in range(VIEWS)]
    imgs = np.ascontiguousarray(ext.scene_render(g, cams, 128).numpy())
    mats = np.zeros((VIEWS, 4, 4), np.float32)
    for i, c in enumerate(cams):
        mats[i, :3, :] = np.array(c.c2w[:], np.float32).reshape(3, 4)
        mats[i, 3, 3] = 1.0
    return cams, imgs, mats


class Context:
    def __init__(self, dataset, occ_res=32):
        cams, imgs, mats = dataset
        self._keep = (imgs, mats)
        d = L.NerfCreateDesc(occ_res, 1 << 20, 4096, 256, imgs.ctypes.data, imgs.nbytes, mats.ctypes.data, mats.nbytes, VIEWS, W, H, cams[0].fx, cams[0].fy, cams[0].cx, cams[0].cy)
        self.h = C.c_void_p()
        L.call("nerf_create_context", C.byref(d), C.byref(self.h))

    def status(self, name, *args):
        return L.status_of(name, self.h, *args)

    def infer(self, camera_idx, samples=128):
        out = np.zeros((H, W), np.uint32)
        req = L.NerfInferenceRequest(camera_idx, samples, L.NERF_MEMORY_HOST, out.ctypes.data, out.nbytes)
        info = L.NerfInferenceInfo()
        L.call("nerf_inference", self.h, C.byref(req), C.byref(info))
        return out, info

    def save(self, path):
        L.call("nerf_save_network_weights", self.h, C.byref(L.NerfCheckpointFileDesc(str(path).encode())))

    def load(self, path):
        return self.status("nerf_load_network_weights", C.byref(L.NerfCheckpointFileDesc(str(path).encode())))

    def close(self):
        if self.h.value:
            L.call("nerf_destroy_context", self.h)
            self.h = C.c_void_p()


def _config(rays=1024, steps=64, warmup=4, interval=4):
    return L.NerfTrainingConfig(0.0, 0.0, 0.0, 1.0, 1.0, 1.0, ext.hyper_params(loss_scale=128.0), ext.occupancy_params(warmup_steps=warmup, update_interval=interval, cells_per_update=1 << 15), rays, steps)


def _read_checkpoint(path):
    raw = open(path, "rb").read()
    (n,) = struct.unpack("<Q", raw[:8])
    header = json.loads(raw[8:8 + n])
    base = 8 + n

    def tensor(name):
        b, e = header[name]["data_offsets"]
        return np.frombuffer(raw[base + b:base + e], np.float32).reshape(header[name]["shape"])

    return header, tensor


def _oracle_image(path, cam, bits=None, res=1, samples=128):
    header, t = _read_checkpoint(path)
    assert header["__metadata__"]["format"] == "nerf/hashgrid-network-v1"
    dp = np.concatenate([t("density.input.weight").ravel(), t("density.output.weight").ravel()])
    cp = np.concatenate([t("color.input.weight").ravel(), t("color.hidden.0.weight").ravel(), t("color.output.weight").ravel()])
    table = t("encoding.hash_table").ravel().astype(np.float16).view(np.uint16)
    grid = oracle_grid(ext.grid_desc(19, L.NERF_EXT_F16))
    ocam = orc.camera_from_bytes(bytes(cam))
    _, rgba, _ = orc.render_rays(grid, table, dp.astype(np.float16).view(np.uint16), cp.astype(np.float16).view(np.uint16), ocam, bits, res, BOX, samples, np.arange(W * H, dtype=np.uint32), threads=8)
    return rgba.reshape(H, W)


def _close_rgba(got, want):
    d = np.abs(got.view(np.uint8).astype(int) - want.view(np.uint8).astype(int))
    assert d.max() <= 1, f"max RGBA8 difference {d.max()}"


def test_state_errors_need_configuration(dataset):
    announce("abi state errors")
    ctx = Context(dataset)
    try:
        assert ctx.status("nerf_train_step") == L.NERF_STATUS_STATE_ERROR
        st = L.NerfTrainStats()
        assert ctx.status("nerf_read_train_stats", C.byref(st)) == L.NERF_STATUS_STATE_ERROR
        out = np.zeros((H, W), np.uint32)
        req = L.NerfInferenceRequest(VIEWS, 64, L.NERF_MEMORY_HOST, out.ctypes.data, out.nbytes)
        assert ctx.status("nerf_inference", C.byref(req), None) == L.NERF_STATUS_INVALID_USAGE
        for bad in (_config(steps=257), _config(rays=0), _config(rays=8192), _config(interval=0)):
            assert ctx.status("nerf_configure_training", C.byref(bad)) == L.NERF_STATUS_INVALID_USAGE
    finally:
        ctx.close()


def test_inference_matches_oracle_and_checkpoint_round_trip(dataset, tmp_path):
    announce("abi inference + checkpoint")
    cams = dataset[0]
    ctx = Context(dataset)
    try:
        path = tmp_path / "a.ckpt"
        ctx.save(path)
        img, info = ctx.infer(1)
        assert (info.width, info.height, info.row_stride_bytes, info.valid_bytes) == (W, H, 4 * W, 4 * W * H)
        _close_rgba(img, _oracle_image(path, cams[1]))
        # Load into a second context: identical weights, identical images and files.
        ctx2 = Context(dataset)
        try:
            assert ctx2.load(path) == L.NERF_STATUS_OK
            img2, _ = ctx2.infer(1)
            assert np.array_equal(img, img2)
            ctx2.save(tmp_path / "b.ckpt")
            assert (tmp_path / "a.ckpt").read_bytes() == (tmp_path / "b.ckpt").read_bytes()
        finally:
            ctx2.close()
        assert ctx.load(tmp_path / "missing.ckpt") == L.NERF_STATUS_IO_ERROR
    finally:
        ctx.close()


def test_training_through_the_abi(dataset, tmp_path):
    announce("abi training 60 steps")
    cams = dataset[0]
    ctx = Context(dataset)
    try:
        assert ctx.status("nerf_configure_training", C.byref(_config())) == L.NERF_STATUS_OK
        losses = []
        for i in range(60):
            L.call("nerf_train_step", ctx.h)
            if i % 10 == 9:
                st = L.NerfTrainStats()
                L.call("nerf_read_train_stats", ctx.h, C.byref(st))
                assert st.has_nonfinite == 0 and np.isfinite(st.loss) and st.grad_norm > 0
                losses.append(st.loss)
        assert st.completed_steps == 60
        assert st.last_train_camera == orc.train_camera(59, VIEWS)
        assert losses[-1] < losses[0]
        img, info = ctx.infer(2)
        assert info.generation == 60
        # Inference of a trained context uses its occupancy bitfield and AABB.
        path = tmp_path / "t.ckpt"
        ctx.save(path)
        # Loading keeps training configured and restarts its step counter.
        assert ctx.load(path) == L.NERF_STATUS_OK
        L.call("nerf_train_step", ctx.h)
        st = L.NerfTrainStats()
        L.call("nerf_read_train_stats", ctx.h, C.byref(st))
        assert st.completed_steps == 1
    finally:
        ctx.close()
