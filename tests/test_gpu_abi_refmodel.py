"""The reference ABI (include/nerf.h) with the reference's own network behind
it: selected with nerf_ext_context_configure or by loading a reference
checkpoint, trained through nerf_configure_training / nerf_train_step,
rendered by nerf_inference with the reference's sampling (spp uniform
samples per ray over the box, no occupancy, no early stop:
backend-cuda.cu:534-635) and saved in the reference's "nerf/network-v1"
format (:2466-2525, tensor names :1213-1241).

Bars: inference RGBA8 within 1 LSB of the oracle's restatement of the
reference's sampling and composite on the same weights; checkpoint headers
equal, byte for byte, the compact sorted-key JSON the reference's writer
produces for these tensors and dimensions; save -> load -> save
byte-identical; a loaded checkpoint renders the image the saving context
rendered.
"""
import ctypes as C
import json
import struct

import numpy as np
import pytest

from conftest import announce
from helpers import L, ext, orc, oracle_grid
from test_gpu_abi import BOX, H, VIEWS, W, Context, _close_rgba, _config, dataset  # noqa: F401  (fixture)

pytestmark = pytest.mark.gpu

REF_TENSORS = [("density.input.weight", [128, 64])] + [(f"density.hidden.{k}.weight", [128, 128]) for k in range(4)] + [("density.output.weight", [16, 128]), ("color.input.weight", [128, 48])] + \
              [(f"color.hidden.{k}.weight", [128, 128]) for k in range(2)] + [("color.output.weight", [16, 128])]
REF_META = {"format": "nerf/network-v1", "density_input_dim": 64, "density_hidden_layers": 5, "density_width": 128, "density_output_dim": 16, "color_input_dim": 48, "color_hidden_layers": 3,
            "color_width": 128, "color_output_dim": 16}


def _configure(ctx, kind, sampling=L.NERF_EXT_SAMPLING_DEFAULT):
    L.call("nerf_ext_context_configure", ctx.h, C.byref(L.NerfExtContextOptions(kind, sampling)))


def _options(ctx):
    o = L.NerfExtContextOptions()
    L.call("nerf_ext_context_options", ctx.h, C.byref(o))
    return o.model_kind, o.inference_sampling


def _header(path):
    raw = open(path, "rb").read()
    (n,) = struct.unpack("<Q", raw[:8])
    return raw, raw[8:8 + n], 8 + n


def _reference_header_bytes(tensors, meta):
    """The header the reference's writer emits: nlohmann::json objects keep
    their keys sorted and dump() is compact."""
    h = {"__metadata__": meta}
    off = 0
    for name, shape in tensors:
        nbytes = 4 * int(np.prod(shape))
        h[name] = {"dtype": "F32", "shape": shape, "data_offsets": [off, off + nbytes]}
        off += nbytes
    return json.dumps(h, sort_keys=True, separators=(",", ":")).encode()


def _ref_weights(path):
    raw, hdr, base = _header(path)
    h = json.loads(hdr)

    def t(name):
        b, e = h[name]["data_offsets"]
        return np.frombuffer(raw[base + b:base + e], np.float32)

    dp = np.concatenate([t(n) for n, _ in REF_TENSORS[:6]]).astype(np.float16).view(np.uint16)
    cp = np.concatenate([t(n) for n, _ in REF_TENSORS[6:]]).astype(np.float16).view(np.uint16)
    return dp, cp


def _oracle_uniform(cams, view, dp, cp, spp, rays, kind=1, grid=None, table=None):
    _, rgba, counts = orc.render_uniform(grid, table, dp, cp, orc.camera_from_bytes(bytes(cams[view])), BOX, spp, rays, threads=8, kind=kind)
    return rgba, counts


def test_reference_model_through_the_abi(dataset, tmp_path):
    cams, _, _ = dataset
    announce("reference model behind nerf.h: train, infer, save, load")
    ctx = Context(dataset)
    try:
        assert _options(ctx) == (L.NERF_EXT_MODEL_HASHGRID, L.NERF_EXT_SAMPLING_DEFAULT)
        _configure(ctx, L.NERF_EXT_MODEL_REFERENCE)
        assert _options(ctx)[0] == L.NERF_EXT_MODEL_REFERENCE
        L.call("nerf_configure_training", ctx.h, C.byref(_config(rays=512, steps=64)))
        for _ in range(30):
            L.call("nerf_train_step", ctx.h)
        st = L.NerfTrainStats()
        L.call("nerf_read_train_stats", ctx.h, C.byref(st))
        assert st.completed_steps == 30 and st.has_nonfinite == 0 and np.isfinite(st.loss) and st.loss > 0
        img, info = ctx.infer(1, samples=24)
        assert info.generation == 30
        path = tmp_path / "ref.ckpt"
        ctx.save(path)
        raw, hdr, _ = _header(path)
        assert hdr == _reference_header_bytes(REF_TENSORS, REF_META), "header differs from the reference writer's"
        assert len(raw) == len(hdr) + 8 + 4 * (75776 + 40960)
        dp, cp = _ref_weights(path)
        rays = np.arange(0, W * H, 3, dtype=np.uint32)
        want, counts = _oracle_uniform(cams, 1, dp, cp, 24, rays)
        assert (counts == 24).mean() > 0.3
        _close_rgba(img.ravel()[rays], want)
        # A fresh context (hash-grid by default) takes the reference file and
        # becomes a reference-model context; same image, same file back.
        ctx2 = Context(dataset)
        try:
            assert ctx2.load(path) == L.NERF_STATUS_OK
            assert _options(ctx2)[0] == L.NERF_EXT_MODEL_REFERENCE
            img2, _ = ctx2.infer(1, samples=24)
            assert np.array_equal(img2, img)
            path2 = tmp_path / "ref2.ckpt"
            ctx2.save(path2)
            assert open(path2, "rb").read() == raw
        finally:
            ctx2.close()
        # Loading into the training context restarts the step counter and
        # keeps training configured on the reference model.
        assert ctx.load(path) == L.NERF_STATUS_OK
        L.call("nerf_train_step", ctx.h)
        L.call("nerf_read_train_stats", ctx.h, C.byref(st))
        assert st.completed_steps == 1 and st.has_nonfinite == 0
    finally:
        ctx.close()


def test_model_switch_rebuilds_training(dataset, tmp_path):
    announce("nerf.h context: model switch with training configured, both ways")
    ctx = Context(dataset)
    try:
        L.call("nerf_configure_training", ctx.h, C.byref(_config(rays=256, steps=64)))
        L.call("nerf_train_step", ctx.h)
        for kind in (L.NERF_EXT_MODEL_REFERENCE, L.NERF_EXT_MODEL_HASHGRID):
            _configure(ctx, kind)
            for _ in range(3):
                L.call("nerf_train_step", ctx.h)
            st = L.NerfTrainStats()
            L.call("nerf_read_train_stats", ctx.h, C.byref(st))
            assert st.completed_steps == 3 and st.has_nonfinite == 0, (kind, st.completed_steps)
        # A hash-grid file switches a reference-model context back.
        path = tmp_path / "hash.ckpt"
        ctx.save(path)
        _configure(ctx, L.NERF_EXT_MODEL_REFERENCE)
        assert ctx.load(path) == L.NERF_STATUS_OK
        assert _options(ctx)[0] == L.NERF_EXT_MODEL_HASHGRID
        # An unknown format is refused and leaves the context as it was.
        bad = tmp_path / "bad.ckpt"
        hdr = b'{"__metadata__":{"format":"something/else"}}'
        bad.write_bytes(struct.pack("<Q", len(hdr)) + hdr)
        assert ctx.load(bad) == L.NERF_STATUS_IO_ERROR
        assert _options(ctx)[0] == L.NERF_EXT_MODEL_HASHGRID
    finally:
        ctx.close()


def test_uniform_sampling_for_the_hash_grid(dataset, tmp_path):
    """The hash-grid model with the reference's sampling selected: nerf_inference
    against the oracle's uniform render of the saved weights."""
    cams, _, _ = dataset
    announce("hash-grid model, uniform inference sampling")
    ctx = Context(dataset)
    try:
        _configure(ctx, L.NERF_EXT_MODEL_HASHGRID, L.NERF_EXT_SAMPLING_UNIFORM)
        L.call("nerf_configure_training", ctx.h, C.byref(_config(rays=1024, steps=64)))
        for _ in range(20):
            L.call("nerf_train_step", ctx.h)
        img, _ = ctx.infer(2, samples=40)
        path = tmp_path / "h.ckpt"
        ctx.save(path)
        raw, hdr, base = _header(path)
        h = json.loads(hdr)

        def t(name):
            b, e = h[name]["data_offsets"]
            return np.frombuffer(raw[base + b:base + e], np.float32)

        dp = np.concatenate([t("density.input.weight"), t("density.output.weight")]).astype(np.float16).view(np.uint16)
        cp = np.concatenate([t("color.input.weight"), t("color.hidden.0.weight"), t("color.output.weight")]).astype(np.float16).view(np.uint16)
        table = t("encoding.hash_table").astype(np.float16).view(np.uint16)
        grid = oracle_grid(ext.grid_desc(19, L.NERF_EXT_F16))
        rays = np.arange(W * H, dtype=np.uint32)
        want, counts = _oracle_uniform(cams, 2, dp, cp, 40, rays, kind=0, grid=grid, table=table)
        assert (counts == 40).mean() > 0.3
        _close_rgba(img.ravel(), want)
    finally:
        ctx.close()


def test_render_uniform_views_and_background(dataset):
    """nerf_ext_render_uniform directly: two views in one call, a coloured
    background, unclamped RGB within 1e-3 of the oracle."""
    cams, _, _ = dataset
    announce("nerf_ext_render_uniform: 2 views, reference model")
    m = ext.RefModel.create()
    dp, cp = m.density.numpy().view(np.uint16), m.color.numpy().view(np.uint16)
    views = [cams[0], cams[3]]
    bg = (0.2, 0.5, 0.9)
    r = ext.Renderer()
    from nerf_amd.device import DeviceArray, synchronize

    rgba = DeviceArray((2, H, W), np.uint32)
    rgb = DeviceArray((2, H, W, 3), np.float32)
    ms = m.struct()
    cam_arr = (L.NerfExtCamera * 2)(*views)
    box = (C.c_float * 6)(*BOX)
    bgc = (C.c_float * 3)(*bg)
    L.call("nerf_ext_render_uniform", r._h, C.byref(ms), cam_arr, 2, C.cast(box, C.c_void_p), 16, C.cast(bgc, C.c_void_p), rgba.ptr, rgb.ptr, None)
    synchronize()
    got_rgb = rgb.numpy()
    rays = np.arange(0, W * H, 5, dtype=np.uint32)
    for v, cam in enumerate(views):
        want_rgb, want_rgba, _ = orc.render_uniform(None, None, dp, cp, orc.camera_from_bytes(bytes(cam)), BOX, 16, rays, bg=bg, threads=8, kind=1)
        g = got_rgb[v].reshape(-1, 3)[rays]
        assert np.max(np.abs(g - want_rgb) / np.maximum(np.abs(want_rgb), 1e-3)) <= 1e-3
        _close_rgba(rgba.numpy()[v].ravel()[rays], want_rgba)


def test_failed_model_switch_leaves_the_context(dataset, tmp_path):
    """A switch that the new model cannot take (the reference model trains on
    at most 2^20 samples per step; this context trains the hash grid on
    8,192 x 256 = 2^21) fails as a whole: the model, its weights, the
    training run and the inference sampling stay as they were, whether the
    switch comes from nerf_ext_context_configure or from loading a reference
    checkpoint."""
    cams, imgs, mats = dataset
    announce("nerf.h context: failed model switch (2^21 samples per step) leaves the context unchanged")
    ref_ctx = Context(dataset)
    try:
        _configure(ref_ctx, L.NERF_EXT_MODEL_REFERENCE)
        ref_path = tmp_path / "ref.ckpt"
        ref_ctx.save(ref_path)
    finally:
        ref_ctx.close()
    ctx = Context.__new__(Context)
    ctx._keep = (imgs, mats)
    d = L.NerfCreateDesc(32, 1 << 22, 8192, 256, imgs.ctypes.data, imgs.nbytes, mats.ctypes.data, mats.nbytes, VIEWS, W, H, cams[0].fx, cams[0].fy, cams[0].cx, cams[0].cy)
    ctx.h = C.c_void_p()
    L.call("nerf_create_context", C.byref(d), C.byref(ctx.h))
    try:
        L.call("nerf_configure_training", ctx.h, C.byref(_config(rays=8192, steps=256)))
        for _ in range(2):
            L.call("nerf_train_step", ctx.h)
        before = tmp_path / "before.ckpt"
        ctx.save(before)
        img0, _ = ctx.infer(1, samples=64)
        assert ctx.status("nerf_ext_context_configure", C.byref(L.NerfExtContextOptions(L.NERF_EXT_MODEL_REFERENCE, L.NERF_EXT_SAMPLING_UNIFORM))) == L.NERF_STATUS_INVALID_USAGE
        assert "2^20" in L.last_error()
        assert _options(ctx) == (L.NERF_EXT_MODEL_HASHGRID, L.NERF_EXT_SAMPLING_DEFAULT)
        assert ctx.load(ref_path) == L.NERF_STATUS_INVALID_USAGE
        assert _options(ctx) == (L.NERF_EXT_MODEL_HASHGRID, L.NERF_EXT_SAMPLING_DEFAULT)
        after = tmp_path / "after.ckpt"
        ctx.save(after)
        assert open(after, "rb").read() == open(before, "rb").read(), "the weights changed"
        img1, _ = ctx.infer(1, samples=64)
        assert np.array_equal(img0, img1)
        # Training is still configured and continues from its step count.
        L.call("nerf_train_step", ctx.h)
        st = L.NerfTrainStats()
        L.call("nerf_read_train_stats", ctx.h, C.byref(st))
        assert st.completed_steps == 3 and st.has_nonfinite == 0
    finally:
        ctx.close()
